import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """(torch, llm_mojo_amd, Context) on cuda:0, ordered on torch's stream.
    Fails (does not skip) when the GPU or libllmq.so is missing."""
    import torch

    import llm_mojo_amd as lm

    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    lm.lib()  # raises if libllmq.so is not built
    ctx = lm.Context(0)
    ctx.set_stream(torch.cuda.current_stream())
    yield torch, lm, ctx
    torch.cuda.synchronize()
