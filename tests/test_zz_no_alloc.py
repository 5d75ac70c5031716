"""llmq_linear_noalloc (no counterpart in the reference: llmq_linear for
callers that cannot allocate) through the C ABI against llmq_linear on the
same inputs: bit-identical outputs on two calls in a row, the second with
fewer tokens, for the prompt GEMM (which keeps its int16 activation codes
in the fixed scratch) and the one-token GEMV; sizes past the scratch are
refused before anything runs."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def run(lm, name, ctx, out, x, w, bias, flags):
    T, IN = x.shape
    f = getattr(lm.lib(), name)
    return f(ctx.h, out.data_ptr(), x.data_ptr(), w.h, bias.data_ptr() if bias is not None else None, T, IN, w.rows,
             flags)


def bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("bits_,group,K,N,Ts", [(4, 32, 768, 2304, (300, 37, 1)), (8, 0, 3072, 768, (64, 5, 1))])
def test_noalloc_matches_linear(gpu, bits_, group, K, N, Ts):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(11 + bits_)
    wt = rng.normal(0, 0.02, (K, N)).astype(np.float32)  # [IN, OUT], reduced over rows
    w = lm.HipQuantMatrix.from_f32(ctx, wt, bits_, group)
    bias = torch.tensor(rng.normal(0, 0.1, N).astype(np.float32), device="cuda")
    flags = lm.LLMQ_BIAS | lm.LLMQ_GELU
    for T in Ts:
        print(f"noalloc int{bits_} g{group} {K}x{N} T={T}", flush=True)
        x = torch.tensor(rng.normal(0, 1, (T, K)).astype(np.float32), device="cuda")
        want = torch.zeros((T, N), dtype=torch.float32, device="cuda")
        got = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
        assert run(lm, "llmq_linear", ctx, want, x, w, bias, flags) == 0, lm.lib().llmq_last_error()
        assert run(lm, "llmq_linear_noalloc", ctx, got, x, w, bias, flags) == 0, lm.lib().llmq_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want)), T
        assert np.isfinite(got.cpu().numpy()).all()


def test_noalloc_refuses_sizes_past_its_scratch(gpu):
    torch, lm, ctx = gpu
    K, N, T = 768, 256, 6000  # 6000 x 768 x 2 bytes > 8 MiB
    w = lm.HipQuantMatrix.from_f32(ctx, np.zeros((K, N), np.float32), 8, 0)
    x = torch.zeros((T, K), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, N), dtype=torch.float32, device="cuda")
    rc = run(lm, "llmq_linear_noalloc", ctx, out, x, w, None, 0)
    assert rc == -1 and b"maximum is 8388608" in lm.lib().llmq_last_error()
    assert run(lm, "llmq_linear", ctx, out, x, w, None, 0) == 0  # llmq_linear grows its workspace instead
    torch.cuda.synchronize()
