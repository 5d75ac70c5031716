"""CPU checks of the C ABI: libllmq.so loads here (no GPU needed to load it)
and exports every function include/llmq.h declares; the Python binding
declares exactly those functions."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "llmq.h")).read()
    return set(re.findall(r"LLMQ_API\s+[\w\s\*]+?\b(llmq_\w+)\s*\(", src))


def test_header_declares_the_api():
    names = declared()
    for n in ("llmq_init", "llmq_mat_from_f32", "llmq_linear", "llmq_head", "llmq_kv_attend", "llmq_gpt2_generate"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from llm_mojo_amd import _lib

    assert os.path.exists(_lib.LIB_PATH), "libllmq.so not built (python -m llm_mojo_amd.build)"
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(declared()) if not hasattr(L, n)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == declared()


def test_binding_raises_without_library(monkeypatch, tmp_path):
    from llm_mojo_amd import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    import pytest

    with pytest.raises(_lib.LlmqError):
        _lib.lib()
