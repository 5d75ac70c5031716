"""llmq_linear_noalloc (no counterpart in the reference: llmq_linear for
callers that cannot allocate) through the C ABI against llmq_linear on the
same inputs: bit-identical outputs on two calls in a row, the second with
fewer tokens, for the prompt GEMM (which keeps its int16 activation codes
in the fixed scratch), the Q4_K matmul (its fp16 activation record there)
and the one-token GEMVs; calls captured into a HIP graph (where allocating
is an error) replay to llmq_linear's results; sizes past the scratch are
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


def q4k(lm, ctx, K, N, seed):
    from llm_mojo_amd import synth

    blocks = synth.gguf_blocks(12, N, K, seed, scale=1e-4)
    return lm.HipGGUFMatrix.from_blocks(ctx, 12, blocks, N, K)


@pytest.mark.parametrize("K,N,Ts", [(2048, 2560, (300, 37, 1)), (5632, 2048, (16, 3, 1))])
def test_noalloc_q4k_matches_linear(gpu, K, N, Ts):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(K + N)
    w = q4k(lm, ctx, K, N, 5)
    bias = torch.tensor(rng.normal(0, 0.1, N).astype(np.float32), device="cuda")
    for T in Ts:
        print(f"noalloc Q4_K {K}x{N} T={T}", flush=True)
        x = torch.tensor(rng.normal(0, 1, (T, K)).astype(np.float32), device="cuda")
        want = torch.zeros((T, N), dtype=torch.float32, device="cuda")
        got = torch.full((T, N), float("nan"), dtype=torch.float32, device="cuda")
        assert run(lm, "llmq_linear", ctx, want, x, w, bias, lm.LLMQ_BIAS) == 0, lm.lib().llmq_last_error()
        assert run(lm, "llmq_linear_noalloc", ctx, got, x, w, bias, lm.LLMQ_BIAS) == 0, lm.lib().llmq_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(want)), T
    w.free()


def test_noalloc_inside_graph_capture(gpu):
    """llmq_linear_noalloc called while a stream is being captured (capture
    mode thread_local: an allocation on this thread would end the capture
    with an error): an a16 prompt GEMM and a Q4_K matmul in one graph,
    replayed three times with new inputs copied in and other eager work
    between the replays; every replay equals llmq_linear run eagerly."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(3)
    K, N, T = 768, 2304, 37
    wa = lm.HipQuantMatrix.from_f32(ctx, rng.normal(0, 0.02, (K, N)).astype(np.float32), 4, 32)
    wq = q4k(lm, ctx, 2048, 2560, 6)
    xa = torch.zeros((T, K), dtype=torch.float32, device="cuda")
    xq = torch.zeros((20, 2048), dtype=torch.float32, device="cuda")
    oa = torch.zeros((T, N), dtype=torch.float32, device="cuda")
    oq = torch.zeros((20, 2560), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    print("noalloc graph: capture", flush=True)
    torch.cuda.synchronize()
    ctx.set_stream(s)
    try:
        with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
            assert run(lm, "llmq_linear_noalloc", ctx, oa, xa, wa, None, lm.LLMQ_GELU) == 0, lm.lib().llmq_last_error()
            assert run(lm, "llmq_linear_noalloc", ctx, oq, xq, wq, None, 0) == 0, lm.lib().llmq_last_error()
    finally:
        ctx.set_stream(torch.cuda.current_stream())
    for rep in range(3):
        print("noalloc graph: replay", rep, flush=True)
        xa.copy_(torch.tensor(rng.normal(0, 1, (T, K)).astype(np.float32)))
        xq.copy_(torch.tensor(rng.normal(0, 1, (20, 2048)).astype(np.float32)))
        oa.fill_(float("nan"))
        oq.fill_(float("nan"))
        wa_ = torch.zeros_like(oa)
        wq_ = torch.zeros_like(oq)
        assert run(lm, "llmq_linear", ctx, wa_, xa, wa, None, lm.LLMQ_GELU) == 0
        assert run(lm, "llmq_linear", ctx, wq_, xq, wq, None, 0) == 0
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(oa), bits(wa_)), rep
        assert np.array_equal(bits(oq), bits(wq_)), rep
    del g
    wa.free()
    wq.free()
