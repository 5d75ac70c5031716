"""GGUF block formats on the GPU against the oracle's restatement of
gguf.mojo: dequantized rows bit-exact (the decoders' float formulas are the
same operations), the float-activation decode GEMV within 1e-5 of max |out|
(the reference's own bar for its GGUF checks)."""
import numpy as np
import pytest

from tests import ggml_pack

pytestmark = pytest.mark.gpu

KINDS = ["Q4_0", "Q4_1", "Q8_0", "Q4_K", "Q5_K", "Q6_K"]


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("kind", KINDS)
def test_gguf_dequant_rows_exact(gpu, orc, kind):
    torch, lm, ctx = gpu
    t = orc.GGML[kind]
    rows, cols = 20, 512
    rng = np.random.default_rng(KINDS.index(kind))
    blocks, _ = ggml_pack.random_blocks(kind, rows * cols // orc.gguf_block_size(t), rng)
    print("gguf dequant", kind, flush=True)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, rows, cols)
    assert g.nbytes() == blocks.size
    want = orc.gguf_dequant(t, blocks, rows, cols)
    for r in (0, 7, rows - 1):
        assert np.array_equal(g.dequant_row(r), want[r])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows,cols", [(70, 512), (768, 2304), (1000, 4096), (6000, 4096), (300, 4352), (300, 11008)])
def test_gguf_gemv_vs_oracle(gpu, orc, kind, rows, cols):
    """(6000, 4096): 16-wave workgroups with runs of several row tiles, waves
    crossing tile boundaries; (300, 4352): 17 superblocks a row; (300, 11008):
    the longest rows (Q8_0: 16 code steps a wave)."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    t = orc.GGML[kind]
    blocks = synth.gguf_blocks(t, rows, cols, seed=rows + cols + t)
    rng = np.random.default_rng(t)
    x = rng.normal(0, 1, cols).astype(np.float32)
    b = rng.normal(0, 0.1, rows).astype(np.float32)
    print("gguf gemv", kind, rows, cols, flush=True)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, rows, cols)
    out = torch.zeros((1, rows), device="cuda")
    lm.linear(ctx, out, dev(torch, x.reshape(1, -1)), g, dev(torch, b))
    torch.cuda.synchronize()
    want = orc.gguf_gemv(t, blocks, rows, cols, x, b, orc.EPI_BIAS)
    got = out.cpu().numpy()[0]
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5


@pytest.mark.parametrize("kind", ["Q4_0", "Q4_1", "Q8_0"])
def test_gguf_gemv_partial_steps(gpu, orc, kind, monkeypatch):
    """cols = 544: 17 chunks of 32 (34 of Q8_0's 16) a row, so the last step
    of every tile is partial; 16-wave workgroups (forced) with runs of 4 row
    tiles, so waves cross tile boundaries mid-run."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    monkeypatch.setenv("LLMQ_GEMV1_NW", "16")
    t = orc.GGML[kind]
    rows, cols = 13000, 544
    blocks = synth.gguf_blocks(t, rows, cols, seed=t)
    rng = np.random.default_rng(t + 1)
    x = rng.normal(0, 1, cols).astype(np.float32)
    res = rng.normal(0, 0.1, rows).astype(np.float32)
    print("gguf gemv partial", kind, flush=True)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, rows, cols)
    out = dev(torch, res.reshape(1, -1))
    lm.linear(ctx, out, dev(torch, x.reshape(1, -1)), g, None, resid=True)
    torch.cuda.synchronize()
    want = orc.gguf_gemv(t, blocks, rows, cols, x, None, 0) + res
    got = out.cpu().numpy()[0]
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5


def test_gguf_unsupported_type(gpu):
    torch, lm, ctx = gpu
    with pytest.raises(lm.LlmqError, match="supported"):
        lm.HipGGUFMatrix.from_blocks(ctx, 1, np.zeros(64, np.uint8), 1, 32)


@pytest.mark.parametrize("kind", ["Q6_K", "Q8_0"])
@pytest.mark.parametrize("V,C,T,big", [(70, 512, 1, False), (300, 768, 5, False), (1000, 2048, 1, True),
                                       (4000, 4096, 2, False), (32000, 2048, 1, False), (300, 768, 20, False),
                                       (32000, 2048, 16, False), (32000, 2048, 16, True), (1000, 2048, 9, True),
                                       (600, 2048, 33, False)])
def test_gguf_int16_head_exact(gpu, orc, kind, V, C, T, big):
    """head_i16 (kernels.mojo:693-736) for Q6_K / Q8_0 heads: the logits equal
    the oracle's dot_row_i16 * sx bit for bit (same int32 lanes, same float
    chain over superblocks / blocks, same 16-lane sum).  (32000, 2048) is the
    TinyLlama Q6_K head; "big" alternates +-(0.9..1) so the int16 codes sit
    near +-32767 and Q6_K's lane sums near 2^31.  From 9 tokens a Q6_K head
    takes the fp16 matrix-core kernel (token tiles of 16, the last one
    partial at 9, 20 and 33 tokens)."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    t = orc.GGML[kind]
    blocks = synth.gguf_blocks(t, V, C, seed=V + C)
    rng = np.random.default_rng(V + T)
    if big:
        h = (rng.uniform(0.9, 1.0, (T, C)) * np.where(np.arange(T * C).reshape(T, C) % 2 == 0, 1, -1))
    else:
        h = rng.normal(0, 1, (T, C))
    h = h.astype(np.float32)
    print("gguf int16 head", kind, V, C, T, flush=True)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, V, C)
    assert g.has_i16()
    logits = torch.zeros((T, V), device="cuda")
    lm.head(ctx, logits, dev(torch, h), g)
    torch.cuda.synchronize()
    want = orc.gguf_head_i16(t, blocks, V, C, h)
    got = logits.cpu().numpy()
    assert np.array_equal(got, want), np.max(np.abs(got - want))


@pytest.mark.parametrize("V,C,T,big", [(32000, 2048, 16, True), (300, 768, 20, False)])
def test_gguf_int16_head_valu_form(gpu, orc, V, C, T, big, monkeypatch):
    """The Q6_K head's VALU kernel at 9-16 tokens a tile (LLMQ_HEAD16_MF=0;
    the default takes the matrix cores there): the same bits as the
    oracle's."""
    monkeypatch.setenv("LLMQ_HEAD16_MF", "0")
    test_gguf_int16_head_exact(gpu, orc, "Q6_K", V, C, T, big)


def test_gguf_float_heads_take_the_float_path(gpu, orc):
    """kernels.head: Q4_K has no int16 kernel, so its head is the float GEMV."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    t = orc.GGML["Q4_K"]
    V, C = 100, 512
    blocks = synth.gguf_blocks(t, V, C, seed=5)
    h = np.random.default_rng(5).normal(0, 1, (1, C)).astype(np.float32)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, V, C)
    assert not g.has_i16()
    logits = torch.zeros((1, V), device="cuda")
    lm.head(ctx, logits, dev(torch, h), g)
    torch.cuda.synchronize()
    want = orc.gguf_gemv(t, blocks, V, C, h[0], None, 0)
    got = logits.cpu().numpy()[0]
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("rows,cols,T", [(70, 512, 5), (300, 2048, 16), (200, 4352, 33), (256, 5632, 17),
                                         (100, 544, 20), (200, 2048, 130), (72, 4352, 70)])
def test_gguf_matmul_several_tokens(gpu, orc, kind, rows, cols, T):
    """matmul_rows for T > 1 (kernels.mojo:314-349): every token's outputs
    within 1e-5 of max |out| of the oracle's one-token GEMV (the same
    dequantized weights; float sums in another order).  (200, 4352): 17
    superblocks a row; (256, 5632): TinyLlama's FFN down projection shape;
    (100, 544): a reduction axis that ends mid-block (Q4_0 / Q4_1 / Q8_0 only);
    130 and 70 tokens: Q4_K's prompt form (records staged in LDS, 4 token
    tiles a workgroup, the last group part-filled)."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    t = orc.GGML[kind]
    if cols % orc.gguf_block_size(t):
        pytest.skip("cols not a whole number of blocks")
    blocks = synth.gguf_blocks(t, rows, cols, seed=rows + cols + T)
    rng = np.random.default_rng(T)
    x = rng.normal(0, 1, (T, cols)).astype(np.float32)
    b = rng.normal(0, 0.1, rows).astype(np.float32)
    res = rng.normal(0, 0.1, (T, rows)).astype(np.float32)
    print("gguf matmul", kind, rows, cols, T, flush=True)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, rows, cols)
    out = dev(torch, res)
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), resid=True)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = np.stack([orc.gguf_gemv(t, blocks, rows, cols, x[i], b, orc.EPI_BIAS) for i in range(T)]) + res
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5


@pytest.mark.parametrize("h16", ["1", "0"])
def test_gguf_q4k_matmul_activation_range(gpu, orc, monkeypatch, h16):
    """The several-token Q4_K matmul over activations of very different
    sizes: a zero token, tokens of scale 1e-30, 1e-6, 1 and 1e3, and one
    whose inputs alternate between 1e4 and 1e-4.  Each token's outputs within
    1e-5 of its own max |out| of the oracle's GEMV (exactly 0 for the zero
    token), on the fp16 matrix cores (per-sub-block power-of-two scales and
    two fp16 planes) and, with LLMQ_GEMM_H16=0, on the fp32 ones."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    monkeypatch.setenv("LLMQ_GEMM_H16", h16)
    t = orc.GGML["Q4_K"]
    rows, cols = 96, 768
    blocks = synth.gguf_blocks(t, rows, cols, seed=31)
    rng = np.random.default_rng(31)
    x = rng.normal(0, 1, (7, cols)).astype(np.float32)
    x[0] = 0.0
    for i, sc in ((1, 1e-30), (2, 1e-6), (3, 1.0), (4, 1e3)):
        x[i] *= sc
    x[5] = np.where(np.arange(cols) % 2 == 0, 1e4, 1e-4) * np.sign(x[5])
    x[6, 100:] = 0.0  # one token nonzero over the first 100 inputs only
    print("gguf q4k activation range", h16, flush=True)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, rows, cols)
    out = dev(torch, np.zeros((7, rows), np.float32))
    lm.linear(ctx, out, dev(torch, x), g)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i in range(7):
        want = orc.gguf_gemv(t, blocks, rows, cols, x[i], None, 0)
        m = np.max(np.abs(want))
        if m == 0:
            assert np.all(got[i] == 0), i
        else:
            assert np.max(np.abs(got[i] - want)) / m < 1e-5, (i, np.max(np.abs(got[i] - want)) / m)


def test_gguf_file_matrices_and_llama(gpu, tmp_path):
    """GGUFFile.matrix (gguf.mojo:622-633) gives the matrix the blocks give,
    and a config-4 decoder read from a GGUF file computes what the same
    tensors passed directly compute."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import llama, synth
    from tests import gguf_write as gw

    cfg = dict(n_layer=2, dim=256, n_head=4, n_kv=2, head_dim=64, ffn=512, vocab=1000, max_t=96, batch=1,
               layer_type=12, head_type=14, embd_type=12, eps=1e-5, theta=10000.0)
    tensors = synth.llama_tensors(cfg, 11)
    shapes = llama.tensor_shapes(cfg)
    entries = []
    for name, a in zip(llama.tensor_names(cfg["n_layer"]), tensors):
        kind = name.rsplit(".", 1)[-1]
        if kind.endswith("norm"):
            entries.append((name + ".weight", 0, [cfg["dim"]], gw.f32_bytes(a)))
        else:
            t = cfg["head_type"] if kind == "output" else (cfg["embd_type"] if kind == "token_embd" else 12)
            rows, cols = shapes[kind]
            entries.append((name + ".weight", t, [cols, rows], np.asarray(a, np.uint8).tobytes()))
    path = tmp_path / "tiny.gguf"
    gw.write(path, entries, [("general.architecture", gw.STRING, "llama")])
    print("gguf file matrix", flush=True)
    g = lm.GGUFFile(path)
    m1 = g.matrix(ctx, "blk.1.ffn_down.weight")
    m2 = lm.HipGGUFMatrix.from_blocks(ctx, 12, tensors[1 + 9 + 8], 256, 512)
    x = torch.from_numpy(np.random.default_rng(1).normal(0, 1, (1, 512)).astype(np.float32)).cuda()
    a = torch.zeros((1, 256), device="cuda")
    b = torch.zeros((1, 256), device="cuda")
    lm.linear(ctx, a, x, m1)
    lm.linear(ctx, b, x, m2)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    g.close()
    print("gguf file llama", flush=True)
    toks = synth.llama_prompts(11, 1, 9, cfg["vocab"])[0]
    f = lm.Llama.from_gguf(ctx, path, cfg)
    d = lm.Llama(ctx, cfg, tensors)
    assert np.array_equal(f.forward(0, toks, 0), d.forward(0, toks, 0))
    f.free()
    d.free()


CONFIG2_KINDS = ["Q4_0", "Q4_K", "Q5_K", "Q6_K", "Q8_0"]


@pytest.mark.parametrize("kind", CONFIG2_KINDS)
@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)])
def test_gguf_gemv_config2_shapes(gpu, orc, kind, K, N):
    """Config 2's own shapes (K x N, batch 1, float activations): every
    matrix of 20 MB or more takes the streamed form (two code steps in
    flight a wave), the K-quants included; 1e-5 of max |out| against the
    oracle's gguf_gemv, and deterministic from run to run."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    t = orc.GGML[kind]
    blocks = synth.gguf_blocks(t, N, K, seed=7 + t)
    rng = np.random.default_rng(K + N + t)
    x = rng.normal(0, 1, K).astype(np.float32)
    print("config 2 gemv", kind, K, N, flush=True)
    g = lm.HipGGUFMatrix.from_blocks(ctx, t, blocks, N, K)
    out = torch.zeros((1, N), device="cuda")
    out2 = torch.zeros((1, N), device="cuda")
    xd = dev(torch, x.reshape(1, -1))
    lm.linear(ctx, out, xd, g)
    lm.linear(ctx, out2, xd, g)
    torch.cuda.synchronize()
    orc.set_threads(16)
    want = orc.gguf_gemv(t, blocks, N, K, x, None, 0)
    got = out.cpu().numpy()[0]
    assert np.array_equal(got, out2.cpu().numpy()[0])
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5
    g.free()
