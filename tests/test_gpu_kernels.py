"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI.

Bars: quantized codes, activation codes and the
per-group integer sums bit-exact; float32 outputs within 1e-5 of max |out|
(the reference's own A16 tolerance, tests/a16_kernels.mojo:70).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REL = 1e-5


def note(*a):
    print(*a, flush=True)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30)


FORMATS = [  # (bits, group, sym)
    (4, 32, False), (4, 32, True), (4, 64, False), (4, 128, True), (4, 0, False), (8, 32, False), (8, 64, False),
    (8, 128, False), (8, 0, False), (8, 0, True),
]


@pytest.mark.parametrize("bits,group,sym", FORMATS)
def test_weight_codes_bit_exact(gpu, orc, bits, group, sym):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(bits * 97 + group + sym)
    IN, OUT = 768, 70  # 70: a partial last row tile
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    w[:, 3] = 0.0
    note("codes", bits, group, sym)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, True)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    codes, scales, zps = g.export()
    assert np.array_equal(codes, o.data)
    assert np.array_equal(scales, o.scale)
    assert np.array_equal(zps, o.zp)
    assert g.nbytes() == o.nbytes()
    assert np.array_equal(g.dequant_row(5), o.dequant()[5])


def test_head_codes_transposed_axis(gpu, orc):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(5)
    V, C = 1000, 768
    wte = rng.normal(0, 0.02, (V, C)).astype(np.float32)
    note("head codes")
    g = lm.HipQuantMatrix.from_f32(ctx, wte, 8, 0, False, True, reduce_rows=False)
    o = orc.QuantMatrix.from_f32(wte, 8, 0, False, True, reduce_rows=False)
    codes, scales, zps = g.export()
    assert np.array_equal(codes, o.data) and np.array_equal(scales, o.scale) and np.array_equal(zps, o.zp)


def test_quantize_rows_bit_exact(gpu, orc):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (6, 3072)).astype(np.float32)
    x[2] = 0.0
    x[4, 7] = 0.5 * np.abs(x[4]).max()  # include ties-ish magnitudes
    note("quantize_rows")
    xd = dev(torch, x)
    xq = torch.zeros((6, 3072), dtype=torch.int16, device="cuda")
    sx = torch.zeros(6, dtype=torch.float32, device="cuda")
    lm.quantize_rows(ctx, xd, xq, sx)
    torch.cuda.synchronize()
    want_q, want_s = orc.quantize_rows(x)
    assert np.array_equal(xq.cpu().numpy(), want_q)
    assert np.array_equal(sx.cpu().numpy(), want_s)


@pytest.mark.parametrize("bits,group,sym", FORMATS)
@pytest.mark.parametrize("IN,OUT,nw", [(768, 2304, None), (3072, 768, None), (768, 70, None), (4096, 6000, None),
                                       (544, 13000, "16")])
def test_group_sums_exact(gpu, orc, bits, group, sym, IN, OUT, nw, monkeypatch):
    """Per-chunk integer partials of the product kernel, summed per group,
    equal the exact int64 group sums; the kernel's activation codes and
    scale equal quantize_rows'.  (4096, 6000): 16-wave workgroups with runs
    of two row tiles; (544, 13000) with 16 waves forced: a partial last step
    in every tile (17 int4 chunks a row) and waves crossing tile boundaries."""
    torch, lm, ctx = gpu
    if IN % (group or IN):
        pytest.skip("group does not divide the row")
    if bits == 4 and group == 32 and IN % 256:
        pytest.skip("int4-g32-a16 (BLOCKED) needs whole 256-weight blocks")
    if nw:
        monkeypatch.setenv("LLMQ_GEMV1_NW", nw)
    rng = np.random.default_rng(IN + OUT + bits + group)
    w = rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (1, IN)).astype(np.float32)
    note("group sums", bits, group, sym, IN, OUT)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, True)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    wpc = 32 if bits == 4 else 16
    CK = IN // wpc
    cs = torch.zeros((OUT, CK), dtype=torch.int32, device="cuda")
    xq = torch.zeros(IN, dtype=torch.int16, device="cuda")
    sx = torch.zeros(1, dtype=torch.float32, device="cuda")
    out = torch.zeros((1, OUT), dtype=torch.float32, device="cuda")
    lm.debug_chunk_sums(ctx, dev(torch, x), g, out, cs, xq, sx)
    torch.cuda.synchronize()
    want_q, want_s = orc.quantize_rows(x)
    assert np.array_equal(xq.cpu().numpy(), want_q[0])
    assert sx.cpu().numpy()[0] == want_s[0]
    gs = cs.cpu().numpy().astype(np.int64).reshape(OUT, IN // o.group, o.group // wpc).sum(-1)
    assert np.array_equal(gs, o.group_sums(want_q[0]))
    want = orc.matmul_rows_a16(x, o, None, 0)
    assert rel_err(out.cpu().numpy(), want) < REL


A16_CASES = [  # tests/a16_kernels.mojo:85-94 and the GPT-2 / Llama layer shapes
    *[((4, 32, False), T, 768, 64, False) for T in (1, 3, 4, 9)],
    *[((4, 32, False), T, 768, 70, False) for T in (1, 3, 4, 9)],
    *[((4, 32, True), T, 3072, 64, False) for T in (1, 5)],
    *[((4, 32, False), T, 3072, 40, True) for T in (1, 5)],
    *[((8, 0, False), T, 768, 64, False) for T in (1, 6)],
    *[((8, 0, False), T, 3072, 64, True) for T in (1, 6)],
    *[((4, 0, True), T, 3072, 40, True) for T in (1, 6)],
    ((4, 32, False), 1, 768, 2304, False), ((4, 32, False), 1, 768, 3072, False),
    ((4, 32, False), 1, 3072, 768, False), ((8, 32, False), 1, 768, 2304, False),
    ((4, 64, False), 1, 768, 768, False), ((4, 128, False), 1, 3072, 768, False),
    ((4, 32, False), 12, 768, 2304, False), ((4, 32, False), 17, 3072, 768, False),
    ((8, 32, False), 12, 768, 3072, False), ((4, 32, False), 1, 4096, 11008, False),
    ((4, 32, False), 1, 11008, 4096, False), ((4, 32, False), 5, 4096, 1024, False),
    ((8, 0, False), 1, 768, 50257, False),
    # prompt GEMMs on the int8 matrix cores (T >= 8): every format, partial
    # token and row tiles, +-32767 activations, the 476-token prompt
    ((4, 32, False), 64, 768, 2304, False), ((4, 32, False), 476, 768, 3072, False),
    ((8, 32, False), 476, 3072, 768, False), ((4, 64, False), 33, 768, 768, False),
    ((4, 128, True), 40, 3072, 768, False), ((8, 0, False), 20, 768, 64, True),
    ((8, 0, True), 24, 3072, 64, True), ((4, 0, True), 16, 3072, 40, True),
    ((8, 128, False), 70, 768, 130, True), ((4, 32, True), 100, 768, 70, True),
    # staged blocks of 64 and 128 inputs (reduction axes of 9 and 10 x 64)
    ((4, 64, False), 40, 576, 100, False), ((8, 32, False), 20, 640, 64, True),
]


@pytest.mark.parametrize("fmt,T,IN,OUT,big", A16_CASES)
def test_linear_vs_oracle(gpu, orc, fmt, T, IN, OUT, big):
    torch, lm, ctx = gpu
    bits, group, sym = fmt
    rng = np.random.default_rng(T * 131 + IN + OUT)
    w = rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32)
    if big:
        x = (rng.uniform(0.9, 1.0, (T, IN)) * np.where(np.arange(T * IN).reshape(T, IN) % 2 == 0, 1, -1)).astype(np.float32)
    else:
        x = rng.uniform(-1, 1, (T, IN)).astype(np.float32)
    b = rng.uniform(-1, 1, OUT).astype(np.float32)
    note("linear", fmt, T, IN, OUT, big)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, True)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b))
    torch.cuda.synchronize()
    want = orc.matmul_rows_a16(x, o, b)
    assert rel_err(out.cpu().numpy(), want) < REL


@pytest.mark.parametrize("fmt", [(4, 32, False), (4, 128, True), (8, 0, False), (4, 0, False)])
@pytest.mark.parametrize("IN,OUT", [(3072, 768), (4096, 200)])
def test_linear_four_wave_long_rows(gpu, orc, fmt, IN, OUT, monkeypatch):
    """4-wave workgroups forced on long rows: one row tile per workgroup,
    up to 8 steps a wave and up to 4 activation units a thread."""
    torch, lm, ctx = gpu
    bits, group, sym = fmt
    monkeypatch.setenv("LLMQ_GEMV1_NW", "4")
    monkeypatch.setenv("LLMQ_EXACT", "0")  # gemv1 itself (the exact kernels take BLOCKED and int8-ch)
    rng = np.random.default_rng(IN + OUT + bits + group)
    w = rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32)
    x = rng.uniform(-1, 1, (1, IN)).astype(np.float32)
    b = rng.uniform(-1, 1, OUT).astype(np.float32)
    note("four-wave linear", fmt, IN, OUT)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, True)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    out = torch.zeros((1, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), resid=True)
    torch.cuda.synchronize()
    want = orc.matmul_rows_a16(x, o, b, orc.EPI_BIAS | orc.EPI_RESID, out=np.zeros((1, OUT), np.float32))
    assert rel_err(out.cpu().numpy(), want) < REL
    g.free()


@pytest.mark.parametrize("bits", [4, 8])
def test_prompt_gemm_matches_tile_order(gpu, orc, bits):
    """The matrix-core GEMM forms each group's exact int32 sum and folds it
    into the float accumulator in tile_i16's order (kernels.mojo:512-573):
    outputs equal the oracle's multi-token path to the last bit."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(bits)
    T, IN, OUT = 37, 768, 192
    w = rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (T, IN)).astype(np.float32)
    b = rng.uniform(-1, 1, OUT).astype(np.float32)
    note("prompt gemm order", bits)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, 32, False, True)
    o = orc.QuantMatrix.from_f32(w, bits, 32, False, True)
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b))
    torch.cuda.synchronize()
    want = orc.matmul_rows_a16(x, o, b)
    got = out.cpu().numpy()
    print("max |diff|", float(np.max(np.abs(got - want))), flush=True)
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("T", [1, 5])
def test_linear_epilogues(gpu, orc, T):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(40 + T)
    IN, OUT = 768, 3072
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (T, IN)).astype(np.float32)
    b = rng.normal(0, 0.1, OUT).astype(np.float32)
    base = rng.normal(0, 1, (T, OUT)).astype(np.float32)
    g = lm.HipQuantMatrix.from_f32(ctx, w, 4, 32, False, True)
    o = orc.QuantMatrix.from_f32(w, 4, 32, False, True)
    note("epilogue gelu", T)
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), gelu=True)
    torch.cuda.synchronize()
    assert rel_err(out.cpu().numpy(), orc.matmul_rows_a16(x, o, b, orc.EPI_BIAS | orc.EPI_GELU)) < REL
    note("epilogue resid", T)
    out = dev(torch, base)
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), resid=True)
    torch.cuda.synchronize()
    want = orc.matmul_rows_a16(x, o, b, orc.EPI_BIAS | orc.EPI_RESID, out=base.copy())
    assert rel_err(out.cpu().numpy(), want) < REL


@pytest.mark.parametrize("T", [1, 4])
def test_ln_linear(gpu, orc, T):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(60 + T)
    IN, OUT = 768, 2304
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    x = rng.normal(0.1, 0.5, (T, IN)).astype(np.float32)
    lw = rng.normal(1, 0.1, IN).astype(np.float32)
    lb = rng.normal(0, 0.1, IN).astype(np.float32)
    b = rng.normal(0, 0.1, OUT).astype(np.float32)
    g = lm.HipQuantMatrix.from_f32(ctx, w, 4, 32, False, True)
    o = orc.QuantMatrix.from_f32(w, 4, 32, False, True)
    note("ln_linear", T)
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), ln=(dev(torch, lw), dev(torch, lb)))
    ln_out = torch.zeros((T, IN), dtype=torch.float32, device="cuda")
    lm.layernorm(ctx, ln_out, dev(torch, x), dev(torch, lw), dev(torch, lb))
    torch.cuda.synchronize()
    xn = orc.layernorm(x, lw, lb)
    assert np.max(np.abs(ln_out.cpu().numpy() - xn)) < 1e-5
    assert rel_err(out.cpu().numpy(), orc.matmul_rows_a16(xn, o, b)) < REL


def test_head_int8_channel(gpu, orc):
    """The GPT-2 output head shape (50257 x 768, HEAD8_A16)."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(77)
    V, C = 50257, 768
    wte = rng.normal(0, 0.02, (V, C)).astype(np.float32)
    h = rng.normal(0, 1, (1, C)).astype(np.float32)
    note("head 50257x768")
    g = lm.HipQuantMatrix.from_f32(ctx, wte, 8, 0, False, True, reduce_rows=False)
    o = orc.QuantMatrix.from_f32(wte, 8, 0, False, True, reduce_rows=False)
    logits = torch.zeros((1, V), dtype=torch.float32, device="cuda")
    lm.head(ctx, logits, dev(torch, h), g)
    torch.cuda.synchronize()
    want = orc.matmul_rows_a16(h, o, None, 0)
    got = logits.cpu().numpy()
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("T,pos0,MT", [(7, 20, 64), (1, 20, 64), (100, 5, 128), (476, 0, 512), (40, 900, 1024)])
def test_kv_store_and_attend(gpu, orc, T, pos0, MT):
    """Prompt attention (query blocks of 16, scores up to the block's last
    position) and the one-token path, against attend_float_one over the same
    int8 cache: partial query blocks, long prompts, late positions."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(9 + T)
    NL, NH, HS = 2, 12, 64
    C = NH * HS
    layer = 1
    qkv_all = rng.normal(0, 1, (pos0 + T, 3 * C)).astype(np.float32)
    qkv_all[3, C:C + HS] = 0.0
    note("kv store/attend", T, pos0, MT)
    kv = lm.QuantKV8(ctx, NL, MT, NH, HS)
    okv = orc.QuantKV8(NL, MT, NH, HS)
    if pos0:
        kv.store(layer, 0, dev(torch, qkv_all[:pos0]))
    q1 = dev(torch, qkv_all[pos0:])
    kv.store(layer, pos0, q1)
    out = torch.zeros((T, C), dtype=torch.float32, device="cuda")
    kv.attend(out, q1, layer, pos0)
    torch.cuda.synchronize()
    for p in range(pos0 + T):
        okv.store(layer, p, qkv_all[p, C:2 * C], qkv_all[p, 2 * C:])
    k, v, ks, vs = kv.export()
    assert np.array_equal(k, okv.k) and np.array_equal(v, okv.v)
    assert np.array_equal(ks, okv.ks) and np.array_equal(vs, okv.vs)
    want = okv.attend(qkv_all[pos0:], layer, T, pos0)
    assert rel_err(out.cpu().numpy(), want) < REL


def test_errors_are_reported(gpu):
    torch, lm, ctx = gpu
    w = np.zeros((100, 8), np.float32)  # 100 is not a multiple of the group
    with pytest.raises(lm.LlmqError, match="group size"):
        lm.HipQuantMatrix.from_f32(ctx, w, 4, 32, False, True)
    with pytest.raises(lm.LlmqError, match="256-weight blocks"):  # BLOCKED needs whole blocks
        lm.HipQuantMatrix.from_f32(ctx, np.zeros((544, 8), np.float32), 4, 32, False, True)
    g = lm.HipQuantMatrix.from_f32(ctx, np.zeros((256, 8), np.float32), 4, 32, False, True)
    out = torch.zeros((1, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(lm.LlmqError, match="IN="):
        lm.linear(ctx, out, torch.zeros((1, 32), device="cuda"), g)


def test_arrays_past_2gib_are_refused(gpu):
    """Kernels address each matrix array with 32-bit buffer offsets, so a
    matrix whose code array would reach 2 GiB is refused at creation, before
    its source is read (the sources here are deliberately tiny)."""
    import ctypes

    torch, lm, ctx = gpu
    src = torch.zeros(64, dtype=torch.float32, device="cuda")
    h = ctypes.c_void_p()
    # int8, 65536 x 65536: 4 GiB of codes
    rc = lm.lib().llmq_mat_from_f32_device(ctx.h, 8, 0, 0, 1, ctypes.c_void_p(src.data_ptr()), 65536, 65536, 0,
                                           ctypes.byref(h))
    assert rc != 0 and not h.value
    assert b"2 GiB" in lm.lib().llmq_last_error()
    with pytest.raises(lm.LlmqError, match="2 GiB"):  # Q8_0 131072 x 32768: 4 GiB of codes
        lm.HipGGUFMatrix.from_blocks(ctx, 8, np.zeros(34, np.uint8), 131072, 32768)
    ok = lm.HipQuantMatrix.from_f32(ctx, torch.zeros((64, 256), dtype=torch.float32, device="cuda"), 8, 0)
    assert ok.nbytes() > 0
