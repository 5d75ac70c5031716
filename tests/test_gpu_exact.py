"""Bit-exact parity of config 0's float path on the GPU: every kernel that
feeds an int16 activation code, a cache entry or a logit computes the
oracle's float32 bits exactly (outputs compared with array_equal, not with
a tolerance).  That is what lets the end-to-end decode
(tests/test_gpu_gpt2.py) agree token for token: a one-ulp difference
before quantize_rows can flip an int16 code, and a flipped code moves the
logits by ~1e-3 of their range.

Covered: the float path's exp / tanh / GELU; LayerNorm (16 lane partials and
the halving tree of kernels.mojo:179-197); the one-token BLOCKED int4-g32
GEMV (tensor.mojo:522-540) with and without LayerNorm, GELU and residual;
the int8 per-channel head (tensor.mojo:541-566) with LN_f; several-token
GEMMs in tile_i16's order (kernels.mojo:512-573); float attention over the
int8 cache (attend_float_one, kvcache.mojo:113-150) for decode and prompts.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def note(*a):
    print(*a, flush=True)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def same_bits(got, want):
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    assert got.shape == want.shape
    diff = got.view(np.uint32) != want.view(np.uint32)
    if diff.any():
        i = np.flatnonzero(diff.reshape(-1))[0]
        raise AssertionError(f"{int(diff.sum())} of {diff.size} values differ, first at {i}: "
                             f"{got.reshape(-1)[i]!r} vs {want.reshape(-1)[i]!r}")


def test_refmath_bit_exact(gpu, orc):
    torch, lm, ctx = gpu
    x = np.concatenate([np.linspace(-100, 100, 2_000_001), np.linspace(-1, 1, 200_001),
                        np.float32([0.0, -0.0, 1e-30, -1e-30, 0.625, -0.625, 10.0, -10.0, 88.5, -87.0, 1e30,
                                    -1e30, np.inf, -np.inf])]).astype(np.float32)
    xd = dev(torch, x)
    yd = torch.empty_like(xd)
    for op, ref in (("exp", orc.ref_exp), ("tanh", orc.ref_tanh), ("gelu", orc.gelu)):
        note("refmath", op)
        lm.debug_refmath(ctx, op, xd, yd)
        torch.cuda.synchronize()
        same_bits(yd.cpu().numpy(), ref(x))


def test_layernorm_bit_exact(gpu, orc):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(5)
    for T, C, scale in ((1, 768, 1.0), (12, 768, 30.0), (3, 2048, 0.01)):
        note("layernorm", T, C)
        x = (rng.normal(0, scale, (T, C)) + rng.normal(0, 3, (T, 1))).astype(np.float32)
        w = rng.normal(1, 0.1, C).astype(np.float32)
        b = rng.normal(0, 0.1, C).astype(np.float32)
        out = torch.zeros((T, C), dtype=torch.float32, device="cuda")
        lm.layernorm(ctx, out, dev(torch, x), dev(torch, w), dev(torch, b))
        torch.cuda.synchronize()
        same_bits(out.cpu().numpy(), orc.layernorm(x, w, b))


GEMV_SHAPES = [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 70), (4096, 4096), (4096, 11008)]


@pytest.mark.parametrize("IN,OUT", GEMV_SHAPES)
@pytest.mark.parametrize("mode", ["plain", "ln", "gelu", "resid", "sym"])
def test_blocked_gemv_bit_exact(gpu, orc, IN, OUT, mode):
    """One token through the BLOCKED int4-g32-a16 GEMV: exactly the
    reference's dot_row_i16 * sx (+ bias, GELU, residual)."""
    torch, lm, ctx = gpu
    if mode == "ln" and IN != 768:
        pytest.skip("LayerNorm precedes the 768-input matrices only")
    rng = np.random.default_rng(IN * 7 + OUT)
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (1, IN)).astype(np.float32)
    b = rng.normal(0, 0.1, OUT).astype(np.float32)
    r0 = rng.normal(0, 1, (1, OUT)).astype(np.float32)
    sym = mode == "sym"
    note("blocked gemv", IN, OUT, mode)
    g = lm.HipQuantMatrix.from_f32(ctx, w, 4, 32, sym, True)
    o = orc.QuantMatrix.from_f32(w, 4, 32, sym, True)
    out = dev(torch, r0)
    if mode == "ln":
        lw = rng.normal(1, 0.1, IN).astype(np.float32)
        lb = rng.normal(0, 0.1, IN).astype(np.float32)
        lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), ln=(dev(torch, lw), dev(torch, lb)))
        want = orc.matmul_rows_a16(orc.layernorm(x, lw, lb), o, b)
    else:
        flags = orc.EPI_BIAS | (orc.EPI_GELU if mode == "gelu" else 0) | (orc.EPI_RESID if mode == "resid" else 0)
        lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), gelu=mode == "gelu", resid=mode == "resid")
        want = orc.matmul_rows_a16(x, o, b, flags, out=r0.copy())
    torch.cuda.synchronize()
    same_bits(out.cpu().numpy(), want)
    g.free()


@pytest.mark.parametrize("V,C,ln", [(50257, 768, True), (50257, 768, False), (1000, 2048, False), (64, 4096, False)])
def test_int8_channel_head_bit_exact(gpu, orc, V, C, ln):
    """The int8 per-channel A16 head (HEAD8_A16): logits = dot_row_i16 * sx,
    with LN_f fused as in the decode step."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(V + C)
    wte = rng.normal(0, 0.02, (V, C)).astype(np.float32)
    h = rng.normal(0, 1, (1, C)).astype(np.float32)
    note("int8-ch head", V, C, ln)
    g = lm.HipQuantMatrix.from_f32(ctx, wte, 8, 0, False, True, reduce_rows=False)
    o = orc.QuantMatrix.from_f32(wte, 8, 0, False, True, reduce_rows=False)
    out = torch.zeros((1, V), dtype=torch.float32, device="cuda")
    if ln:
        lw = rng.normal(1, 0.1, C).astype(np.float32)
        lb = rng.normal(0, 0.1, C).astype(np.float32)
        lm.linear(ctx, out, dev(torch, h), g, None, ln=(dev(torch, lw), dev(torch, lb)))
        want = orc.matmul_rows_a16(orc.layernorm(h, lw, lb), o, None, 0)
    else:
        lm.linear(ctx, out, dev(torch, h), g, None)
        want = orc.matmul_rows_a16(h, o, None, 0)
    torch.cuda.synchronize()
    same_bits(out.cpu().numpy(), want)
    g.free()


@pytest.mark.parametrize("fmt", [(4, 32, False), (8, 32, False), (8, 0, False)])
@pytest.mark.parametrize("T", [2, 3, 5, 7, 12, 33])
def test_prompt_gemm_bit_exact(gpu, orc, fmt, T):
    """Several tokens (prompts) in tile_i16's order, GPT-2 layer shapes, and
    row counts that leave n % 32 rows to rows_i16's order (kernels.mojo:
    576-614): 70 and 50 rows, and 17 (fewer than one tile)."""
    torch, lm, ctx = gpu
    bits, group, sym = fmt
    rng = np.random.default_rng(T * 3 + bits)
    for IN, OUT, flags in ((768, 2304, 0), (3072, 768, 1), (768, 3072, 2), (768, 70, 2), (3072, 50, 1), (768, 17, 0)):
        w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
        x = rng.normal(0, 1, (T, IN)).astype(np.float32)
        b = rng.normal(0, 0.1, OUT).astype(np.float32)
        r0 = rng.normal(0, 1, (T, OUT)).astype(np.float32)
        note("prompt gemm", fmt, T, IN, OUT, flags)
        g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, True)
        o = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
        out = dev(torch, r0)
        lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), resid=flags == 1, gelu=flags == 2)
        ef = orc.EPI_BIAS | (orc.EPI_RESID if flags == 1 else 0) | (orc.EPI_GELU if flags == 2 else 0)
        want = orc.matmul_rows_a16(x, o, b, ef, out=r0.copy())
        torch.cuda.synchronize()
        same_bits(out.cpu().numpy(), want)
        g.free()


# Instantiations of the group-32 fp16 matrix-core GEMM: token tiles, row
# tiles a wave, groups a step, waves a workgroup.
F16_TILES = ["1,1,4", "1,1,2", "1,1,1", "2,1,4", "1,2,4", "1,1,8", "1,1,4,8", "2,1,4,8", "1,1,8,8"]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("tile", F16_TILES)
def test_prompt_gemm_f16_tiles(gpu, orc, tile, bits, monkeypatch):
    """Every instantiation of the int4-g32 and int8-g32 prompt GEMM on the
    fp16 matrix cores (LLMQ_F16_TILE) in tile_i16's order, with ragged token
    counts (a partial token tile, a partial workgroup of row tiles) and 16
    rows left to rows_i16."""
    torch, lm, ctx = gpu
    monkeypatch.setenv("LLMQ_F16_TILE", tile)
    rng = np.random.default_rng(sum(map(int, tile.split(","))) + bits)
    for T, IN, OUT, flags in ((37, 768, 2304, 2), (19, 3072, 816, 1), (2, 256, 48, 0)):
        w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
        x = rng.normal(0, 1, (T, IN)).astype(np.float32)
        b = rng.normal(0, 0.1, OUT).astype(np.float32)
        r0 = rng.normal(0, 1, (T, OUT)).astype(np.float32)
        note("prompt gemm f16", bits, tile, T, IN, OUT, flags)
        g = lm.HipQuantMatrix.from_f32(ctx, w, bits, 32, False, True)
        o = orc.QuantMatrix.from_f32(w, bits, 32, False, True)
        out = dev(torch, r0)
        lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), resid=flags == 1, gelu=flags == 2)
        ef = orc.EPI_BIAS | (orc.EPI_RESID if flags == 1 else 0) | (orc.EPI_GELU if flags == 2 else 0)
        want = orc.matmul_rows_a16(x, o, b, ef, out=r0.copy())
        torch.cuda.synchronize()
        same_bits(out.cpu().numpy(), want)
        g.free()


@pytest.mark.parametrize("bits", [4, 8])
def test_prompt_gemm_f16_extremes(gpu, orc, bits):
    """The fp16 form at the largest sums it has to hold: every |x| equal
    (codes +-32767: planes 256 * 127 + 255 and 256 * -128 + 1) against
    groups whose weights are 31 of +a (or -a) and one 0, which quantize to
    u - zp = +-15 (int4: |G| = 31 * 15 * 32767, ~15.2 M, of the 2^24 one
    exact fp32 chain holds) or +-255 (int8: |G| ~259 M, so the hi and lo
    sums, each exact, meet in one rounded add that must equal the
    reference's float(G)); also the sign mixes in between."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(77 + bits)
    IN, OUT, T = 768, 256 + 17, 20
    sign = np.where(rng.random(OUT) < 0.5, -1.0, 1.0)
    w = np.tile(0.03 * sign, (IN, 1)).astype(np.float32)
    w[::32, :] = 0.0
    w[:, -40:] *= np.where(rng.random((IN, 40)) < 0.5, -1.0, 1.0)  # mixed groups
    x = np.where(rng.random((T, IN)) < 0.5, -1.0, 1.0).astype(np.float32)
    x[0] = 1.0
    x[1] = -1.0
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, 32, False, True)
    o = orc.QuantMatrix.from_f32(w, bits, 32, False, True)
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, None)
    want = orc.matmul_rows_a16(x, o, None, 0)
    torch.cuda.synchronize()
    same_bits(out.cpu().numpy(), want)
    # tokens 0 and 1 meet every group of the unmixed rows at its extreme:
    # 744 weights of 0.03
    assert np.abs(want[:2, :OUT - 40]).min() > 0.99 * 744 * 0.03
    g.free()


@pytest.mark.parametrize("bits", [4, 8])
def test_prompt_gemm_f16_matches_int8_form(gpu, orc, monkeypatch, bits):
    """A 476-token prompt with the LayerNorm in front (the qkv GEMM of
    config 3, int4-g32 and int8-g32): the fp16 matrix-core form and the
    int8-MFMA form (LLMQ_MFMA_F16=0) give the same bits, and both the
    oracle's."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(476 + bits)
    T, IN, OUT = 476, 768, 2304
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (T, IN)).astype(np.float32)
    lw = rng.normal(1, 0.1, IN).astype(np.float32)
    lb = rng.normal(0, 0.1, IN).astype(np.float32)
    b = rng.normal(0, 0.1, OUT).astype(np.float32)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, 32, False, True)
    o = orc.QuantMatrix.from_f32(w, bits, 32, False, True)
    outs = []
    for f16 in ("1", "0"):
        note("prompt gemm 476", bits, "LLMQ_MFMA_F16 =", f16)
        monkeypatch.setenv("LLMQ_MFMA_F16", f16)
        out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
        lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), ln=(dev(torch, lw), dev(torch, lb)))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    same_bits(outs[0], outs[1])
    same_bits(outs[0], orc.matmul_rows_a16(orc.layernorm(x, lw, lb), o, b, orc.EPI_BIAS))
    g.free()


@pytest.mark.parametrize("T,pos0", [(1, 0), (1, 11), (1, 111), (1, 300), (12, 0), (5, 40), (64, 100), (17, 0),
                                   (476, 0), (300, 700)])
def test_attention_bit_exact(gpu, orc, T, pos0):
    """attend_float_one over the int8 cache: one token (decode) and prompts."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(T * 1000 + pos0)
    NL, NH, HS, MT = 2, 12, 64, 1024
    C = NH * HS
    layer = 1
    qkv_all = rng.normal(0, 1, (pos0 + T, 3 * C)).astype(np.float32)
    note("attention", T, pos0)
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
    same_bits(out.cpu().numpy(), okv.attend(qkv_all[pos0:], layer, T, pos0))
    kv.free()


@pytest.mark.parametrize("T,pos0", [(476, 0), (37, 300)])
def test_prompt_attention_two_chain_form(gpu, orc, T, pos0, monkeypatch):
    """The prompt attention's value pass with two chains a thread
    (LLMQ_PROMPT_SV=0; the default runs four, two tokens x two
    dimensions): the same bits as attend_float_one's."""
    monkeypatch.setenv("LLMQ_PROMPT_SV", "0")
    test_attention_bit_exact(gpu, orc, T, pos0)


def act_layout(K):
    ck = K // 32
    xq = ck * 72
    xsl = (xq + 2 * K + 15) & ~15
    return {"planes": 0, "hsum": ck * 64, "xq": xq, "xsl": xsl, "sx": xsl + 64, "bytes": xsl + 80}


@pytest.mark.parametrize("K,ln", [(768, False), (768, True), (3072, False), (4096, False), (11008, False)])
def test_act_record_contents(gpu, orc, K, ln):
    """llmq_act_prepare: the record's codes and scale are quantize_rows'
    (after LayerNorm when given), its half and lane sums the codes' sums."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(K + ln)
    x = rng.normal(0, 1, (1, K)).astype(np.float32)
    L = act_layout(K)
    assert lm.act_bytes(K) == L["bytes"]
    rec = torch.zeros(L["bytes"], dtype=torch.uint8, device="cuda")
    if ln:
        lw = rng.normal(1, 0.1, K).astype(np.float32)
        lb = rng.normal(0, 0.1, K).astype(np.float32)
        lm.act_prepare(ctx, dev(torch, x), rec, ln=(dev(torch, lw), dev(torch, lb)))
        x = orc.layernorm(x, lw, lb)
    else:
        lm.act_prepare(ctx, dev(torch, x), rec)
    torch.cuda.synchronize()
    b = rec.cpu().numpy()
    q, s = orc.quantize_rows(x)
    xq = b[L["xq"]:L["xq"] + 2 * K].view(np.int16)
    assert np.array_equal(xq, q[0])
    assert b[L["sx"]:L["sx"] + 4].view(np.float32)[0] == s[0]
    hs = b[L["hsum"]:L["hsum"] + 8 * (K // 32)].view(np.int32)
    assert np.array_equal(hs, q[0].astype(np.int64).reshape(-1, 16).sum(1))
    xsl = b[L["xsl"]:L["xsl"] + 64].view(np.int32)
    assert np.array_equal(xsl, q[0].astype(np.int64).reshape(-1, 16, 2).sum((0, 2)))


@pytest.mark.parametrize("fmt,IN,OUT", [((4, 32), 768, 2304), ((4, 32), 3072, 768), ((4, 32), 4096, 11008),
                                        ((8, 0), 768, 50257), ((8, 0), 4096, 200)])
def test_linear_act_bit_exact(gpu, orc, fmt, IN, OUT):
    """llmq_linear_act over a prepared record equals llmq_linear bit for bit
    (and the oracle's matmul_rows_a16)."""
    torch, lm, ctx = gpu
    bits, group = fmt
    rng = np.random.default_rng(IN + OUT)
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (1, IN)).astype(np.float32)
    b = rng.normal(0, 0.1, OUT).astype(np.float32)
    note("linear_act", fmt, IN, OUT)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, False, True)
    o = orc.QuantMatrix.from_f32(w, bits, group, False, True)
    rec = torch.zeros(lm.act_bytes(IN), dtype=torch.uint8, device="cuda")
    xd = dev(torch, x)
    lm.act_prepare(ctx, xd, rec)
    out1 = torch.zeros((1, OUT), dtype=torch.float32, device="cuda")
    out2 = torch.zeros((1, OUT), dtype=torch.float32, device="cuda")
    lm.linear_act(ctx, out1, rec, g, dev(torch, b), gelu=bits == 4)
    lm.linear(ctx, out2, xd, g, dev(torch, b), gelu=bits == 4)
    torch.cuda.synchronize()
    same_bits(out1.cpu().numpy(), out2.cpu().numpy())
    want = orc.matmul_rows_a16(x, o, b, orc.EPI_BIAS | (orc.EPI_GELU if bits == 4 else 0))
    same_bits(out1.cpu().numpy(), want)
    g.free()


DOT_ROW_CASES = [  # (bits, group, sym, IN, OUT, reduce_rows): every dot_row_i16 branch
    (4, 32, False, 768, 2304, True), (4, 32, True, 3072, 768, True),  # BLOCKED
    (8, 0, False, 768, 50257, False), (8, 0, False, 3072, 64, True),  # int8 per channel
    (4, 64, False, 768, 70, True), (4, 128, True, 3072, 40, True), (4, 0, False, 768, 33, True),  # general loop
    (8, 32, False, 768, 64, True), (8, 128, True, 1024, 17, True),
]


@pytest.mark.parametrize("bits,group,sym,IN,OUT,rr", DOT_ROW_CASES)
@pytest.mark.parametrize("big", [False, True])
def test_dot_row_i16_bit_exact(gpu, orc, bits, group, sym, IN, OUT, rr, big):
    """llmq_dot_row_i16 against the oracle's QuantMatrix.dot_row_i16 row by
    row (BLOCKED rows fed permute_x_i16's activations and lane sums), for
    normal codes and for +-32767 codes (the int32 sums' extremes)."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(bits * 1000 + group + IN + OUT + big)
    shape = (IN, OUT) if rr else (OUT, IN)
    w = rng.normal(0, 0.02, shape).astype(np.float32)
    xq = (rng.choice([-32767, 32767], IN) if big else rng.integers(-32767, 32768, IN)).astype(np.int16)
    note("dot_row_i16", bits, group, sym, IN, OUT, "big" if big else "")
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, True, reduce_rows=rr)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, True, reduce_rows=rr)
    out = torch.full((OUT,), float("nan"), dtype=torch.float32, device="cuda")
    g.dot_row_i16(0, dev(torch, xq), out, nrows=OUT)
    one = torch.zeros(1, dtype=torch.float32, device="cuda")
    g.dot_row_i16(OUT - 1, dev(torch, xq), one)  # a single row, the last
    torch.cuda.synchronize()
    ok, x1, xs = o.permute_x_i16(xq)
    if not ok:
        x1 = xq
    want = np.array([o.dot_row_i16(r, x1, xs) for r in range(OUT)], np.float32)
    same_bits(out.cpu().numpy(), want)
    same_bits(one.cpu().numpy(), want[-1:])
    with pytest.raises(lm.LlmqError, match="beyond"):
        g.dot_row_i16(OUT - 1, dev(torch, xq), out, nrows=2)
    g.free()


def test_dot_row_i16_needs_int16_format(gpu):
    torch, lm, ctx = gpu
    w = np.zeros((64, 16), np.float32)
    g = lm.HipQuantMatrix.from_f32(ctx, w, 4, 32, False, False)
    out = torch.zeros(16, dtype=torch.float32, device="cuda")
    with pytest.raises(lm.LlmqError, match="int16 path"):
        g.dot_row_i16(0, torch.zeros(64, dtype=torch.int16, device="cuda"), out)
    g.free()
