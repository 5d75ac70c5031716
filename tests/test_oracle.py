"""Pins the CPU oracle (oracle/llmq_oracle.c) before it is trusted as the
parity checker.  The reference commits no golden vectors for this path, so
each oracle function is checked against something it does not share code
with: a library routine (numpy's float16), the reference's own second spec
(tests/reference.py's fake_quant/aq/kvq restated from its text), the layout
descriptions in the reference's docstrings, ggml's published block layouts
(tests/ggml_pack.py), exact int64 / float64 brute force, or the reference's
own test patterns (tests/a16_kernels.mojo, tests/gguf_int_head.mojo) with
their tolerances.
"""
import numpy as np
import pytest

from tests import ggml_pack


# ----------------------------------------------------------------- float16

def test_f16_rne_matches_numpy(orc):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 1, 4000), rng.normal(0, 1e-5, 2000), rng.normal(0, 1e4, 1000),
        # exact ties between two float16 values, normal and subnormal
        (np.arange(1, 200) + 0.5) * 2.0 ** -10, (np.arange(1, 200) + 0.5) * 2.0 ** -24,
        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e5, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, 6e-8],
    ]).astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16_bits(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)
    back = np.array([orc.f16_bits_to_f32(int(h)) for h in want], np.float32)
    assert np.array_equal(back, want.view(np.float16).astype(np.float32))


# ---------------------------------------------------------------- quantizer

def fake_quant_spec(w, bits, group, sym, reduce_rows):
    """tests/reference.py:135-158 (the reference's NumPy restatement of
    QuantMatrix.from_f32), with round-half-away-from-zero for the tie rule
    the oracle defaults to.  Returns (u, zp, s) in [n, k] / [n, groups]."""
    W = w if reduce_rows else w.T
    rows, cols = W.shape
    g = rows if group == 0 else group
    Wg = W.reshape(rows // g, g, cols).astype(np.float32)
    levels = 2 ** bits - 1
    lo = np.minimum(Wg.min(axis=1), 0)
    hi = np.maximum(Wg.max(axis=1), 0)
    if sym:
        s = np.maximum(-lo, hi) / np.float32(2 ** (bits - 1) - 1)
    else:
        s = (hi - lo) / np.float32(levels)
    s = np.where(s == 0, np.float32(1), s).astype(np.float32).astype(np.float16).astype(np.float32)
    rnd = lambda v: np.sign(v) * np.floor(np.abs(v) + 0.5)
    if sym:
        zp = np.full_like(s, 2 ** (bits - 1))
    else:
        zp = np.clip(rnd((-lo / s).astype(np.float32)), 0, levels)
    u = np.clip(rnd((Wg / s[:, None, :]).astype(np.float32)) + zp[:, None, :], 0, levels)
    # back to [n, k] and [n, groups]
    u = u.reshape(rows, cols).T
    return u.astype(np.int64), zp.T.astype(np.int64), s.T


@pytest.mark.parametrize("bits,group,sym,a16", [
    (4, 32, False, True), (4, 32, True, True), (4, 32, False, False), (4, 64, False, True),
    (4, 128, True, True), (4, 0, False, True), (8, 32, False, True), (8, 0, False, True), (8, 0, True, False),
])
def test_quantizer_matches_reference_py_spec(orc, bits, group, sym, a16):
    rng = np.random.default_rng(bits * 1000 + group + sym)
    IN, OUT = 256, 48
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    w[:, 0] = 0.0  # all-zero groups: scale 1, exact zeros
    w[5, 3] = 0.0
    m = orc.QuantMatrix.from_f32(w, bits, group, sym, a16, reduce_rows=True)
    u_spec, zp_spec, s_spec = fake_quant_spec(w, bits, group, sym, True)
    assert m.blocked == (a16 and bits == 4 and group == 32)
    assert np.array_equal(m.codes().astype(np.int64), u_spec)
    assert np.array_equal(m.zps().astype(np.int64), zp_spec)
    assert np.array_equal(m.scales_f32(), s_spec)
    # invariants: zero weights are exact, the all-zero group has scale 1
    deq = m.dequant()
    assert deq[0, :32].tolist() == [0.0] * 32
    assert deq[3, 5] == 0.0
    assert np.all(m.scales_f32()[0] == 1.0)
    levels = 2 ** bits - 1
    assert m.codes().max() <= levels and m.zps().max() <= levels
    # reconstruction within half a step wherever the code did not clamp
    sc = np.repeat(m.scales_f32(), m.group, axis=1)
    err = np.abs(deq - w.T)
    u = m.codes()
    free = (u > 0) & (u < levels)
    assert np.all((err <= sc / 2 * (1 + 1e-6) + 1e-12)[free])
    # a clamped code is off by less than one step beyond the half step (the
    # float16 scale can be slightly below the group's exact range / levels)
    assert np.all(err <= sc * 1.5)
    assert m.nbytes() == OUT * IN * bits // 8 + 3 * OUT * IN // m.group


def test_quantizer_transposed_head_axis(orc):
    rng = np.random.default_rng(3)
    V, C = 40, 256
    wte = rng.normal(0, 0.02, (V, C)).astype(np.float32)
    m = orc.QuantMatrix.from_f32(wte, 8, 0, False, True, reduce_rows=False)
    u_spec, zp_spec, s_spec = fake_quant_spec(wte, 8, 0, False, False)
    assert (m.n, m.k, m.group) == (V, C, C)
    assert np.array_equal(m.codes().astype(np.int64), u_spec)
    assert np.array_equal(m.scales_f32(), s_spec)


def test_quantizer_tie_rule_switch(orc):
    # one group whose max is 15 * s with s exactly representable: values at
    # k + 0.5 steps are exact ties
    s = 0.0078125  # 2^-7, exact in float16
    col = np.zeros(32, np.float32)
    col[0] = 15 * s
    col[1] = 2.5 * s
    col[2] = -0.0
    w = col.reshape(32, 1)
    try:
        m = orc.QuantMatrix.from_f32(w, 4, 32, False, False, reduce_rows=True)
        assert m.codes()[0, 1] == 3  # half away from zero
        orc.set_round_half_even(True)
        m = orc.QuantMatrix.from_f32(w, 4, 32, False, False, reduce_rows=True)
        assert m.codes()[0, 1] == 2  # half to even
    finally:
        orc.set_round_half_even(False)


# ------------------------------------------------------------- code layouts

def test_blocked_layout_matches_docstring(orc):
    """tensor.mojo:277-288: each 256 weights are 8 steps of 16 bytes; step
    s's lane i (int16 pair i of the 32 codes unpacked as (b & 0xF) ++ (b >> 4))
    holds codes 2p and 2p+1 of group i % 8, with p = 8 * (i // 8) + s."""
    want = {}
    for s in range(8):
        for i in range(16):
            for e in range(2):
                q = 2 * i + e  # position among the 32 unpacked codes
                byte, high = s * 16 + q % 16, q >= 16
                p = 8 * (i // 8) + s
                col = (i % 8) * 32 + 2 * p + e
                want[col] = (byte, high)
    byte, high = orc.nibble_layout(True, np.arange(256))
    assert sorted(want) == list(range(256))
    assert all(want[c] == (int(byte[c]), bool(high[c])) for c in range(256))
    # the C restatement agrees with the vectorised one
    import ctypes
    b, h = ctypes.c_int64(), ctypes.c_int()
    for col in range(0, 512, 7):
        orc.lib().orc_nibble_at(1, col, ctypes.byref(b), ctypes.byref(h))
        bb, hh = orc.nibble_layout(True, [col])
        assert (b.value, bool(h.value)) == (int(bb[0]), bool(hh[0]))


def test_q4_0_style_layout(orc):
    """tensor.mojo:258-260: byte j of each 32 holds weight j low, j+16 high."""
    byte, high = orc.nibble_layout(False, np.arange(64))
    for col in range(64):
        c, j = divmod(col, 32)
        assert (byte[col], high[col]) == (c * 16 + j % 16, j >= 16)


# ------------------------------------------------- activations, integer sums

def test_quantize_rows_invariants(orc):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (5, 768)).astype(np.float32)
    x[3] = 0.0
    xq, sx = orc.quantize_rows(x)
    for t in range(5):
        mx = np.abs(x[t]).max()
        if mx == 0:
            assert sx[t] == 1.0 and not xq[t].any()
            continue
        assert sx[t] == np.float32(mx) / np.float32(32767)
        assert np.abs(xq[t]).max() == 32767
        inv = np.float32(1) / sx[t]
        assert np.all(np.abs(x[t] * inv - xq[t]) <= 0.5)


def exact_rows(m, xq):
    """float64 sum_g scale_g * G[o, g] from brute-force int64 group sums."""
    u = m.codes().astype(np.int64)
    zp = np.repeat(m.zps().astype(np.int64), m.group, axis=1)
    prod = xq.astype(np.int64)[None, :] * (u - zp)
    G = prod.reshape(m.n, m.k // m.group, m.group).sum(axis=2)
    return G, (G.astype(np.float64) * m.scales_f32().astype(np.float64)).sum(axis=1)


@pytest.mark.parametrize("bits,group,sym", [(4, 32, False), (4, 32, True), (4, 64, False), (4, 128, False),
                                            (4, 0, True), (8, 32, False), (8, 0, False)])
def test_dot_row_i16_and_group_sums(orc, bits, group, sym):
    rng = np.random.default_rng(7 + bits + group)
    IN, OUT = 768, 24
    w = rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32)
    m = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    x = rng.uniform(-1, 1, (1, IN)).astype(np.float32)
    xq, sx = orc.quantize_rows(x)
    G, want = exact_rows(m, xq[0])
    assert np.array_equal(m.group_sums(xq[0]), G)
    ok, xp, xs = m.permute_x_i16(xq[0])
    assert ok == m.blocked
    x1 = xp if ok else xq[0]
    got = np.array([m.dot_row_i16(o, x1, xs) for o in range(OUT)], np.float64)
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-6
    # unpack_row_i16: natural-order codes minus the zero point, group scales
    u = m.codes().astype(np.int64)
    zp = np.repeat(m.zps().astype(np.int64), m.group, axis=1)
    for o in (0, 5, OUT - 1):
        dst, sc = m.unpack_row_i16(o)
        assert np.array_equal(dst.astype(np.int64), u[o] - zp[o])
        assert np.array_equal(sc, m.scales_f32()[o])
    # permuted activations' lane sums are exact sums of the lane's inputs
    # (tensor.mojo:282-284: lanes 0-7 hold the first halves of the 8 groups
    # of each 256, lanes 8-15 the second halves)
    if ok:
        xb = xq[0].astype(np.int64).reshape(-1, 8, 2, 16).sum(-1)  # [blk, group, half]
        assert np.array_equal(xs.reshape(-1, 2, 8), xb.transpose(0, 2, 1).astype(np.float32))


def test_dequant_row_exact(orc):
    rng = np.random.default_rng(11)
    w = rng.normal(0, 0.02, (256, 16)).astype(np.float32)
    for bits, group in ((4, 32), (4, 128), (8, 0)):
        for a16 in (False, True):
            m = orc.QuantMatrix.from_f32(w, bits, group, False, a16)
            want = (m.codes().astype(np.float64) - np.repeat(m.zps(), m.group, axis=1)) * \
                np.repeat(m.scales_f32().astype(np.float64), m.group, axis=1)
            assert np.array_equal(m.dequant().astype(np.float64), want)
            x = rng.normal(0, 1, 256).astype(np.float32)
            got = np.array([m.dot_row(o, x) for o in range(16)])
            ref = want @ x.astype(np.float64)
            assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-5


A16_CASES = [  # tests/a16_kernels.mojo:85-94 (format, T, IN, OUT, big)
    *[((4, 32, False), T, 768, 64, False) for T in (1, 3, 4, 9)],
    *[((4, 32, False), T, 768, 70, False) for T in (1, 3, 4, 9)],
    *[((4, 32, True), T, 3072, 64, False) for T in (1, 5)],
    *[((4, 32, False), T, 3072, 40, True) for T in (1, 5)],
    *[((8, 0, False), T, 768, 64, False) for T in (1, 6)],
    *[((8, 0, False), T, 3072, 64, True) for T in (1, 6)],
    *[((4, 0, True), T, 3072, 40, True) for T in (1, 6)],
]


@pytest.mark.parametrize("fmt,T,IN,OUT,big", A16_CASES)
def test_matmul_rows_a16_vs_exact_float64(orc, fmt, T, IN, OUT, big):
    """The reference's own kernel test (tests/a16_kernels.mojo:26-78): the A16
    kernels against float64 over the same quantized values, error relative
    to max |out| below 1e-5."""
    bits, group, sym = fmt
    rng = np.random.default_rng(T * 100 + IN + OUT)
    w = rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32)
    m = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    if big:
        x = (rng.uniform(0.9, 1.0, (T, IN)) * np.where(np.arange(T * IN).reshape(T, IN) % 2 == 0, 1, -1)).astype(np.float32)
    else:
        x = rng.uniform(-1, 1, (T, IN)).astype(np.float32)
    b = rng.uniform(-1, 1, OUT).astype(np.float32)
    out = orc.matmul_rows_a16(x, m, b)
    xq, sx = orc.quantize_rows(x)
    deq = m.dequant().astype(np.float64)
    want = (xq.astype(np.float64) @ deq.T) * sx.astype(np.float64)[:, None] + b
    assert np.max(np.abs(out - want)) / np.max(np.abs(want)) < 1e-5


def test_matmul_epilogues(orc):
    rng = np.random.default_rng(5)
    IN, OUT, T = 256, 40, 3
    m = orc.QuantMatrix.from_f32(rng.normal(0, 0.05, (IN, OUT)).astype(np.float32), 4, 32, False, True)
    x = rng.normal(0, 1, (T, IN)).astype(np.float32)
    b = rng.normal(0, 1, OUT).astype(np.float32)
    plain = orc.matmul_rows_a16(x, m, b, orc.EPI_BIAS).astype(np.float64)
    g = orc.matmul_rows_a16(x, m, b, orc.EPI_BIAS | orc.EPI_GELU)
    want = 0.5 * plain * (1 + np.tanh(np.sqrt(2 / np.pi) * (plain + 0.044715 * plain ** 3)))
    assert np.max(np.abs(g - want)) < 1e-5
    base = rng.normal(0, 1, (T, OUT)).astype(np.float32)
    r = orc.matmul_rows_a16(x, m, b, orc.EPI_BIAS | orc.EPI_RESID, out=base.copy())
    assert np.max(np.abs(r - (plain + base))) < 1e-5
    nb = orc.matmul_rows_a16(x, m, b, 0)
    assert np.max(np.abs(nb - (plain - b))) < 1e-5


# gpt2t.mojo's float-activation --dtype formats (1315-1334): QuantMatrix[B, G, S, A16=False]
FLOAT_ACT = [(8, 0, False), (8, 0, True), (4, 0, False), (4, 0, True), (4, 128, False), (4, 128, True),
             (4, 64, False), (4, 64, True), (4, 32, False), (4, 32, True)]


@pytest.mark.parametrize("fmt", FLOAT_ACT)
@pytest.mark.parametrize("T", [1, 5])
def test_matmul_rows_float_vs_exact_float64(orc, fmt, T):
    """matmul_rows over float activations: T == 1 through dot_row, T > 1
    through mm_tile (rows 0..63) and rows_dot (the 6 tail rows), against
    float64 on the same quantized values, 1e-5 of max |out|, with GELU and
    the residual."""
    bits, group, sym = fmt
    rng = np.random.default_rng(T * 7 + bits + group)
    IN, OUT = 512, 70
    m = orc.QuantMatrix.from_f32(rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32), bits, group, sym, False)
    x = rng.uniform(-1, 1, (T, IN)).astype(np.float32)
    b = rng.uniform(-1, 1, OUT).astype(np.float32)
    want = x.astype(np.float64) @ m.dequant().astype(np.float64).T + b
    out = orc.matmul_rows(x, m, b)
    assert np.max(np.abs(out - want)) / np.max(np.abs(want)) < 1e-5
    g = orc.matmul_rows(x, m, b, orc.EPI_BIAS | orc.EPI_GELU)
    gw = 0.5 * want * (1 + np.tanh(np.sqrt(2 / np.pi) * (want + 0.044715 * want ** 3)))
    assert np.max(np.abs(g - gw)) < 1e-5
    base = rng.normal(0, 1, (T, OUT)).astype(np.float32)
    r = orc.matmul_rows(x, m, b, orc.EPI_BIAS | orc.EPI_RESID, out=base.copy())
    assert np.max(np.abs(r - (want + base))) < 1e-5


@pytest.mark.parametrize("fmt", [(8, 0, False), (4, 32, True), (4, 128, False)])
def test_matmul_rows_float_one_hot_exact(orc, fmt):
    """x = unit rows: every path (dot_row, mm_tile, rows_dot) returns the
    selected dequantized column plus the bias bit for bit, which pins the
    row / column indexing and the transposition."""
    bits, group, sym = fmt
    rng = np.random.default_rng(3)
    IN, OUT = 256, 70
    m = orc.QuantMatrix.from_f32(rng.normal(0, 0.05, (IN, OUT)).astype(np.float32), bits, group, sym, False)
    deq = m.dequant()
    b = rng.normal(0, 1, OUT).astype(np.float32)
    cols = [3, 100, 255, 31, 32]
    x = np.zeros((len(cols), IN), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    want = deq[:, cols].T + b
    assert np.array_equal(orc.matmul_rows(x, m, b), want)
    assert np.array_equal(orc.matmul_rows(x[1:2], m, b), want[1:2])


# ---------------------------------------------------------------------- GGUF

KINDS = ["Q4_0", "Q4_1", "Q8_0", "Q4_K", "Q5_K", "Q6_K"]


def test_k_scale_min_all_patterns(orc):
    rng = np.random.default_rng(2)
    for _ in range(200):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = ggml_pack.pack_k_scales(sc, mn)
        for j in range(8):
            assert orc.k_scale_min(q, j) == (sc[j], mn[j])
    for v in (0, 63, 0b110000, 0b001111):  # boundary bit patterns
        q = ggml_pack.pack_k_scales(np.full(8, v), np.full(8, 63 - v))
        assert all(orc.k_scale_min(q, j) == (v, 63 - v) for j in range(8))


@pytest.mark.parametrize("kind", KINDS)
def test_gguf_dequant_known_answers(orc, kind):
    rng = np.random.default_rng(KINDS.index(kind))
    t = orc.GGML[kind]
    bs = orc.gguf_block_size(t)
    nb = 8
    blocks, w = ggml_pack.random_blocks(kind, nb, rng)
    assert blocks.size == nb * orc.gguf_block_bytes(t)
    got = orc.gguf_dequant(t, blocks, 1, nb * bs)[0].astype(np.float64)
    tol = 1e-6 * np.max(np.abs(w)) if kind in ("Q4_1", "Q4_K", "Q5_K") else 0.0
    assert np.max(np.abs(got - w)) <= tol
    x = rng.normal(0, 1, nb * bs).astype(np.float32)
    d = orc.gguf_dot_row(t, blocks, nb * bs, x)
    want = w @ x.astype(np.float64)
    assert abs(d - want) <= 1e-5 * np.sum(np.abs(w * x))


def test_gguf_constant_blocks(orc):
    # all-constant codes: every weight equals the closed form
    b, w = ggml_pack.pack_q4_0(0.5, np.full(32, 11))
    assert np.all(orc.gguf_dequant(2, b, 1, 32) == 1.5)
    b, w = ggml_pack.pack_q6_k(0.25, np.r_[np.full(15, 0), 2], np.full(256, 33))
    got = orc.gguf_dequant(14, b, 1, 256)[0]
    assert np.all(got[:240] == 0.0) and np.all(got[240:] == 0.5)


@pytest.mark.parametrize("kind", ["Q6_K", "Q8_0"])
@pytest.mark.parametrize("big", [False, True])
def test_gguf_int16_head(orc, kind, big):
    """tests/gguf_int_head.mojo:26-77: the int16 head agrees with float64
    over the int16 activations (< 1e-5 of max |logit|) and one-token equals
    many-token bit for bit."""
    rng = np.random.default_rng(31 + big)
    t = orc.GGML[kind]
    V, C, T = 40, 512, 5
    blocks, w = ggml_pack.random_blocks(kind, V * C // orc.gguf_block_size(t), rng)
    w = w.reshape(V, C)
    if big:
        h = (rng.uniform(0.9, 1.0, (T, C)) * np.where(np.arange(T * C).reshape(T, C) % 2 == 0, 1, -1)).astype(np.float32)
    else:
        h = rng.uniform(-3, 3, (T, C)).astype(np.float32)
    many = orc.gguf_head_i16(t, blocks, V, C, h)
    for tt in range(T):
        one = orc.gguf_head_i16(t, blocks, V, C, h[tt])
        assert np.array_equal(one[0], many[tt])
    xq, sx = orc.quantize_rows(h)
    want = (xq.astype(np.float64) @ w.T) * sx[:, None].astype(np.float64)
    assert np.max(np.abs(many - want)) / np.max(np.abs(want)) < 1e-5
    # unpack_row_i16 gives exact int16 weights and the group's d
    rb = C // orc.gguf_block_size(t) * orc.gguf_block_bytes(t)
    dst, sc = orc.gguf_unpack_row_i16(t, blocks[:rb], C)
    G = orc.gguf_block_size(t)
    recon = dst.astype(np.float64) * np.repeat(sc.astype(np.float64), G)
    assert np.allclose(recon, w[0], rtol=0, atol=1e-12)


# ------------------------------------------------------- LN, KV, attention

def test_layernorm_closed_form(orc):
    rng = np.random.default_rng(4)
    x = rng.normal(0.3, 2, (3, 768)).astype(np.float32)
    w = rng.normal(1, 0.1, 768).astype(np.float32)
    b = rng.normal(0, 0.1, 768).astype(np.float32)
    got = orc.layernorm(x, w, b)
    xd = x.astype(np.float64)
    want = (xd - xd.mean(-1, keepdims=True)) / np.sqrt(xd.var(-1, keepdims=True) + 1e-5) * w + b
    assert np.max(np.abs(got - want)) < 2e-5


def test_kv_store_and_attention_vs_float64(orc):
    """QuantKV[8] store (kvcache.mojo:320-342, invariants as quantize_rows with
    127) and attend_float_one against textbook softmax attention in float64
    over the dequantized cache (the int_attention_check pattern)."""
    rng = np.random.default_rng(9)
    NL, MT, NH, HS = 2, 32, 3, 64
    C = NH * HS
    kv = orc.QuantKV8(NL, MT, NH, HS)
    T, pos0, layer = 5, 7, 1
    qkv_all = rng.normal(0, 1, (pos0 + T, 3 * C)).astype(np.float32)
    qkv_all[2, C:C + HS] = 0.0  # a zero head: scale 1, zero codes
    for p in range(pos0 + T):
        kv.store(layer, p, qkv_all[p, C:2 * C], qkv_all[p, 2 * C:])
    K = kv.k.reshape(NL, MT, NH, HS)[layer]
    ks = kv.ks.reshape(NL, MT, NH)[layer]
    assert ks[2, 0] == 1.0 and not K[2, 0].any()
    for p in range(pos0 + T):
        for h in range(NH):
            k = qkv_all[p, C + h * HS:C + (h + 1) * HS]
            mx = np.abs(k).max()
            if mx:
                assert ks[p, h] == np.float32(mx) / np.float32(127)
                assert np.abs(K[p, h]).max() == 127
                assert np.all(np.abs(k * (np.float32(1) / ks[p, h]) - K[p, h]) <= 0.5)
    out = kv.attend(qkv_all[pos0:], layer, T, pos0)
    V = kv.v.reshape(NL, MT, NH, HS)[layer].astype(np.float64) * kv.vs.reshape(NL, MT, NH)[layer][..., None]
    Kd = K.astype(np.float64) * ks[..., None]
    worst = 0.0
    for t in range(T):
        for h in range(NH):
            q = qkv_all[pos0 + t, h * HS:(h + 1) * HS].astype(np.float64)
            n = pos0 + t + 1
            s = Kd[:n, h] @ q / 8.0
            p = np.exp(s - s.max())
            p /= p.sum()
            want = p @ V[:n, h]
            worst = max(worst, np.max(np.abs(out[t, h * HS:(h + 1) * HS] - want)) / np.max(np.abs(want)))
    assert worst < 1e-5


def test_argmax_first_max_wins(orc):
    a = np.zeros(50257, np.float32)
    a[[7, 9, 50000]] = 3.0
    assert orc.argmax(a) == 7


# -------------------------------------------------------- exp, tanh, GELU

def _ulps(got, want64):
    """|got - want| in units of the float32 spacing at want."""
    sp = np.spacing(np.abs(want64).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / sp


def test_exp_within_one_ulp_of_float64(orc):
    """orc_exp (the float path's softmax exp) against float64 exp over the
    range softmax feeds it and beyond, plus its special values."""
    x = np.concatenate([np.linspace(-87.0, 88.0, 3_000_001), np.linspace(-1, 1, 200_001)]).astype(np.float32)
    got = orc.ref_exp(x)
    assert _ulps(got, np.exp(x.astype(np.float64))).max() < 1.0
    assert orc.ref_exp(np.float32([0.0]))[0] == 1.0
    assert orc.ref_exp(np.float32([-87.5, -1e30, -np.inf]))[:].tolist() == [0.0, 0.0, 0.0]
    assert np.isinf(orc.ref_exp(np.float32([89.0]))[0]) and np.isnan(orc.ref_exp(np.float32([np.nan]))[0])
    # monotone on a fine grid (a dropped term or a wrong reduction breaks it)
    g = orc.ref_exp(np.linspace(-20, 20, 400_001).astype(np.float32))
    assert np.all(np.diff(g.astype(np.float64)) >= 0)


def test_tanh_within_ulps_of_float64(orc):
    x = np.concatenate([np.linspace(-12, 12, 2_400_001), np.linspace(-0.7, 0.7, 200_001),
                        np.float32([1e-30, -1e-30, 0.0, 0.625, -0.625, 10.0, 50.0])]).astype(np.float32)
    got = orc.ref_tanh(x)
    assert _ulps(got, np.tanh(x.astype(np.float64))).max() < 1.5
    assert np.array_equal(orc.ref_tanh(-x), -got)  # odd
    assert orc.ref_tanh(np.float32([10.0, 1e6]))[:].tolist() == [1.0, 1.0]


def test_gelu_closed_form(orc):
    """store_out's GELU (kernels.mojo:43-45) in float64 against the oracle."""
    r = np.linspace(-12, 12, 200_001).astype(np.float32)
    r64 = r.astype(np.float64)
    want = 0.5 * r64 * (1 + np.tanh(0.7978845608028654 * (r64 + 0.044715 * r64 ** 3)))
    got = orc.gelu(r).astype(np.float64)
    # 1 + tanh cancels for r << 0 in the reference's own formula, so the
    # bound there is absolute, in units of |r| * 2^-24.
    pos = r > 0
    assert np.max(np.abs(got[pos] - want[pos]) / want[pos]) < 4e-7
    assert np.max(np.abs(got - want) / (np.maximum(np.abs(r64), 1.0) * 2.0 ** -24)) < 4.0
