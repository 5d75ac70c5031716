"""TEST INFRASTRUCTURE ONLY: ctypes bindings to the CPU oracle (llmq_oracle.c).

The oracle is a C restatement of llm_mojo's CPU arithmetic for the quantized
matmul path (tensor.mojo, kernels.mojo, gguf.mojo, kvcache.mojo,
gpt2t.mojo).  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg import this module, and only as the checker or the timed CPU baseline;
the product (llm_mojo_amd/) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

EPI_BIAS, EPI_GELU, EPI_RESID = 1, 2, 4
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


def build():
    """Compiles liboracle.so with oracle/Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class QM(ctypes.Structure):
    """orc_qm: a QuantMatrix in the reference's own storage layout."""

    _fields_ = [
        ("bits", ctypes.c_int32),
        ("sym", ctypes.c_int32),
        ("a16", ctypes.c_int32),
        ("blocked", ctypes.c_int32),
        ("perch", ctypes.c_int32),
        ("n", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("group", ctypes.c_int64),
        ("data", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("zp", ctypes.c_void_p),
    ]


class KV(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_int32),
        ("max_t", ctypes.c_int32),
        ("n_head", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("ks", ctypes.c_void_p),
        ("vs", ctypes.c_void_p),
    ]


P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int


def _declare(L):
    sig = {
        "orc_set_round_half_even": (None, [I32]),
        "orc_ties": (None, [P]),
        "orc_cpu_vnni": (I32, []),
        "orc_cpu_generate": (I32, [P, P, I32, I32, I32, P, P]),
        "orc_cpu_decode": (P, [P, I64, I32, I32]),
        "orc_cpu_head_seconds": (ctypes.c_double, [P, I32, I32]),
        "orc_cpu_set_fast": (I32, [I32]),
        "orc_cpu_prompt": (P, [P, P, I32, I32, P]),
        "orc_cpu_gemv_seconds": (ctypes.c_double, [P, I32, P, P, I32, I32]),
        "orc_cpu_gguf_gemv_seconds": (ctypes.c_double, [I32, P, I32, I64, I64, P, P, I32, I32]),
        "orc_cpu_gguf_dot_row": (ctypes.c_float, [I32, P, I64, P]),
        "orc_reset_ties": (None, []),
        "orc_exp": (ctypes.c_float, [ctypes.c_float]),
        "orc_tanh": (ctypes.c_float, [ctypes.c_float]),
        "orc_exp_n": (None, [P, P, I64]),
        "orc_tanh_n": (None, [P, P, I64]),
        "orc_gelu_n": (None, [P, P, I64]),
        "orc_set_threads": (None, [I32]),
        "orc_get_threads": (I32, []),
        "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_nibble_at": (None, [I32, I64, P, P]),
        "orc_qm_from_f32": (I32, [P, P, I64, I64, I32]),
        "orc_qm_code": (I32, [P, I64, I64]),
        "orc_qm_nbytes": (I64, [P]),
        "orc_qm_dequant_row": (None, [P, I64, P]),
        "orc_qm_dot_row": (ctypes.c_float, [P, I64, P]),
        "orc_qm_matmul_rows": (None, [P, P, P, P, I64, I64, I64, I32]),
        "orc_qm_permute_x_i16": (I32, [P, P, I64, P, P]),
        "orc_qm_dot_row_i16": (ctypes.c_float, [P, I64, P, P]),
        "orc_qm_unpack_row_i16": (None, [P, I64, P, P]),
        "orc_qm_group_sums": (None, [P, P, P]),
        "orc_quantize_rows": (None, [P, I64, I64, P, P]),
        "orc_matmul_rows_a16": (None, [P, P, P, P, I64, I64, I64, I32]),
        "orc_gguf_block_size": (I32, [I32]),
        "orc_gguf_block_bytes": (I32, [I32]),
        "orc_k_scale_min": (None, [P, I32, P, P]),
        "orc_gguf_dequant_row": (None, [I32, P, I64, P]),
        "orc_gguf_dequant_rows": (None, [I32, P, I64, I64, I64, P]),
        "orc_gguf_dot_row": (ctypes.c_float, [I32, P, I64, P]),
        "orc_gguf_dot_row_i16": (ctypes.c_float, [I32, P, I64, P]),
        "orc_gguf_unpack_row_i16": (None, [I32, P, I64, P, P]),
        "orc_gguf_gemv": (None, [I32, P, I64, I64, P, P, P, I32]),
        "orc_gguf_head_i16": (None, [I32, P, I64, I64, P, I64, P]),
        "orc_layernorm": (None, [P, P, P, P, I64, I64]),
        "orc_kv_store": (None, [P, I32, I32, P, P]),
        "orc_kv_attend_one": (None, [P, P, P, I32, I32, I32, I32]),
        "orc_kv_attend": (None, [P, P, P, I32, I32, I32]),
        "orc_exp_multiplier": (I64, [ctypes.c_double]),
        "orc_exp2_neg": (I64, [I64, I64]),
        "orc_masked_exp": (I64, [P, P, I32, I32, I64, P]),
        "orc_masked_softmax": (None, [P, P, I32, I32, I64, P]),
        "orc_ikv_store": (None, [P, I32, I32, P, P]),
        "orc_ikv_attend_one": (None, [P, P, P, I32, I32, I32, I32]),
        "orc_ikv_attend": (None, [P, P, P, I32, I32, I32]),
        "orc_rng_init": (None, [P, I64]),
        "orc_rng_uniform": (ctypes.c_float, [P]),
        "orc_argmax": (I64, [P, I64]),
        "orc_gpt2_new": (P, [P, I32, I32, I32]),
        "orc_gpt2_new_fmt": (P, [P, I32, I32, I32, I32, I32, I32, I32, I32]),
        "orc_gpt2_free": (None, [P]),
        "orc_gpt2_set_capture": (None, [P, P]),
        "orc_gpt2_set_attention": (None, [P, I32]),
        "orc_gpt2_forward_all": (None, [P, P, I32, P]),
        "orc_score_rows": (None, [P, I64, P, P, P, I32, I32, I32]),
        "orc_gpt2_mat": (P, [P, I32]),
        "orc_gpt2_kv": (P, [P]),
        "orc_gpt2_act": (P, [P, I32]),
        "orc_gpt2_forward": (P, [P, P, I32, I32]),
        "orc_gpt2_generate": (I32, [P, P, I32, I32, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def set_round_half_even(on):
    lib().orc_set_round_half_even(1 if on else 0)


TIE_SITES = ("weights", "activations", "kv", "other")


def cpu_vnni():
    """1 when this CPU runs the baseline's VPDPWSSD path (cpuid: AVX-512
    F/BW/DQ/VL/VNNI, F16C, FMA, OS-enabled), 0 for the scalar emulation."""
    return int(lib().orc_cpu_vnni())


def ties(reset=False):
    """Exact .5 ties the rounding sites met since the last reset (the cases
    where the unpinned tie rule decides a code): {site: count}."""
    out = np.zeros(4, np.int64)
    lib().orc_ties(out.ctypes.data)
    if reset:
        lib().orc_reset_ties()
    return dict(zip(TIE_SITES, (int(v) for v in out)))


def set_threads(n):
    lib().orc_set_threads(int(n))


def cpu_set_fast(on):
    """Switches the oracle's matmuls, quantizer and attention to their AVX-512
    VNNI forms (bit-identical; the CPU baseline) or back; returns whether on."""
    return bool(lib().orc_cpu_set_fast(1 if on else 0))


def cpu_gemv_seconds(mats, x, threads, reps=100):
    """linear_team of one token (kernels.mojo:774-866) on a team of
    `threads`: median seconds over `reps` calls cycling over `mats` (copies
    of one QuantMatrix, from memory rather than cache)."""
    arr = (ctypes.c_void_p * len(mats))(*[ctypes.addressof(m.s) for m in mats])
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(mats[0].n, np.float32)
    t = lib().orc_cpu_gemv_seconds(arr, len(mats), ptr(x), ptr(out), int(threads), int(reps))
    return float(t), out


def cpu_gguf_gemv_seconds(t, blocks_list, rows, cols, x, threads, reps=100):
    """GGUFMatrix.dot_row over every row (AVX-512 decoders) on a team of
    `threads`: median seconds over `reps` calls cycling over the copies."""
    keep = [np.ascontiguousarray(b, np.uint8) for b in blocks_list]
    arr = (ctypes.c_void_p * len(keep))(*[b.ctypes.data for b in keep])
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(rows, np.float32)
    sec = lib().orc_cpu_gguf_gemv_seconds(int(t), arr, len(keep), int(rows), int(cols), ptr(x), ptr(out),
                                          int(threads), int(reps))
    return float(sec), out


def cpu_gguf_dot_row(t, row_bytes, cols, x):
    """One row through the baseline's AVX-512 GGUF decoder."""
    return lib().orc_cpu_gguf_dot_row(t, ptr(np.ascontiguousarray(row_bytes, np.uint8)), cols,
                                      ptr(np.ascontiguousarray(x, np.float32)))


def f32_to_f16_bits(v):
    return lib().orc_f32_to_f16(ctypes.c_float(v))


def f16_bits_to_f32(h):
    return lib().orc_f16_to_f32(ctypes.c_uint16(h))


class QuantMatrix:
    """QuantMatrix[bits, group, sym, a16] (tensor.mojo:230-661) on the CPU."""

    def __init__(self, bits, group, sym, a16):
        self.bits, self.group_param, self.sym, self.a16 = bits, group, sym, a16

    @classmethod
    def from_f32(cls, src, bits, group, sym=False, a16=True, reduce_rows=True):
        src = np.ascontiguousarray(src, dtype=np.float32)
        rows, cols = src.shape
        self = cls(bits, group, sym, a16)
        n, k = (cols, rows) if reduce_rows else (rows, cols)
        g = k if group == 0 else group
        if a16 and bits == 4 and g == 32 and k % 256:
            # BLOCKED (tensor.mojo:296, 394-404) addresses whole 256-weight blocks
            raise ValueError("int4-g32-a16 needs the reduction axis in whole 256-weight blocks")
        self.data = np.zeros(n * k * bits // 8, np.uint8)
        self.scale = np.zeros(n * k // g, np.uint16)
        self.zp = np.zeros(n * k // g, np.uint8)
        self.s = QM(bits, 1 if sym else 0, 1 if a16 else 0, 0, 0, 0, 0, group,
                    self.data.ctypes.data, self.scale.ctypes.data, self.zp.ctypes.data)
        rc = lib().orc_qm_from_f32(ctypes.byref(self.s), ptr(src), rows, cols, 1 if reduce_rows else 0)
        if rc != 0:
            raise ValueError("group size must divide the reduction axis and be a multiple of 32")
        self.n, self.k, self.group = self.s.n, self.s.k, self.s.group
        self.blocked = bool(self.s.blocked)
        return self

    def clone(self):
        """A copy with its own codes, scales and zero points (for timing over
        rotated buffers)."""
        c = QuantMatrix(self.bits, self.group_param, self.sym, self.a16)
        c.data, c.scale, c.zp = self.data.copy(), self.scale.copy(), self.zp.copy()
        c.s = QM(self.s.bits, self.s.sym, self.s.a16, self.s.blocked, self.s.perch, self.s.n, self.s.k, self.s.group,
                 c.data.ctypes.data, c.scale.ctypes.data, c.zp.ctypes.data)
        c.n, c.k, c.group, c.blocked = self.n, self.k, self.group, self.blocked
        return c

    @property
    def ref(self):
        return ctypes.byref(self.s)

    def nbytes(self):
        return lib().orc_qm_nbytes(self.ref)

    def code(self, row, col):
        return lib().orc_qm_code(self.ref, row, col)

    def codes(self):
        """All codes u[n, k] in natural column order (via nibble_at)."""
        if self.bits == 8:
            return self.data.reshape(self.n, self.k).copy()
        d = self.data.reshape(self.n, self.k // 2)
        cols = np.arange(self.k)
        byte, high = nibble_layout(self.blocked, cols)
        b = d[:, byte]
        return np.where(high[None, :], b >> 4, b & 0xF).astype(np.uint8)

    def scales_f32(self):
        return self.scale.view(np.float16).astype(np.float32).reshape(self.n, self.k // self.group)

    def zps(self):
        return self.zp.reshape(self.n, self.k // self.group)

    def dequant(self):
        out = np.zeros((self.n, self.k), np.float32)
        for r in range(self.n):
            lib().orc_qm_dequant_row(self.ref, r, ptr(out[r]))
        return out

    def dot_row(self, row, x):
        x = np.ascontiguousarray(x, np.float32)
        return lib().orc_qm_dot_row(self.ref, row, ptr(x))

    def permute_x_i16(self, xq):
        xp = np.zeros(self.k, np.int16)
        xs = np.zeros(self.k // 16, np.float32)
        ok = lib().orc_qm_permute_x_i16(self.ref, ptr(xq), self.k, ptr(xp), ptr(xs))
        return bool(ok), xp, xs

    def dot_row_i16(self, row, x1, xs):
        return lib().orc_qm_dot_row_i16(self.ref, row, ptr(x1), ptr(xs))

    def unpack_row_i16(self, row):
        dst = np.zeros(self.k, np.int16)
        sc = np.zeros(self.k // self.group, np.float32)
        lib().orc_qm_unpack_row_i16(self.ref, row, ptr(dst), ptr(sc))
        return dst, sc

    def group_sums(self, xq):
        G = np.zeros(self.n * (self.k // self.group), np.int64)
        lib().orc_qm_group_sums(self.ref, ptr(np.ascontiguousarray(xq, np.int16)), ptr(G))
        return G.reshape(self.n, self.k // self.group)


def nibble_layout(blocked, cols):
    """Vectorised nibble_at (tensor.mojo:385-404): (byte, high) per column."""
    cols = np.asarray(cols, np.int64)
    if blocked:
        w = cols % 256
        e = w % 32
        p = e // 2
        lane = w // 32 + 8 * (p // 8)
        chunk = (cols // 256) * 8 + p % 8
        j = 2 * lane + e % 2
    else:
        chunk = cols // 32
        j = cols % 32
    return chunk * 16 + j % 16, j >= 16


def _map_f32(fn, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    getattr(lib(), fn)(ptr(x), ptr(y), x.size)
    return y


def ref_exp(x):
    """The float path's exp (orc_exp), elementwise."""
    return _map_f32("orc_exp_n", x)


def ref_tanh(x):
    """The float path's tanh (orc_tanh), elementwise."""
    return _map_f32("orc_tanh_n", x)


def gelu(x):
    """store_out's GELU (kernels.mojo:43-45) on the oracle's tanh."""
    return _map_f32("orc_gelu_n", x)


def quantize_rows(x):
    x = np.ascontiguousarray(x, np.float32)
    T, IN = x.shape
    xq = np.zeros((T, IN), np.int16)
    sx = np.zeros(T, np.float32)
    lib().orc_quantize_rows(ptr(x), T, IN, ptr(xq), ptr(sx))
    return xq, sx


def matmul_rows_a16(x, w, b=None, flags=EPI_BIAS, out=None):
    """out[T, OUT] (+)= act(x @ w^T + b) as kernels.matmul_rows_a16."""
    x = np.ascontiguousarray(x, np.float32)
    T, IN = x.shape
    if out is None:
        out = np.zeros((T, w.n), np.float32)
    if b is None:
        b = np.zeros(w.n, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    lib().orc_matmul_rows_a16(ptr(out), ptr(x), w.ref, ptr(b), T, IN, w.n, flags)
    return out


def matmul_rows(x, w, b=None, flags=EPI_BIAS, out=None):
    """out[T, OUT] (+)= act(x @ w^T + b) as kernels.matmul_rows over a
    QuantMatrix with A16 = False (float activations)."""
    x = np.ascontiguousarray(x, np.float32)
    T, IN = x.shape
    if out is None:
        out = np.zeros((T, w.n), np.float32)
    if b is None:
        b = np.zeros(w.n, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    lib().orc_qm_matmul_rows(ptr(out), ptr(x), w.ref, ptr(b), T, IN, w.n, flags)
    return out


def gguf_block_size(t):
    return lib().orc_gguf_block_size(t)


def gguf_block_bytes(t):
    return lib().orc_gguf_block_bytes(t)


def gguf_dequant(t, w, rows, cols):
    w = np.ascontiguousarray(w, np.uint8)
    rb = cols // gguf_block_size(t) * gguf_block_bytes(t)
    assert w.size >= rows * rb, "gguf_dequant: too few block bytes"
    out = np.zeros((rows, cols), np.float32)
    lib().orc_gguf_dequant_rows(t, w.ctypes.data, rows, rb, cols, ptr(out))
    return out


def gguf_dot_row(t, row_bytes, cols, x):
    return lib().orc_gguf_dot_row(t, ptr(np.ascontiguousarray(row_bytes, np.uint8)), cols,
                                  ptr(np.ascontiguousarray(x, np.float32)))


def gguf_gemv(t, w, rows, cols, x, b=None, flags=0, out=None):
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    if out is None:
        out = np.zeros(rows, np.float32)
    if b is None:
        b = np.zeros(rows, np.float32)
    lib().orc_gguf_gemv(t, ptr(w), rows, cols, ptr(x), ptr(np.ascontiguousarray(b, np.float32)), ptr(out), flags)
    return out


def gguf_head_i16(t, w, V, C, h):
    h = np.ascontiguousarray(h, np.float32).reshape(-1, C)
    T = h.shape[0]
    out = np.zeros((T, V), np.float32)
    lib().orc_gguf_head_i16(t, ptr(np.ascontiguousarray(w, np.uint8)), V, C, ptr(h), T, ptr(out))
    return out


def gguf_dot_row_i16(t, row_bytes, cols, xq):
    return lib().orc_gguf_dot_row_i16(t, ptr(np.ascontiguousarray(row_bytes, np.uint8)), cols,
                                      ptr(np.ascontiguousarray(xq, np.int16)))


def gguf_unpack_row_i16(t, row_bytes, cols):
    dst = np.zeros(cols, np.int16)
    sc = np.zeros(cols // (256 if t == GGML["Q6_K"] else 32), np.float32)
    lib().orc_gguf_unpack_row_i16(t, ptr(np.ascontiguousarray(row_bytes, np.uint8)), cols, ptr(dst), ptr(sc))
    return dst, sc


def k_scale_min(q12, j):
    q12 = np.ascontiguousarray(q12, np.uint8)
    sc = ctypes.c_int()
    mn = ctypes.c_int()
    lib().orc_k_scale_min(ptr(q12), j, ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


def layernorm(x, w, b):
    x = np.ascontiguousarray(x, np.float32)
    T, C = x.shape
    out = np.zeros_like(x)
    lib().orc_layernorm(ptr(out), ptr(x), ptr(np.ascontiguousarray(w, np.float32)),
                        ptr(np.ascontiguousarray(b, np.float32)), T, C)
    return out


class QuantKV8:
    """QuantKV[8] (kvcache.mojo:248-385) on the CPU."""

    def __init__(self, n_layer, max_t, n_head, head_dim):
        n = n_layer * max_t * n_head * head_dim
        ns = n_layer * max_t * n_head
        self.k = np.zeros(n, np.int8)
        self.v = np.zeros(n, np.int8)
        self.ks = np.zeros(ns, np.float32)
        self.vs = np.zeros(ns, np.float32)
        self.s = KV(n_layer, max_t, n_head, head_dim, self.k.ctypes.data, self.v.ctypes.data,
                    self.ks.ctypes.data, self.vs.ctypes.data)
        self.C = n_head * head_dim

    def store(self, layer, pos, k, v):
        lib().orc_kv_store(ctypes.byref(self.s), layer, pos, ptr(np.ascontiguousarray(k, np.float32)),
                           ptr(np.ascontiguousarray(v, np.float32)))

    def attend(self, qkv, layer, T, pos0):
        qkv = np.ascontiguousarray(qkv, np.float32)
        out = np.zeros((T, self.C), np.float32)
        lib().orc_kv_attend(ctypes.byref(self.s), ptr(out), ptr(qkv), layer, T, pos0)
        return out


MASKED = -(1 << 31)  # intmath.mojo:35


def exp_multiplier(scale):
    """intmath.exp_multiplier (intmath.mojo:48-50)."""
    return lib().orc_exp_multiplier(float(scale))


def exp2_neg(d, mult):
    """intmath.exp2_neg (intmath.mojo:53-65) for one score difference."""
    return lib().orc_exp2_neg(int(d), int(mult))


def _padded_i32(x, n):
    nr = (n + 15) // 16 * 16
    buf = np.zeros(max(nr, 16), np.int32)
    buf[:len(x)] = x
    return buf


def masked_exp(x, n, mult, mask=None):
    """intmath.masked_exp (intmath.mojo:93-123): (e [nr] in Q30, int64 total)."""
    xb = _padded_i32(np.asarray(x, np.int32), n)
    mb = _padded_i32(np.asarray(mask, np.int32), n) if mask is not None else None
    e = np.zeros_like(xb)
    t = lib().orc_masked_exp(ptr(xb), ptr(mb), 1 if mask is not None else 0, n, int(mult), ptr(e))
    return e[:(n + 15) // 16 * 16], t


def masked_softmax(x, n, mult, mask=None):
    """intmath.masked_softmax (intmath.mojo:126-140): Q15 uint16 [nr]."""
    xb = _padded_i32(np.asarray(x, np.int32), n)
    mb = _padded_i32(np.asarray(mask, np.int32), n) if mask is not None else None
    p = np.zeros(len(xb), np.uint16)
    lib().orc_masked_softmax(ptr(xb), ptr(mb), 1 if mask is not None else 0, n, int(mult), ptr(p))
    return p[:(n + 15) // 16 * 16]


class IntAttnKV:
    """IntAttnKV (int_attention.mojo:62-269) on the CPU: int8 keys and values
    [layer, pos, head, head_dim], scales * 2^24 as int32 [layer, pos, head]."""

    def __init__(self, n_layer, max_t, n_head, head_dim):
        n = n_layer * max_t * n_head * head_dim
        ns = n_layer * max_t * n_head
        self.k = np.zeros(n, np.int8)
        self.v = np.zeros(n, np.int8)
        self.kq = np.zeros(ns, np.int32)
        self.vq = np.zeros(ns, np.int32)
        self.s = KV(n_layer, max_t, n_head, head_dim, self.k.ctypes.data, self.v.ctypes.data,
                    self.kq.ctypes.data, self.vq.ctypes.data)
        self.C = n_head * head_dim

    def store(self, layer, pos, k, v):
        lib().orc_ikv_store(ctypes.byref(self.s), layer, pos, ptr(np.ascontiguousarray(k, np.float32)),
                            ptr(np.ascontiguousarray(v, np.float32)))

    def attend(self, qkv, layer, T, pos0):
        qkv = np.ascontiguousarray(qkv, np.float32)
        out = np.zeros((T, self.C), np.float32)
        lib().orc_ikv_attend(ctypes.byref(self.s), ptr(out), ptr(qkv), layer, T, pos0)
        return out


class Rng:
    """gpt2t.mojo's Rng (777-789)."""

    class _S(ctypes.Structure):
        _fields_ = [("state", ctypes.c_uint64)]

    def __init__(self, seed):
        self.s = Rng._S()
        lib().orc_rng_init(ctypes.byref(self.s), seed)

    def uniform(self):
        return lib().orc_rng_uniform(ctypes.byref(self.s))


def argmax(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    return lib().orc_argmax(ptr(logits), logits.size)


def score_rows(logits, targets, r0, r1, base=None):
    """score_rows (gpt2t.mojo:1040-1095): stats [6, rows] (NLL, NLL_BASE,
    AGREE, KL, DIFF_MAX, DIFF_SUM; all but NLL zero without base)."""
    logits = np.ascontiguousarray(logits, np.float32)
    base = np.ascontiguousarray(base, np.float32) if base is not None else None
    targets = np.ascontiguousarray(targets, np.int64)
    rows, V = logits.shape
    stats = np.zeros((6, rows))
    lib().orc_score_rows(ptr(stats), rows, ptr(logits), ptr(base), ptr(targets), r0, r1, V)
    return stats


# ------------------------------------------------------------ GGUF files

def gguf_index(path):
    """GGUFFile.__init__ (gguf.mojo:535-590) restated: (data_start, {name:
    (kind, cols, rows, offset)}), reading as the reference does (general.
    alignment honoured, every other metadata value skipped by skip_value,
    gguf.mojo:600-620)."""
    import struct

    b = open(path, "rb").read()

    def u32(pos):
        return struct.unpack_from("<I", b, pos)[0]

    def u64(pos):
        return struct.unpack_from("<Q", b, pos)[0]

    def string_at(pos):
        n = u64(pos)
        return b[pos + 8:pos + 8 + n].decode("utf-8", "replace")

    def skip_value(vtype, pos):
        if vtype in (0, 1, 7):
            return pos + 1
        if vtype in (2, 3):
            return pos + 2
        if vtype in (4, 5, 6):
            return pos + 4
        if vtype in (10, 11, 12):
            return pos + 8
        if vtype == 8:
            return pos + 8 + u64(pos)
        if vtype == 9:
            etype, count = u32(pos), u64(pos + 4)
            q = pos + 12
            for _ in range(count):
                q = skip_value(etype, q)
            return q
        raise ValueError(f"unknown GGUF metadata type {vtype}")

    if u32(0) != 0x46554747:
        raise ValueError(f"{path} is not a GGUF file")
    if u32(4) < 2:
        raise ValueError(f"GGUF version {u32(4)} is not supported")
    n_tensors, n_kv = u64(8), u64(16)
    pos, alignment = 24, 32
    for _ in range(n_kv):
        key = string_at(pos)
        pos += 8 + len(key.encode())
        vtype = u32(pos)
        pos += 4
        if key == "general.alignment":
            alignment = u32(pos)
        pos = skip_value(vtype, pos)
    tensors = {}
    for _ in range(n_tensors):
        name = string_at(pos)
        pos += 8 + len(name.encode())
        ndims = u32(pos)
        pos += 4
        cols = u64(pos)
        rows = 1
        for d in range(1, ndims):
            rows *= u64(pos + 8 * d)
        pos += 8 * ndims
        tensors[name] = (u32(pos), cols, rows, u64(pos + 4))
        pos += 12
    return (pos + alignment - 1) // alignment * alignment, tensors


# ------------------------------------------------------------ saved models
# gpt2t.mojo:612-698 in serialize.mojo's encoding (integers 8 bytes
# little-endian, strings a length and the bytes, raw buffers).

SAVED_MAGIC = b"llm_mojo GPT-2 124M weights"  # gpt2t.mojo:621
SAVED_VERSION = 1  # gpt2t.mojo:622
VEC_PARAM = [0, 1, 3, 5, 6, 7, 9, 11]  # VEC_NAMES (gpt2t.mojo:108-118) within a layer's params


def _i64(v):
    return int(v).to_bytes(8, "little", signed=True)


def _str(b):
    return _i64(len(b)) + b


def qm_name(q):
    """QuantMatrix.name (tensor.mojo:325-331)."""
    g = "ch" if q.perch else f"g{q.group}"
    return f"int{q.bits}-{g}" + ("-sym" if q.sym else "") + ("-a16" if q.a16 else "")


def qm_save_bytes(q):
    """QuantMatrix.save (tensor.mojo:634-644): rows, cols, group, codes (in
    the reference's own layout), float16 scales, zero points."""
    groups = q.n * (q.k // q.group)
    return (_i64(q.n) + _i64(q.k) + _i64(q.group) + ctypes.string_at(q.data, q.n * q.k * q.bits // 8)
            + ctypes.string_at(q.scale, 2 * groups) + ctypes.string_at(q.zp, groups))


def small_floats(params):
    """Model.small (gpt2t.mojo:249-265, 574-576): per layer the VEC_NAMES
    tensors, then wpe, ln_f.weight, ln_f.bias, as float32."""
    parts = []
    for l in range(12):
        lp = params[4 + 12 * l: 16 + 12 * l]
        parts += [np.ascontiguousarray(lp[i], np.float32).ravel() for i in VEC_PARAM]
    parts += [np.ascontiguousarray(params[i], np.float32).ravel() for i in (1, 2, 3)]
    return np.concatenate(parts)


def save_model(model, params, path):
    """save_model (gpt2t.mojo:630-650) for an oracle GPT2 built from params."""
    wte, mats = model.mat(-1), [model.mat(i) for i in range(48)]
    small = small_floats(params)
    with open(path, "wb") as f:
        f.write(_str(SAVED_MAGIC) + _i64(SAVED_VERSION) + _str(qm_name(mats[0]).encode())
                + _str(qm_name(wte).encode()))
        f.write(qm_save_bytes(wte))
        for q in mats:
            f.write(qm_save_bytes(q))
        f.write(_i64(len(small)) + small.tobytes())


def read_saved(path):
    """load_saved's reading (gpt2t.mojo:653-698): formats, the 49 matrices as
    (rows, cols, group, codes, scales, zps) and the small floats."""
    b = open(path, "rb").read()
    pos = 0

    def i64():
        nonlocal pos
        v = int.from_bytes(b[pos:pos + 8], "little", signed=True)
        pos += 8
        return v

    def raw(n):
        nonlocal pos
        if pos + n > len(b):
            raise ValueError("unexpected end of " + str(path))
        out = b[pos:pos + n]
        pos += n
        return out

    if i64() != len(SAVED_MAGIC) or raw(len(SAVED_MAGIC)) != SAVED_MAGIC:
        raise ValueError(f"{path} is not a saved llm_mojo model (see --save)")
    if i64() != SAVED_VERSION:
        raise ValueError("unsupported version")
    layers = raw(i64()).decode()
    head = raw(i64()).decode()
    bits = [8] + [int(layers[3])] * 48
    mats = []
    for bt in bits:
        rows, cols, group = i64(), i64(), i64()
        groups = rows * (cols // group)
        mats.append((rows, cols, group, np.frombuffer(raw(rows * cols * bt // 8), np.uint8),
                     np.frombuffer(raw(2 * groups), np.uint16), np.frombuffer(raw(groups), np.uint8)))
    n = i64()
    small = np.frombuffer(raw(4 * n), np.float32)
    return {"layers": layers, "head": head, "mats": mats, "small": small, "end": pos == len(b)}


class GPT2:
    """The reference GPT-2 (gpt2t.mojo Model, int4-g32-a16 layers by default,
    HEAD8_A16 head, QuantKV[8], or IntAttnKV with attention="int") on the
    CPU."""

    def __init__(self, params, bits=4, group=32, sym=False, attention="float", a16=True, head=None):
        """head: (bits, group, sym, a16) of E; None for the int8 per-channel
        head with the layers' A16 (run_quantized's --head int8)."""
        self._keep = [np.ascontiguousarray(p, np.float32) for p in params]
        arr = (ctypes.c_void_p * len(self._keep))(*[p.ctypes.data for p in self._keep])
        e = head if head is not None else (8, 0, False, a16)
        self.h = lib().orc_gpt2_new_fmt(arr, bits, group, 1 if sym else 0, 1 if a16 else 0, e[0], e[1],
                                        1 if e[2] else 0, 1 if e[3] else 0)
        self._keep = None  # the model copied what it keeps
        # --attention int (gpt2t.mojo:1251-1257): IntAttnKV
        lib().orc_gpt2_set_attention(self.h, 1 if attention == "int" else 0)

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_gpt2_free(self.h)
            self.h = None

    def set_capture(self, codes):
        """codes: int16 array of 49 * 3072 (or None): one-token forwards
        store each linear's input codes there (slot 4 l + k, 48 the head)."""
        self._capture = codes
        lib().orc_gpt2_set_capture(self.h, ptr(codes))

    def forward(self, tokens, pos0):
        toks = np.ascontiguousarray(tokens, np.int64)
        p = lib().orc_gpt2_forward(self.h, ptr(toks), len(toks), pos0)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), shape=(50257,)).copy()

    def cpu_generate(self, prompt, steps, threads):
        """The CPU baseline: the prompt through forward(), then greedy decode
        through the team decode (gpt2t.mojo:350-447) on `threads` threads
        with VPDPWSSD dots where the CPU has AVX-512 VNNI (cpu_vnni()).
        Returns (tokens, prompt seconds, decode seconds)."""
        toks = np.ascontiguousarray(prompt, np.int64)
        out = np.zeros(max(steps, 1), np.int64)
        secs = np.zeros(2, np.float64)
        n = lib().orc_cpu_generate(self.h, ptr(toks), len(toks), steps, threads, ptr(out), ptr(secs))
        if n < 0:
            raise ValueError("cpu_generate: bad arguments or no threads")
        return out[:n], float(secs[0]), float(secs[1])

    def cpu_decode(self, token, pos, threads):
        """One token at pos through the team decode: its logits."""
        p = lib().orc_cpu_decode(self.h, int(token), int(pos), int(threads))
        if not p:
            raise ValueError("cpu_decode: bad arguments or no threads")
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), shape=(50257,)).copy()

    def cpu_prompt(self, tokens, threads):
        """Model.forward of a prompt on the CPU baseline's AVX-512 VNNI forms
        over `threads` threads: (logits, seconds); logits equal forward()'s."""
        toks = np.ascontiguousarray(tokens, np.int64)
        secs = np.zeros(1, np.float64)
        p = lib().orc_cpu_prompt(self.h, ptr(toks), len(toks), int(threads), ptr(secs))
        if not p:
            raise ValueError("cpu_prompt: bad arguments")
        lg = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), shape=(50257,)).copy()
        return lg, float(secs[0])

    def cpu_head_seconds(self, threads, reps=50):
        """Median seconds of the int8 per-channel head on a team of `threads`."""
        return float(lib().orc_cpu_head_seconds(self.h, int(threads), int(reps)))

    def forward_all(self, tokens):
        """Model.forward_all (gpt2t.mojo:448-459): logits [T, V]."""
        toks = np.ascontiguousarray(tokens, np.int64)
        out = np.zeros((len(toks), 50257), np.float32)
        lib().orc_gpt2_forward_all(self.h, ptr(toks), len(toks), ptr(out))
        return out

    def generate(self, prompt, steps):
        prompt = np.ascontiguousarray(prompt, np.int64)
        out = np.zeros(steps, np.int64)
        n = lib().orc_gpt2_generate(self.h, ptr(prompt), len(prompt), steps, ptr(out))
        return out[:n]

    def mat(self, i):
        """The orc_qm of layer matrix i (l * 4 + j), or of the head for -1."""
        return ctypes.cast(lib().orc_gpt2_mat(self.h, i), ctypes.POINTER(QM)).contents

    def act(self, which, n):
        p = lib().orc_gpt2_act(self.h, which)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), shape=(n,)).copy()
