"""Host-side mirror of llm_mojo's format traits over libllmq.so.

HipQuantMatrix mirrors QuantMatrix[BITS, GROUP, SYMMETRIC, A16] through the
WeightMatrix trait (tensor.mojo:49-147, 230-661); QuantKV8 mirrors
QuantKV[8] through KVCache (kvcache.mojo:31-87, 248-385).  The kernels are
driven per whole matmul (kernels.linear / head), not per row, and work on
device buffers (torch tensors or raw addresses).
"""
import ctypes
import os

import numpy as np

from ._lib import LLMQ_BIAS, LLMQ_GELU, LLMQ_RESID, check, dptr, hptr, lib


class HipQuantMatrix:
    """A QuantMatrix held on the GPU (values are handles: free() once)."""

    OUT_MAJOR = True
    FROM_GGUF = False

    def __init__(self, ctx, handle, bits, group, sym, a16):
        self.ctx, self.h = ctx, handle
        self.bits, self.group_param, self.sym, self.a16 = bits, group, sym, a16
        rows, cols = ctypes.c_int64(), ctypes.c_int64()
        check(lib().llmq_mat_shape(self.h, ctypes.byref(rows), ctypes.byref(cols)))
        self.rows, self.cols = rows.value, cols.value

    @property
    def ACT16(self):
        return self.a16

    def name(self):
        """QuantMatrix.name (tensor.mojo:325-331)."""
        g = "ch" if self.group_param == 0 else f"g{self.group_param}"
        s = f"int{self.bits}-{g}" + ("-sym" if self.sym else "")
        return s + "-a16" if self.a16 else s

    @classmethod
    def from_f32(cls, ctx, src, bits, group, sym=False, a16=True, reduce_rows=True):
        """QuantMatrix.from_f32 (tensor.mojo:334-383), quantized on the GPU.
        src: a float32 [rows, cols] numpy array (host) or torch tensor (device)."""
        h = ctypes.c_void_p()
        if isinstance(src, np.ndarray):
            src = np.ascontiguousarray(src, np.float32)
            rows, cols = src.shape
            check(lib().llmq_mat_from_f32(ctx.h, bits, group, 1 if sym else 0, 1 if a16 else 0, hptr(src), rows,
                                          cols, 1 if reduce_rows else 0, ctypes.byref(h)))
        else:
            rows, cols = src.shape
            check(lib().llmq_mat_from_f32_device(ctx.h, bits, group, 1 if sym else 0, 1 if a16 else 0, dptr(src),
                                                 rows, cols, 1 if reduce_rows else 0, ctypes.byref(h)))
        return cls(ctx, h, bits, group, sym, a16)

    def nbytes(self):
        return lib().llmq_mat_nbytes(self.h)

    def group_size(self):
        return lib().llmq_mat_group_size(self.h)

    @classmethod
    def restore(cls, ctx, bits, group, sym, a16, rows, cols, codes, scales, zps):
        """QuantMatrix.restore (tensor.mojo:646-656): from codes in the
        reference's own layout (BLOCKED for int4-g32-a16), float16 scale bits
        and zero points, as export() returns them."""
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.uint16)
        zps = np.ascontiguousarray(zps, np.uint8)
        g = cols if group == 0 else group
        if codes.size != rows * cols * bits // 8 or scales.size != rows * cols // g or zps.size != scales.size:
            raise ValueError("restore: buffer sizes do not match the shape")
        h = ctypes.c_void_p()
        check(lib().llmq_mat_restore(ctx.h, bits, group, 1 if sym else 0, 1 if a16 else 0, rows, cols, hptr(codes),
                                     hptr(scales), hptr(zps), ctypes.byref(h)))
        return cls(ctx, h, bits, group, sym, a16)

    def has_i16(self):
        """tensor.mojo:102-104: the A16 formats."""
        return bool(lib().llmq_mat_has_i16(self.h))

    def export(self):
        """(codes, float16 scale bits, zero points) in the reference's own
        QuantMatrix layout (BLOCKED for int4-g32-a16)."""
        n, k = self.rows, self.cols
        g = self.group_size()
        codes = np.zeros(n * k * self.bits // 8, np.uint8)
        scales = np.zeros(n * k // g, np.uint16)
        zps = np.zeros(n * k // g, np.uint8)
        check(lib().llmq_mat_export(self.ctx.h, self.h, hptr(codes), hptr(scales), hptr(zps)))
        return codes, scales, zps

    def dequant_row(self, row):
        dst = np.zeros(self.cols, np.float32)
        check(lib().llmq_mat_dequant_row(self.ctx.h, self.h, row, hptr(dst)))
        return dst

    def dot_row_i16(self, row, xq, out, nrows=1):
        """dot_row_i16 (tensor.mojo:518-577) of rows row .. row + nrows - 1
        with int16 codes xq (device, natural column order) into out (device
        floats), in weight scale; stream-ordered."""
        check(lib().llmq_dot_row_i16(self.ctx.h, self.h, row, nrows, dptr(xq), dptr(out)))

    def free(self):
        if getattr(self, "h", None):
            lib().llmq_mat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HipGGUFMatrix:
    """A GGUF tensor on the GPU: GGUFMatrix (gguf.mojo:344-511), blocks used
    as stored (re-placed into the device row-tile layout)."""

    OUT_MAJOR = True
    FROM_GGUF = True
    ACT16 = False

    def __init__(self, ctx, handle, kind):
        self.ctx, self.h, self.kind = ctx, handle, kind
        rows, cols = ctypes.c_int64(), ctypes.c_int64()
        check(lib().llmq_mat_shape(self.h, ctypes.byref(rows), ctypes.byref(cols)))
        self.rows, self.cols = rows.value, cols.value

    @staticmethod
    def name():
        return "gguf"

    @classmethod
    def from_blocks(cls, ctx, kind, blocks, rows, cols):
        """blocks: uint8 [rows * row_bytes] as in a GGUF file; kind: ggml type id."""
        blocks = np.ascontiguousarray(blocks, np.uint8)
        h = ctypes.c_void_p()
        check(lib().llmq_mat_from_gguf(ctx.h, kind, hptr(blocks), rows, cols, ctypes.byref(h)))
        return cls(ctx, h, kind)

    def nbytes(self):
        return lib().llmq_mat_nbytes(self.h)

    def group_size(self):
        return lib().llmq_mat_group_size(self.h)

    def has_i16(self):
        """gguf.mojo:456-457: Q6_K and Q8_0 heads take the int16 path."""
        return bool(lib().llmq_mat_has_i16(self.h))

    def dequant_row(self, row):
        dst = np.zeros(self.cols, np.float32)
        check(lib().llmq_mat_dequant_row(self.ctx.h, self.h, row, hptr(dst)))
        return dst

    def free(self):
        if getattr(self, "h", None):
            lib().llmq_mat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def quantize_rows(ctx, x, xq, sx):
    """kernels.quantize_rows (kernels.mojo:400-416) on device tensors."""
    T, K = x.shape
    check(lib().llmq_quantize_rows(ctx.h, dptr(x), T, K, dptr(xq), dptr(sx)))


def linear(ctx, out, x, w, bias=None, resid=False, gelu=False, ln=None):
    """kernels.linear (kernels.mojo:655-673): out (+)= act(x @ w^T + bias);
    ln=(weight, bias) applies LayerNorm to the input rows first."""
    T, IN = x.shape
    flags = (LLMQ_BIAS if bias is not None else 0) | (LLMQ_GELU if gelu else 0) | (LLMQ_RESID if resid else 0)
    if ln is None:
        check(lib().llmq_linear(ctx.h, dptr(out), dptr(x), w.h, dptr(bias), T, IN, w.rows, flags))
    else:
        check(lib().llmq_ln_linear(ctx.h, dptr(out), dptr(x), dptr(ln[0]), dptr(ln[1]), w.h, dptr(bias), T, IN,
                                   w.rows, flags))


def head(ctx, logits, h, w):
    """kernels.head (kernels.mojo:676-690): logits[T, V] = h @ w^T."""
    T, C = h.shape
    check(lib().llmq_head(ctx.h, dptr(logits), dptr(h), w.h, T, w.rows, C))


def layernorm(ctx, out, x, w, b):
    T, C = x.shape
    check(lib().llmq_layernorm(ctx.h, dptr(out), dptr(x), dptr(w), dptr(b), T, C))


def debug_chunk_sums(ctx, x, w, out, chunk_sums, xq, sx):
    check(lib().llmq_debug_chunk_sums(ctx.h, dptr(x), w.h, dptr(out), dptr(chunk_sums), dptr(xq), dptr(sx)))


def act_bytes(K):
    """Bytes of a prepared activation record for a K-long row."""
    return int(lib().llmq_act_bytes(K))


def act_prepare(ctx, x, act, ln=None):
    """linear_team's prepared activations of one token's row x ([1, K] or
    [K] on the device; LayerNorm with ln=(weight, bias) first) into act (a
    device uint8 tensor of act_bytes(K))."""
    K = x.shape[-1]
    check(lib().llmq_act_prepare(ctx.h, dptr(x), K, dptr(ln[0]) if ln else None, dptr(ln[1]) if ln else None,
                                 dptr(act)))


def linear_act(ctx, out, act, w, bias=None, resid=False, gelu=False):
    """One token's linear over a prepared record (bit-identical to linear)."""
    flags = (LLMQ_BIAS if bias is not None else 0) | (LLMQ_GELU if gelu else 0) | (LLMQ_RESID if resid else 0)
    check(lib().llmq_linear_act(ctx.h, dptr(out), dptr(act), w.h, dptr(bias), w.cols, w.rows, flags))


def debug_read(ctx, buf, out, grid):
    """Pure read of a device tensor buf (the read floor): one XOR per
    workgroup into out (uint32 / int32 tensor of grid entries)."""
    check(lib().llmq_debug_read(ctx.h, dptr(buf), buf.numel() * buf.element_size(), dptr(out), grid))


REFMATH_OPS = {"exp": 0, "tanh": 1, "gelu": 2}


def debug_refmath(ctx, op, x, y):
    """The kernels' exp / tanh / GELU over device floats x into y."""
    check(lib().llmq_debug_refmath(ctx.h, REFMATH_OPS[op], dptr(x), dptr(y), x.numel()))


class GGUFFile:
    """GGUFFile (gguf.mojo:527-636): a GGUF v2 / v3 file's tensor index over
    a read-only mapping of the file (libllmq's parser, bounds-checked)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib().llmq_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.h = h
        self.path = path

    def _index(self, name):
        i = ctypes.c_int64()
        check(lib().llmq_gguf_find(self.h, name.encode(), ctypes.byref(i)))
        return i.value

    def has(self, name):
        """GGUFFile.has (gguf.mojo:635-636)."""
        return self._index(name) >= 0

    def names(self):
        return [self.info_at(i)[0] for i in range(lib().llmq_gguf_n_tensors(self.h))]

    def info_at(self, i):
        nm, t = ctypes.c_char_p(), ctypes.c_int()
        rows, cols, off = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        check(lib().llmq_gguf_tensor_info(self.h, i, ctypes.byref(nm), ctypes.byref(t), ctypes.byref(rows),
                                          ctypes.byref(cols), ctypes.byref(off)))
        return nm.value.decode(), t.value, rows.value, cols.value, off.value

    def info(self, name):
        """(ggml type, rows, cols, offset) of a tensor (TensorInfo, gguf.mojo:519-524)."""
        i = self._index(name)
        if i < 0:
            raise KeyError("tensor not in GGUF file: " + name)
        return self.info_at(i)[1:]

    def tensor_bytes(self, name):
        """A copy of the tensor's bytes as stored."""
        i = self._index(name)
        if i < 0:
            raise KeyError("tensor not in GGUF file: " + name)
        p, n = ctypes.c_void_p(), ctypes.c_int64()
        check(lib().llmq_gguf_tensor_data(self.h, i, ctypes.byref(p), ctypes.byref(n)))
        return np.frombuffer(ctypes.string_at(p, n.value), np.uint8).copy()

    def f32(self, name):
        """An F32 tensor as float32 [rows, cols] (gguf_f32, gpt2t.mojo:721-726)."""
        t, rows, cols, _ = self.info(name)
        if t != 0:
            raise ValueError(f"{name} is ggml type {t}, expected F32")
        return self.tensor_bytes(name).view(np.float32).reshape(rows, cols)

    def matrix(self, ctx, name):
        """GGUFFile.matrix (gguf.mojo:622-633) on the device."""
        h = ctypes.c_void_p()
        check(lib().llmq_gguf_matrix(ctx.h, self.h, name.encode(), ctypes.byref(h)))
        return HipGGUFMatrix(ctx, h, self.info(name)[0])

    def close(self):
        if getattr(self, "h", None):
            lib().llmq_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QuantKV8:
    """QuantKV[8] (kvcache.mojo:248-385) on the GPU."""

    _create = "llmq_kv_create"

    def __init__(self, ctx, n_layer, max_t, n_head, head_dim):
        self.ctx = ctx
        self.n_layer, self.max_t, self.n_head, self.head_dim = n_layer, max_t, n_head, head_dim
        h = ctypes.c_void_p()
        check(getattr(lib(), self._create)(ctx.h, n_layer, max_t, n_head, head_dim, ctypes.byref(h)))
        self.h = h

    @staticmethod
    def name():
        return "int8"

    def nbytes(self):
        return lib().llmq_kv_nbytes(self.h)

    def store(self, layer, pos0, qkv):
        """QuantKV.store for every row of qkv [T, 3C] at positions pos0.."""
        check(lib().llmq_kv_store(self.ctx.h, self.h, layer, pos0, dptr(qkv), qkv.shape[0]))

    def attend(self, out, qkv, layer, pos0):
        check(lib().llmq_kv_attend(self.ctx.h, self.h, dptr(out), dptr(qkv), layer, qkv.shape[0], pos0))

    def export(self):
        n = self.n_layer * self.max_t * self.n_head
        k = np.zeros(n * self.head_dim, np.int8)
        v = np.zeros(n * self.head_dim, np.int8)
        ks = np.zeros(n, np.float32)
        vs = np.zeros(n, np.float32)
        check(lib().llmq_kv_export(self.ctx.h, self.h, hptr(k), hptr(v), hptr(ks), hptr(vs)))
        return k, v, ks, vs

    def free(self):
        if getattr(self, "h", None):
            lib().llmq_kv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class IntAttnKV(QuantKV8):
    """IntAttnKV (int_attention.mojo:62-269) on the GPU: the int8 cache with
    int32 scales (scale * 2^24) and attention computed in integers.  store,
    attend, nbytes and free as for QuantKV8; export returns (k, v, kq, vq)."""

    _create = "llmq_ikv_create"

    @staticmethod
    def name():
        return "int8-intattn"  # int_attention.mojo:94-96

    def export(self):
        n = self.n_layer * self.max_t * self.n_head
        k = np.zeros(n * self.head_dim, np.int8)
        v = np.zeros(n * self.head_dim, np.int8)
        kq = np.zeros(n, np.int32)
        vq = np.zeros(n, np.int32)
        check(lib().llmq_ikv_export(self.ctx.h, self.h, hptr(k), hptr(v), hptr(kq), hptr(vq)))
        return k, v, kq, vq
