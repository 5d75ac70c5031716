"""ctypes binding of libllmq.so (include/llmq.h).

The library is loaded from this package directory only.  There is no
fallback: if libllmq.so is missing or does not load, importing the compute
API raises, so nothing can silently run on the CPU instead.
"""
import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libllmq.so")

LLMQ_BIAS, LLMQ_GELU, LLMQ_RESID = 1, 2, 4
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


class LlmqError(RuntimeError):
    pass


P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
PP = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); the exported C ABI, as declared in include/llmq.h
SIGNATURES = {
    "llmq_init": (I32, [I32, PP]),
    "llmq_destroy": (I32, [P]),
    "llmq_last_error": (ctypes.c_char_p, []),
    "llmq_set_stream": (I32, [P, P]),
    "llmq_sync": (I32, [P]),
    "llmq_malloc": (I32, [P, ctypes.c_size_t, PP]),
    "llmq_free": (I32, [P, P]),
    "llmq_memcpy_h2d": (I32, [P, P, P, ctypes.c_size_t]),
    "llmq_memcpy_d2h": (I32, [P, P, P, ctypes.c_size_t]),
    "llmq_mat_from_f32": (I32, [P, I32, I32, I32, I32, P, I64, I64, I32, PP]),
    "llmq_mat_from_f32_device": (I32, [P, I32, I32, I32, I32, P, I64, I64, I32, PP]),
    "llmq_mat_from_gguf": (I32, [P, I32, P, I64, I64, PP]),
    "llmq_mat_free": (I32, [P]),
    "llmq_mat_nbytes": (I64, [P]),
    "llmq_mat_group_size": (I64, [P]),
    "llmq_mat_has_i16": (I32, [P]),
    "llmq_mat_shape": (I32, [P, ctypes.POINTER(I64), ctypes.POINTER(I64)]),
    "llmq_mat_export": (I32, [P, P, P, P, P]),
    "llmq_mat_dequant_row": (I32, [P, P, I64, P]),
    "llmq_dot_row_i16": (I32, [P, P, I64, I64, P, P]),
    "llmq_quantize_rows": (I32, [P, P, I64, I64, P, P]),
    "llmq_linear": (I32, [P, P, P, P, P, I64, I64, I64, I32]),
    "llmq_linear_noalloc": (I32, [P, P, P, P, P, I64, I64, I64, I32]),
    "llmq_ln_linear": (I32, [P, P, P, P, P, P, P, I64, I64, I64, I32]),
    "llmq_head": (I32, [P, P, P, P, I64, I64, I64]),
    "llmq_layernorm": (I32, [P, P, P, P, P, I64, I64]),
    "llmq_debug_chunk_sums": (I32, [P, P, P, P, P, P, P]),
    "llmq_debug_refmath": (I32, [P, I32, P, P, I64]),
    "llmq_act_bytes": (I64, [I64]),
    "llmq_debug_read": (I32, [P, P, I64, P, I32]),
    "llmq_act_prepare": (I32, [P, P, I64, P, P, P]),
    "llmq_linear_act": (I32, [P, P, P, P, P, I64, I64, I32]),
    "llmq_gpt2_debug_codes": (I32, [P, P]),
    "llmq_kv_create": (I32, [P, I32, I32, I32, I32, PP]),
    "llmq_kv_free": (I32, [P]),
    "llmq_kv_nbytes": (I64, [P]),
    "llmq_kv_store": (I32, [P, P, I32, I32, P, I32]),
    "llmq_kv_attend": (I32, [P, P, P, P, I32, I32, I32]),
    "llmq_kv_export": (I32, [P, P, P, P, P, P]),
    "llmq_ikv_create": (I32, [P, I32, I32, I32, I32, PP]),
    "llmq_kv_is_integer": (I32, [P]),
    "llmq_ikv_export": (I32, [P, P, P, P, P, P]),
    "llmq_gpt2_create": (I32, [P, P, I32, I32, I32, PP]),
    "llmq_gpt2_create_ex": (I32, [P, P, I32, I32, I32, I32, PP]),
    "llmq_gpt2_create_fmt": (I32, [P, P, ctypes.c_char_p, ctypes.c_char_p, I32, PP]),
    "llmq_gguf_open": (I32, [ctypes.c_char_p, PP]),
    "llmq_gguf_close": (I32, [P]),
    "llmq_gguf_n_tensors": (I64, [P]),
    "llmq_gguf_find": (I32, [P, ctypes.c_char_p, ctypes.POINTER(I64)]),
    "llmq_gguf_tensor_info": (I32, [P, I64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(I32),
                                    ctypes.POINTER(I64), ctypes.POINTER(I64), ctypes.POINTER(I64)]),
    "llmq_gguf_tensor_data": (I32, [P, I64, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(I64)]),
    "llmq_gguf_matrix": (I32, [P, P, ctypes.c_char_p, PP]),
    "llmq_gpt2_save": (I32, [P, ctypes.c_char_p]),
    "llmq_gpt2_forward_all": (I32, [P, P, I32, P]),
    "llmq_score_rows": (I32, [P, P, P, P, I32, I32, I32, P, I64]),
    "llmq_gpt2_load_gguf": (I32, [P, ctypes.c_char_p, I32, PP]),
    "llmq_gpt2_load": (I32, [P, ctypes.c_char_p, I32, PP]),
    "llmq_saved_formats": (I32, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, I32]),
    "llmq_mat_restore": (I32, [P, I32, I32, I32, I32, I64, I64, P, P, P, PP]),
    "llmq_gpt2_free": (I32, [P]),
    "llmq_gpt2_weight_bytes": (I64, [P]),
    "llmq_gpt2_forward": (I32, [P, P, I32, I32, P]),
    "llmq_gpt2_generate": (I32, [P, P, I32, I32, P, ctypes.POINTER(I32), ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(ctypes.c_double)]),
    "llmq_gpt2_logits_device": (I32, [P, ctypes.POINTER(ctypes.c_void_p)]),
    "llmq_llama_create": (I32, [P, P, P, PP]),
    "llmq_llama_free": (I32, [P]),
    "llmq_llama_weight_bytes": (I64, [P]),
    "llmq_llama_forward": (I32, [P, I32, P, I32, I32, P]),
    "llmq_llama_generate": (I32, [P, P, I32, I32, I32, P, ctypes.POINTER(ctypes.c_double),
                                  ctypes.POINTER(ctypes.c_double)]),
}


class LlamaCfg(ctypes.Structure):
    """llmq_llama_cfg (include/llmq.h)."""
    _fields_ = [(n, ctypes.c_int) for n in ("n_layer", "dim", "n_head", "n_kv", "head_dim", "ffn", "vocab", "max_t",
                                            "batch", "layer_type", "head_type", "embd_type")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float)]

_lib = None


def lib():
    """The loaded libllmq.so; raises LlmqError if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LlmqError(f"{LIB_PATH} is not built (python -m llm_mojo_amd.build); "
                            "llm_mojo_amd has no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        msg = lib().llmq_last_error()
        raise LlmqError(f"llmq error {rc}: {msg.decode() if msg else ''}")
    return rc


def dptr(t):
    """Device address of a torch tensor (or an int address)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def hptr(a):
    """Host address of a numpy array."""
    return None if a is None else a.ctypes.data


class DeviceBuffer:
    """nbytes of device memory from llmq_malloc (freed with the object)."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        p = ctypes.c_void_p()
        check(lib().llmq_malloc(ctx.h, nbytes, ctypes.byref(p)))
        self.ptr, self.nbytes = p.value, nbytes

    def upload(self, a):
        check(lib().llmq_memcpy_h2d(self.ctx.h, self.ptr, hptr(a), a.nbytes))

    def download(self, a):
        check(lib().llmq_memcpy_d2h(self.ctx.h, hptr(a), self.ptr, a.nbytes))
        return a

    def free(self):
        if getattr(self, "ptr", None):
            lib().llmq_free(self.ctx.h, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One GPU and the stream the library's work is ordered on."""

    def __init__(self, device=0, stream=None):
        h = ctypes.c_void_p()
        check(lib().llmq_init(device, ctypes.byref(h)))
        self.h = h
        if stream is not None:
            self.set_stream(stream)

    def set_stream(self, stream):
        """stream: a torch.cuda.Stream, a raw hipStream_t address, or None."""
        s = getattr(stream, "cuda_stream", stream)
        check(lib().llmq_set_stream(self.h, s))

    def sync(self):
        check(lib().llmq_sync(self.h))

    def close(self):
        if getattr(self, "h", None):
            lib().llmq_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
