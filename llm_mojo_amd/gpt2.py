"""GPT-2 124M on libllmq.so: the caller of the quantized path
(gpt2t.mojo Model / load_model / generate, 198-609, 929-1009).

Layers are QuantMatrix[bits, group, sym, A16] (int4-g32-a16 by default; any
of gpt2t.mojo's quantized --dtype names), the tied embedding / head int8 per
channel (HEAD8_A16 / HEAD8) or the layers' format (--head same), the cache
QuantKV[8] or IntAttnKV, all resident on one GPU.  Greedy generation runs on
the device: each step's argmax picks the next token without a round trip to
the host.
"""
import ctypes
import os

import numpy as np

from ._lib import check, hptr, lib

N_LAYER, N_HEAD, C, HS, MAX_T, V, EOT = 12, 12, 768, 64, 1024, 50257, 50256

# gpt2t.mojo:89-118 names, in the order llmq_gpt2_create takes them
LAYER_PARAMS = [
    "ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias", "attn.c_proj.weight",
    "attn.c_proj.bias", "ln_2.weight", "ln_2.bias", "mlp.c_fc.weight", "mlp.c_fc.bias", "mlp.c_proj.weight",
    "mlp.c_proj.bias",
]
SHAPES = {
    "wte.weight": (V, C), "wpe.weight": (MAX_T, C), "ln_f.weight": (C,), "ln_f.bias": (C,),
    "ln_1.weight": (C,), "ln_1.bias": (C,), "attn.c_attn.weight": (C, 3 * C), "attn.c_attn.bias": (3 * C,),
    "attn.c_proj.weight": (C, C), "attn.c_proj.bias": (C,), "ln_2.weight": (C,), "ln_2.bias": (C,),
    "mlp.c_fc.weight": (C, 4 * C), "mlp.c_fc.bias": (4 * C,), "mlp.c_proj.weight": (4 * C, C),
    "mlp.c_proj.bias": (C,),
}


def param_names():
    names = ["wte.weight", "wpe.weight", "ln_f.weight", "ln_f.bias"]
    for l in range(N_LAYER):
        names += [f"h.{l}.{p}" for p in LAYER_PARAMS]
    return names


def param_shape(name):
    return SHAPES[name.split(".", 2)[2] if name.startswith("h.") else name]


def params_list(tensors):
    """The tensors of a {name: array} dict in param_names() order, checked."""
    out = []
    for name in param_names():
        a = np.ascontiguousarray(tensors[name], np.float32)
        if a.shape != param_shape(name):
            raise ValueError(f"{name}: shape {a.shape}, expected {param_shape(name)}")
        out.append(a)
    return out


def load_safetensors(path):
    """Hugging Face GPT-2 float32 safetensors -> {name: array} (gpt2t.mojo
    read_safetensors / tensor, with the same names)."""
    from safetensors.numpy import load_file

    return load_file(path)


ATTENTION = {"float": 0, "int": 1}  # LLMQ_ATTN_FLOAT, LLMQ_ATTN_INT


def saved_formats(path):
    """saved_formats (gpt2t.mojo:661-666): (layer format, head format) of a
    saved model file."""
    a, b = ctypes.create_string_buffer(128), ctypes.create_string_buffer(128)
    check(lib().llmq_saved_formats(os.fsencode(path), a, b, 128))
    return a.value.decode(), b.value.decode()


def quant_name(bits, group, sym, a16):
    """QuantMatrix.name (tensor.mojo:326-331)."""
    g = "ch" if group == 0 else f"g{group}"
    return f"int{bits}-{g}" + ("-sym" if sym else "") + ("-a16" if a16 else "")


def head_format(dtype, head):
    """run_quantized's E (gpt2t.mojo:1282-1292): "int8" is HEAD8_A16 for -a16
    layers and HEAD8 otherwise; "same" is the layers' format."""
    if head == "int8":
        return "int8-ch-a16" if dtype.endswith("-a16") else "int8-ch"
    if head == "same":
        return dtype
    raise ValueError(f"unknown --head {head} (int8 or same)")


class GPT2:
    """Model[W, E, KV] with W = QuantMatrix[bits, group, sym, A16] (dtype names
    it as gpt2t.mojo's --dtype does, 1307-1348; else bits / group / sym with
    A16), E chosen by head as --head does, KV = QuantKV[8] for
    attention="float" and IntAttnKV for "int" (--attention, 1251-1257)."""

    def __init__(self, ctx, tensors, bits=4, group=32, sym=False, attention="float", dtype=None, head="int8"):
        if attention not in ATTENTION:
            raise ValueError(f"unknown --attention {attention} (float or int)")
        if dtype is None:
            dtype = quant_name(bits, group, sym, True)
        head_fmt = head_format(dtype, head)
        self.ctx = ctx
        params = params_list(tensors)
        arr = (ctypes.c_void_p * len(params))(*[p.ctypes.data for p in params])
        h = ctypes.c_void_p()
        check(lib().llmq_gpt2_create_fmt(ctx.h, arr, dtype.encode(), head.encode(), ATTENTION[attention],
                                         ctypes.byref(h)))
        self.h = h
        self.attention = attention
        self._set_formats(dtype, head_fmt)

    def _set_formats(self, dtype, head_fmt):
        self.dtype, self.head_fmt = dtype, head_fmt
        self.bits = int(dtype[3])
        g = dtype.split("-")[1]
        self.group = 0 if g == "ch" else int(g[1:])
        self.sym = "-sym" in dtype
        self.a16 = dtype.endswith("-a16")

    @classmethod
    def load(cls, ctx, path, attention="float"):
        """load_saved (gpt2t.mojo:668-698): a model from a file written by
        save / the reference's --save."""
        if attention not in ATTENTION:
            raise ValueError(f"unknown --attention {attention} (float or int)")
        h = ctypes.c_void_p()
        check(lib().llmq_gpt2_load(ctx.h, os.fsencode(path), ATTENTION[attention], ctypes.byref(h)))
        self = cls.__new__(cls)
        self.ctx, self.h, self.attention = ctx, h, attention
        self._set_formats(*saved_formats(path))
        return self

    @classmethod
    def from_gguf(cls, ctx, path, attention="float"):
        """load_gguf (gpt2t.mojo:728-760): Model[GGUFMatrix, GGUFMatrix] from a
        llama.cpp GGUF file of GPT-2 124M, matrices used as stored."""
        if attention not in ATTENTION:
            raise ValueError(f"unknown --attention {attention} (float or int)")
        h = ctypes.c_void_p()
        check(lib().llmq_gpt2_load_gguf(ctx.h, os.fsencode(path), ATTENTION[attention], ctypes.byref(h)))
        self = cls.__new__(cls)
        self.ctx, self.h, self.attention = ctx, h, attention
        self.dtype = self.head_fmt = self.bits = self.group = self.sym = self.a16 = None
        return self

    def save(self, path):
        """save_model (gpt2t.mojo:630-650): the converted weights, byte for
        byte the reference's saved-model format."""
        check(lib().llmq_gpt2_save(self.h, os.fsencode(path)))

    def name(self):
        """model_name (gpt2t.mojo:1222-1228)."""
        kv = "int8-intattn" if self.attention == "int" else "int8"
        if self.dtype is None:  # GGUFMatrix layers and head (gguf.mojo:374-375)
            return "gguf+kv-" + kv
        n = self.dtype if self.head_fmt == self.dtype else self.dtype + "+head-" + self.head_fmt
        return n + "+kv-" + kv

    def weight_bytes(self):
        return lib().llmq_gpt2_weight_bytes(self.h)

    def forward(self, tokens, pos0):
        """Model.forward: the last token's logits [V] (host)."""
        toks = np.ascontiguousarray(tokens, np.int64)
        logits = np.zeros(V, np.float32)
        check(lib().llmq_gpt2_forward(self.h, hptr(toks), len(toks), pos0, hptr(logits)))
        return logits

    def debug_codes(self, codes):
        """Capture each linear's int16 input codes of later one-token
        forwards into codes (a device int16 tensor of 49 * 3072, or None to
        stop): slot 4 l + k for layer l's qkv / proj / fc / fcproj, 48 the
        head."""
        check(lib().llmq_gpt2_debug_codes(self.h, None if codes is None else codes.data_ptr()))

    def forward_all(self, tokens, logits):
        """Model.forward_all (gpt2t.mojo:448-459): logits for every position
        into logits (device address or torch tensor, [T, V] float32)."""
        toks = np.ascontiguousarray(tokens, np.int64)
        addr = logits if isinstance(logits, int) else logits.data_ptr()
        check(lib().llmq_gpt2_forward_all(self.h, hptr(toks), len(toks), addr))

    def generate(self, prompt, steps):
        """Greedy generate (-t 0): (tokens, prefill_ms, decode_ms) with the
        reference's timing spans (gpt2t.mojo:949-1005)."""
        prompt = np.ascontiguousarray(prompt, np.int64)
        out = np.zeros(max(steps, 1), np.int64)
        n = ctypes.c_int()
        pm, dm = ctypes.c_double(), ctypes.c_double()
        check(lib().llmq_gpt2_generate(self.h, hptr(prompt), len(prompt), steps, hptr(out), ctypes.byref(n),
                                       ctypes.byref(pm), ctypes.byref(dm)))
        return out[:n.value], pm.value, dm.value

    def free(self):
        if getattr(self, "h", None):
            lib().llmq_gpt2_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
