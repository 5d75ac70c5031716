"""A TinyLlama-shaped decoder over GGUF weights on libllmq.so (the
benchmark's fifth configuration: Q4_K layers, Q6_K head, int8 KV cache, grouped key / value heads,
RMSNorm, RoPE, SwiGLU).  The reference has no such model (its model code is
GPT-2 only, gpt2t.mojo:74-81); the GGUF kernels it runs on are the
reference's (gguf.mojo:344-511, kernels.mojo:285-349, 693-736).
"""
import ctypes

import numpy as np

from ._lib import GGML, LlamaCfg, check, hptr, lib

TINYLLAMA = dict(n_layer=22, dim=2048, n_head=32, n_kv=4, head_dim=64, ffn=5632, vocab=32000, max_t=1152, batch=1,
                 layer_type=GGML["Q4_K"], head_type=GGML["Q6_K"], embd_type=GGML["Q4_K"], eps=1e-5, theta=10000.0)


def tensor_names(n_layer):
    """The order llmq_llama_create takes its tensors in (GGUF tensor names)."""
    names = ["token_embd"]
    for l in range(n_layer):
        names += [f"blk.{l}.{n}" for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                                            "ffn_gate", "ffn_up", "ffn_down")]
    return names + ["output_norm", "output"]


def tensor_shapes(cfg):
    """{GGUF name suffix: (rows, cols)} of the matrices; norms are (dim,)."""
    d, kv, f, v = cfg["dim"], cfg["n_kv"] * cfg["head_dim"], cfg["ffn"], cfg["vocab"]
    return {"token_embd": (v, d), "attn_q": (d, d), "attn_k": (kv, d), "attn_v": (kv, d), "attn_output": (d, d),
            "ffn_gate": (f, d), "ffn_up": (f, d), "ffn_down": (d, f), "output": (v, d)}


class Llama:
    """The decoder on one GPU; up to cfg["batch"] independent sequences share the weights."""

    def __init__(self, ctx, cfg, tensors):
        self.ctx = ctx
        self.cfg = dict(cfg)
        self._c = LlamaCfg(**self.cfg)
        arrs = [np.ascontiguousarray(t) for t in tensors]
        if len(arrs) != len(tensor_names(cfg["n_layer"])):
            raise ValueError(f"{len(arrs)} tensors, expected {len(tensor_names(cfg['n_layer']))}")
        ptrs = (ctypes.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
        h = ctypes.c_void_p()
        check(lib().llmq_llama_create(ctx.h, ctypes.byref(self._c), ptrs, ctypes.byref(h)))
        self.h = h

    @classmethod
    def from_gguf(cls, ctx, path, cfg):
        """The decoder from a llama.cpp GGUF file (GGUFFile, gguf.mojo:519-636):
        tensors `<name>.weight` in tensor_names order, norms F32, matrices of
        the cfg's types."""
        from .formats import GGUFFile

        g = GGUFFile(path)
        shapes = tensor_shapes(cfg)
        tensors = []
        try:
            for name in tensor_names(cfg["n_layer"]):
                kind = name.rsplit(".", 1)[-1]
                full = name + ".weight"
                if kind.endswith("norm"):
                    tensors.append(g.f32(full).reshape(-1))
                    continue
                want = cfg["head_type"] if kind == "output" else (
                    cfg["embd_type"] if kind == "token_embd" else cfg["layer_type"])
                t, rows, cols, _ = g.info(full)
                if t != want or (rows, cols) != shapes[kind]:
                    raise ValueError(f"{full}: ggml type {t} {rows}x{cols}, expected type {want} {shapes[kind]}")
                tensors.append(g.tensor_bytes(full))
        finally:
            g.close()
        return cls(ctx, cfg, tensors)

    def weight_bytes(self):
        return lib().llmq_llama_weight_bytes(self.h)

    def forward(self, seq, tokens, pos0):
        """Logits of the last of `tokens` of sequence `seq` at positions pos0.."""
        tokens = np.ascontiguousarray(tokens, np.int64)
        out = np.zeros(self.cfg["vocab"], np.float32)
        check(lib().llmq_llama_forward(self.h, seq, hptr(tokens), len(tokens), pos0, hptr(out)))
        return out

    def generate(self, prompts, steps):
        """prompts [B, n], B <= cfg batch: (tokens [steps, B], prefill_ms, decode_ms)."""
        prompts = np.ascontiguousarray(prompts, np.int64)
        B, n = prompts.shape
        out = np.zeros((steps, B), np.int64)
        pm, dm = ctypes.c_double(), ctypes.c_double()
        check(lib().llmq_llama_generate(self.h, hptr(prompts), B, n, steps, hptr(out), ctypes.byref(pm),
                                        ctypes.byref(dm)))
        return out, pm.value, dm.value

    def free(self):
        if getattr(self, "h", None):
            lib().llmq_llama_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
