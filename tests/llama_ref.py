"""A NumPy statement of the config-4 decoder (llm_mojo_amd/llama.py), the
spec its GPU model is tested against.  The reference has no such model
(gpt2t.mojo is GPT-2 only), so this pins our own definition, not the
reference's: model-level parity is unpinned.  The parts the reference does
define come from the oracle: GGUF dequantization (gguf.mojo:178-297), the
int8 cache store (QuantKV.store, kvcache.mojo:320-342) and the int16 head
(head_i16, kernels.mojo:693-736).

Tokens go through in blocks (a prompt at once: every operation is per row
except attention, which masks positions after each query, so a block gives
what one token at a time gives); matmuls in float64, the rest in float32 as
the kernels compute it.
"""
import os

import numpy as np

import oracle
from llm_mojo_amd.llama import tensor_names, tensor_shapes

HD = 64


def round_away(x):
    return np.trunc(x + np.copysign(np.float32(0.5), x)).astype(np.float32)


class NumpyLlama:
    def __init__(self, cfg, tensors, n_seq=1):
        self.c = cfg
        oracle.set_threads(min(16, os.cpu_count() or 1))  # (results do not depend on it)
        shapes = tensor_shapes(cfg)
        self.t = {}
        for name, a in zip(tensor_names(cfg["n_layer"]), tensors):
            kind = name.rsplit(".", 1)[-1]
            if kind.endswith("norm"):
                self.t[name] = np.asarray(a, np.float32)
            elif kind == "output":
                self.t[name] = a  # blocks: the int16 head reads them
            else:
                ty = cfg["embd_type"] if kind == "token_embd" else cfg["layer_type"]
                rows, cols = shapes[kind]
                self.t[name] = oracle.gguf_dequant(ty, a, rows, cols).astype(np.float64)
        self.cache = [oracle.QuantKV8(cfg["n_layer"], cfg["max_t"], cfg["n_kv"], HD) for _ in range(n_seq)]
        self.causal = True  # (tests plant a missing mask by clearing it)

    def rmsnorm(self, x, g):
        """Rows of x (float32) normalized by their own root mean square."""
        x = np.atleast_2d(x)
        ss = np.sum(x.astype(np.float64) ** 2, axis=1).astype(np.float32)
        r = np.float32(1.0) / np.sqrt(ss / np.float32(x.shape[1]) + np.float32(self.c["eps"]))
        return (x * r[:, None]) * g

    def rope(self, v, pos):
        """v[T, heads, HD] at positions pos[T]: adjacent pairs rotated."""
        i = np.arange(HD // 2, dtype=np.float32)
        freq = np.power(np.float32(self.c["theta"]), -(2 * i) / np.float32(HD)).astype(np.float32)
        ang = (np.asarray(pos, np.float32)[:, None] * freq[None, :]).astype(np.float64)[:, None, :]
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = v[..., 0::2].astype(np.float64), v[..., 1::2].astype(np.float64)
        out = np.empty_like(v)
        out[..., 0::2] = x0 * c - x1 * s
        out[..., 1::2] = x0 * s + x1 * c
        return out

    def block(self, seq, toks, pos0):
        """Tokens toks at positions pos0 ..: the final hidden rows (normed)."""
        c, t = self.c, self.t
        nh, nkv, L, MT = c["n_head"], c["n_kv"], c["n_layer"], c["max_t"]
        group = nh // nkv
        kv = self.cache[seq]
        T = len(toks)
        pos = np.arange(pos0, pos0 + T)
        x = t["token_embd"][np.asarray(toks, np.int64)].astype(np.float32)
        for l in range(L):
            p = f"blk.{l}."
            n1 = self.rmsnorm(x, t[p + "attn_norm"]).astype(np.float64)
            q = (n1 @ t[p + "attn_q"].T).astype(np.float32).reshape(T, nh, HD)
            k = (n1 @ t[p + "attn_k"].T).astype(np.float32).reshape(T, nkv, HD)
            v = (n1 @ t[p + "attn_v"].T).astype(np.float32).reshape(T, nkv, HD)
            q, k = self.rope(q, pos), self.rope(k, pos)
            for i in range(T):
                kv.store(l, pos0 + i, k[i].reshape(-1), v[i].reshape(-1))
            n = pos0 + T
            K = kv.k.reshape(L, MT, nkv, HD)[l, :n].astype(np.float64)
            V = kv.v.reshape(L, MT, nkv, HD)[l, :n].astype(np.float64)
            KS = kv.ks.reshape(L, MT, nkv)[l, :n].astype(np.float64)
            VS = kv.vs.reshape(L, MT, nkv)[l, :n].astype(np.float64)
            masked = np.arange(n)[None, :] > pos[:, None]  # [T, n]: key after the query
            if not self.causal:
                masked[:] = np.arange(n)[None, :] >= n
            att = np.zeros((T, nh, HD))
            for h in range(nh):
                g = h // group
                sc = (q[:, h].astype(np.float64) @ K[:, g].T) * KS[None, :, g] / np.sqrt(HD)
                sc[masked] = -np.inf
                e = np.exp(sc - sc.max(axis=1, keepdims=True))
                pr = e / e.sum(axis=1, keepdims=True)
                att[:, h] = (pr * VS[None, :, g]) @ V[:, g]
            x = x + (att.reshape(T, -1) @ t[p + "attn_output"].T).astype(np.float32)
            n2 = self.rmsnorm(x, t[p + "ffn_norm"]).astype(np.float64)
            gt, up = n2 @ t[p + "ffn_gate"].T, n2 @ t[p + "ffn_up"].T
            hh = gt / (1.0 + np.exp(-gt)) * up
            x = x + (hh @ t[p + "ffn_down"].T).astype(np.float32)
        return self.rmsnorm(x, t["output_norm"])

    def step(self, seq, tok, pos):
        """One token at position pos: returns the final hidden row (normed)."""
        return self.block(seq, [tok], pos)[0]

    def logits(self, h):
        c = self.c
        if c["head_type"] in (8, 14):  # the int16 head (head_i16)
            return oracle.gguf_head_i16(c["head_type"], self.t["output"], c["vocab"], c["dim"], h)[0]
        w = oracle.gguf_dequant(c["head_type"], self.t["output"], c["vocab"], c["dim"]).astype(np.float64)
        return (w @ h.astype(np.float64)).astype(np.float32)

    def forward(self, seq, tokens, pos0):
        """Logits of the last of tokens (at positions pos0 ..)."""
        return self.logits(self.block(seq, tokens, pos0)[-1])
