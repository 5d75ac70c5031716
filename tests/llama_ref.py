"""A NumPy statement of the config-4 decoder (llm_mojo_amd/llama.py), the
spec its GPU model is tested against.  The reference has no such model
(gpt2t.mojo is GPT-2 only), so this pins our own definition, not the
reference's: model-level parity is unpinned.  The parts the reference does
define come from the oracle: GGUF dequantization (gguf.mojo:178-297), the
int8 cache store (QuantKV.store, kvcache.mojo:320-342) and the int16 head
(head_i16, kernels.mojo:693-736).

Tokens are processed one at a time (causal attention by construction);
matmuls in float64, the rest in float32 as the kernels compute it.
"""
import numpy as np

import oracle
from llm_mojo_amd.llama import tensor_names, tensor_shapes

HD = 64


def round_away(x):
    return np.trunc(x + np.copysign(np.float32(0.5), x)).astype(np.float32)


class NumpyLlama:
    def __init__(self, cfg, tensors, n_seq=1):
        self.c = cfg
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

    def rmsnorm(self, x, g):
        ss = np.float32(np.sum(x.astype(np.float64) ** 2))
        r = np.float32(1.0) / np.sqrt(ss / np.float32(len(x)) + np.float32(self.c["eps"]))
        return (x * r) * g

    def rope(self, v, pos):
        i = np.arange(HD // 2, dtype=np.float32)
        freq = np.power(np.float32(self.c["theta"]), -(2 * i) / np.float32(HD)).astype(np.float32)
        ang = (np.float32(pos) * freq).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = v[:, 0::2].astype(np.float64), v[:, 1::2].astype(np.float64)
        out = np.empty_like(v)
        out[:, 0::2] = x0 * c - x1 * s
        out[:, 1::2] = x0 * s + x1 * c
        return out

    def step(self, seq, tok, pos):
        """One token at position pos: returns the final hidden row (normed)."""
        c, t = self.c, self.t
        nh, nkv = c["n_head"], c["n_kv"]
        group = nh // nkv
        kv = self.cache[seq]
        x = t["token_embd"][tok].astype(np.float32)
        for l in range(c["n_layer"]):
            p = f"blk.{l}."
            n1 = self.rmsnorm(x, t[p + "attn_norm"]).astype(np.float64)
            q = (t[p + "attn_q"] @ n1).astype(np.float32).reshape(nh, HD)
            k = (t[p + "attn_k"] @ n1).astype(np.float32).reshape(nkv, HD)
            v = (t[p + "attn_v"] @ n1).astype(np.float32).reshape(nkv, HD)
            q, k = self.rope(q, pos), self.rope(k, pos)
            kv.store(l, pos, k.reshape(-1), v.reshape(-1))
            K = kv.k.reshape(c["n_layer"], c["max_t"], nkv, HD)[l, :pos + 1].astype(np.float64)
            V = kv.v.reshape(c["n_layer"], c["max_t"], nkv, HD)[l, :pos + 1].astype(np.float64)
            KS = kv.ks.reshape(c["n_layer"], c["max_t"], nkv)[l, :pos + 1].astype(np.float64)
            VS = kv.vs.reshape(c["n_layer"], c["max_t"], nkv)[l, :pos + 1].astype(np.float64)
            att = np.zeros((nh, HD))
            for h in range(nh):
                g = h // group
                sc = (K[:, g] @ q[h].astype(np.float64)) * KS[:, g] / np.sqrt(HD)
                e = np.exp(sc - sc.max())
                pr = e / e.sum()
                att[h] = (pr * VS[:, g]) @ V[:, g]
            x = x + (t[p + "attn_output"] @ att.reshape(-1)).astype(np.float32)
            n2 = self.rmsnorm(x, t[p + "ffn_norm"]).astype(np.float64)
            gt, up = t[p + "ffn_gate"] @ n2, t[p + "ffn_up"] @ n2
            hh = gt / (1.0 + np.exp(-gt)) * up
            x = x + (t[p + "ffn_down"] @ hh).astype(np.float32)
        return self.rmsnorm(x, t["output_norm"])

    def logits(self, h):
        c = self.c
        if c["head_type"] in (8, 14):  # the int16 head (head_i16)
            return oracle.gguf_head_i16(c["head_type"], self.t["output"], c["vocab"], c["dim"], h)[0]
        w = oracle.gguf_dequant(c["head_type"], self.t["output"], c["vocab"], c["dim"]).astype(np.float64)
        return (w @ h.astype(np.float64)).astype(np.float32)

    def forward(self, seq, tokens, pos0):
        for i, tok in enumerate(tokens):
            h = self.step(seq, int(tok), pos0 + i)
        return self.logits(h)
