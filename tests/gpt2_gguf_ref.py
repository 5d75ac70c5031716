"""load_gguf's model (gpt2t.mojo:728-760, Model[GGUFMatrix, GGUFMatrix])
stated on the CPU from the oracle's parts: GGUF row dequantization for the
embedding (gguf.mojo:381-382), the float GGUF GEMV per token with bias,
GELU and residual (GGUFMatrix.dot_row + finish, kernels.mojo:285-312), the
oracle's LayerNorm and int8 cache attention, and head_i16 for a Q6_K / Q8_0
head (kernels.mojo:693-736).  Also writes synthetic GPT-2 GGUF files with
tests/gguf_write.py.
"""
import numpy as np

import oracle
from tests import gguf_write as gw

NL, NH, HS, C, V, MAXT = 12, 12, 64, 768, 50257, 1024
MATS = ["attn_qkv", "attn_output", "ffn_up", "ffn_down"]
MAT_SHAPES = {"attn_qkv": (3 * C, C), "attn_output": (C, C), "ffn_up": (4 * C, C), "ffn_down": (C, 4 * C)}
VECS = [("attn_norm.weight", C), ("attn_norm.bias", C), ("attn_qkv.bias", 3 * C), ("attn_output.bias", C),
        ("ffn_norm.weight", C), ("ffn_norm.bias", C), ("ffn_up.bias", 4 * C), ("ffn_down.bias", C)]
BIAS, GELU, RESID = 1, 2, 4
SCALE = {2: 4e-3, 3: 4e-3, 8: 3e-4, 12: 1e-4, 13: 1e-4, 14: 2e-5}  # float16 d -> weights of size ~0.02


def write_gpt2_gguf(path, seed, layer_type, embd_type, head_type=None):
    """A GPT-2 124M GGUF file with seeded random blocks; head_type None
    ties the head to token_embd.  Returns {name: (type, rows, cols, data)}."""
    from llm_mojo_amd import synth

    rng = np.random.default_rng(seed)
    t = {}

    def mat(name, kind, rows, cols, s):
        t[name] = (kind, rows, cols, synth.gguf_blocks(kind, rows, cols, s, scale=SCALE[kind]))

    mat("token_embd.weight", embd_type, V, C, seed * 1000)
    if head_type is not None:
        mat("output.weight", head_type, V, C, seed * 1000 + 1)
    for l in range(NL):
        for j, m in enumerate(MATS):
            mat(f"blk.{l}.{m}.weight", layer_type, *MAT_SHAPES[m], seed * 1000 + 10 + 4 * l + j)
        for name, n in VECS:
            v = np.ones(n, np.float32) if name.endswith("norm.weight") else rng.normal(0, 0.02, n).astype(np.float32)
            t[f"blk.{l}.{name}"] = (0, 1, n, v)
    t["position_embd.weight"] = (0, MAXT, C, rng.normal(0, 0.01, (MAXT, C)).astype(np.float32))
    t["output_norm.weight"] = (0, 1, C, np.ones(C, np.float32))
    t["output_norm.bias"] = (0, 1, C, np.zeros(C, np.float32))
    entries = []
    for name, (kind, rows, cols, data) in t.items():
        dims = [cols] if rows == 1 else [cols, rows]
        raw = gw.f32_bytes(data) if kind == 0 else np.asarray(data, np.uint8).tobytes()
        entries.append((name, kind, dims, raw))
    gw.write(path, entries, [("general.architecture", gw.STRING, "gpt2")])
    return t


class GGUFGPT2Ref:
    def __init__(self, t, attention="float"):
        self.t = t
        kv = oracle.IntAttnKV if attention == "int" else oracle.QuantKV8
        self.kv = kv(NL, MAXT, NH, HS)
        self.lm = t.get("output.weight", t["token_embd.weight"])

    def f32(self, name):
        return np.asarray(self.t[name][3], np.float32)

    def linear(self, name, x, b, flags, resid=None):
        kind, rows, cols, data = self.t[name]
        out = [oracle.gguf_gemv(kind, data, rows, cols, x[i], b, flags,
                                out=None if resid is None else resid[i].copy()) for i in range(len(x))]
        return np.stack(out)

    def forward(self, tokens, pos0):
        """Model.forward: the last token's logits."""
        kind, rows, cols, data = self.t["token_embd.weight"]
        rb = cols // oracle.gguf_block_size(kind) * oracle.gguf_block_bytes(kind)
        T = len(tokens)
        x = np.stack([oracle.gguf_dequant(kind, data[int(tok) * rb:(int(tok) + 1) * rb], 1, cols)[0]
                      for tok in tokens])
        x = (x + self.f32("position_embd.weight")[pos0:pos0 + T]).astype(np.float32)
        for l in range(NL):
            p = f"blk.{l}."
            xn = oracle.layernorm(x, self.f32(p + "attn_norm.weight"), self.f32(p + "attn_norm.bias"))
            qkv = self.linear(p + "attn_qkv.weight", xn, self.f32(p + "attn_qkv.bias"), BIAS)
            for i in range(T):
                self.kv.store(l, pos0 + i, qkv[i, C:2 * C], qkv[i, 2 * C:])
            att = self.kv.attend(qkv, l, T, pos0)
            x = self.linear(p + "attn_output.weight", att, self.f32(p + "attn_output.bias"), BIAS | RESID, x)
            xn = oracle.layernorm(x, self.f32(p + "ffn_norm.weight"), self.f32(p + "ffn_norm.bias"))
            fc = self.linear(p + "ffn_up.weight", xn, self.f32(p + "ffn_up.bias"), BIAS | GELU)
            x = self.linear(p + "ffn_down.weight", fc, self.f32(p + "ffn_down.bias"), BIAS | RESID, x)
        h = oracle.layernorm(x[-1:], self.f32("output_norm.weight"), self.f32("output_norm.bias"))
        kind, rows, cols, data = self.lm
        if kind in (8, 14):
            return oracle.gguf_head_i16(kind, data, V, C, h)[0]
        return oracle.gguf_gemv(kind, data, V, C, h[0])
