"""Seeded synthetic inputs of the benchmark configurations (no network, no
real checkpoints): GPT-2 124M random-init weights written as a Hugging Face
layout safetensors file, and random prompt ids.

Normals come from SplitMix64 (the published 64-bit mixer of Steele, Lea and
Flood) through Box-Muller in float64, cast to float32; one stream per tensor,
seeded by (seed, tensor index), so any tensor can be regenerated alone.
Prompt ids use llm_mojo's own Rng (xorshift64*, gpt2t.mojo:777-789) as
floor(uniform * 50257).
"""
import os

import numpy as np

from .gpt2 import C, MAX_T, V, param_names, param_shape

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(seed, n, start=0):
    """n outputs of SplitMix64 seeded with `seed`, from position `start`."""
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def normal(seed, n, std=1.0):
    """n float32 samples of N(0, std^2) (Box-Muller on pairs of uniforms
    from the top 53 bits)."""
    m = (n + 1) // 2
    out = np.empty(2 * m, np.float32)
    step = 1 << 22
    for s in range(0, m, step):
        k = min(step, m - s)
        z = splitmix64(seed, 2 * k, 2 * s)
        u = (z >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
        u1 = 1.0 - u[0::2]  # (0, 1]
        u2 = u[1::2]
        r = np.sqrt(-2.0 * np.log(u1)) * std
        out[2 * s:2 * (s + k):2] = (r * np.cos(2 * np.pi * u2)).astype(np.float32)
        out[2 * s + 1:2 * (s + k):2] = (r * np.sin(2 * np.pi * u2)).astype(np.float32)
    return out[:n]


def gpt2_tensors(seed=1337, std=0.02):
    """{name: float32 array}: weights N(0, std), biases 0, LayerNorm gain 1."""
    out = {}
    for i, name in enumerate(param_names()):
        shape = param_shape(name)
        if name.endswith(".bias"):
            out[name] = np.zeros(shape, np.float32)
        elif name.startswith("ln") or ".ln_" in name:
            out[name] = np.ones(shape, np.float32)
        else:
            out[name] = normal(seed * 1000003 + i, int(np.prod(shape)), std).reshape(shape)
    return out


def gpt2_safetensors(path, seed=1337):
    """Writes (once) and returns the path of the synthetic checkpoint."""
    if not os.path.exists(path):
        from safetensors.numpy import save_file

        tmp = path + ".tmp"
        save_file(gpt2_tensors(seed), tmp)
        os.replace(tmp, path)
    return path


class Rng:
    """gpt2t.mojo Rng (777-789): xorshift64*, uniform floats in [0, 1)."""

    def __init__(self, seed):
        self.state = (seed * 0x9E3779B97F4A7C15 + 1) & 0xFFFFFFFFFFFFFFFF

    def uniform(self):
        s = self.state
        s ^= s >> 12
        s ^= (s << 25) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 27
        self.state = s
        r = ((s * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) >> 40
        return np.float32(r) / np.float32(1 << 24)


GGUF_BLOCK = {  # ggml type id: (weights per block, bytes per block), gguf.mojo:72-98
    2: (32, 18), 3: (32, 20), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def k_scales_bytes(sc, m):
    """The 12 bytes of a K-quant superblock's eight 6-bit sub-block scales sc
    and mins m ([n, 8] each): the packing k_scale_min reads (gguf.mojo:205-221)."""
    sc = np.asarray(sc, np.uint8)
    m = np.asarray(m, np.uint8)
    q = np.zeros((sc.shape[0], 12), np.uint8)
    for j in range(4):
        q[:, j] = sc[:, j] | ((sc[:, j + 4] >> 4) << 6)
        q[:, j + 4] = m[:, j] | ((m[:, j + 4] >> 4) << 6)
        q[:, j + 8] = (sc[:, j + 4] & 0xF) | ((m[:, j + 4] & 0xF) << 4)
    return q


def gguf_blocks(kind, rows, cols, seed, scale=0.01, centered=False):
    """Random GGUF blocks of the Llama GEMV sweep: every code field uniform over
    its range (random bytes), 6-bit sub-scales / mins uniform (random bytes),
    and the float16 scales |N(0, scale)| (Q4_1's min negative, as a min is).
    centered (Q4_K / Q5_K): each sub-block's min equals its scale and dmin is
    d times the codes' mean (7.5 / 15.5), so the weights d sc (q - mean) have
    mean ~0, as trained weights do; uniform codes with random mins give every
    row a common positive offset that swamps a model's dependence on its input."""
    bs, bb = GGUF_BLOCK[kind]
    nb = rows * (cols // bs)
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    if centered and kind in (12, 13):
        d = np.abs(rng.normal(0, scale, nb)).astype(np.float16)
        dmin = (d.astype(np.float32) * (7.5 if kind == 12 else 15.5)).astype(np.float16)
        b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
        b[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
        sc = rng.integers(1, 64, (nb, 8), dtype=np.uint8)
        b[:, 4:16] = k_scales_bytes(sc, sc)
        return b.reshape(-1)

    def f16(col, neg=False):
        v = np.abs(rng.normal(0, scale, nb)).astype(np.float16)
        if neg:
            v = -v
        b[:, col:col + 2] = v.view(np.uint8).reshape(nb, 2)

    if kind in (2, 8):
        f16(0)
    elif kind == 3:
        f16(0)
        f16(2, neg=True)
    elif kind in (12, 13):
        f16(0)
        f16(2)
    elif kind == 14:
        f16(208)
    return b.reshape(-1)


def llama_tensors(cfg, seed, centered=False):
    """Seeded random weights of the config-4 decoder, in llmq_llama_create's
    order (llm_mojo_amd.llama.tensor_names): GGUF blocks whose float16 scales
    keep weights near N(0, 0.02) in size (Q4_K d |N(0, 1e-4)|, Q6_K d
    |N(0, 2e-5)|), norm gains 1."""
    from .llama import tensor_names, tensor_shapes

    shapes = tensor_shapes(cfg)
    out = []
    for i, name in enumerate(tensor_names(cfg["n_layer"])):
        kind = name.rsplit(".", 1)[-1]
        if kind.endswith("norm"):
            out.append(np.ones(cfg["dim"], np.float32))
            continue
        t = cfg["head_type"] if kind == "output" else (cfg["embd_type"] if kind == "token_embd" else cfg["layer_type"])
        rows, cols = shapes[kind]
        out.append(gguf_blocks(t, rows, cols, seed * 1000 + i, scale=2e-5 if t == 14 else 1e-4, centered=centered))
    return out


def llama_prompts(seed, batch, n, vocab):
    """batch x n token ids from the reference's Rng, id = floor(uniform * vocab)."""
    rng = Rng(seed)
    return np.array([[min(vocab - 1, int(rng.uniform() * vocab)) for _ in range(n)] for _ in range(batch)], np.int64)


def prompt_ids(seed, n):
    rng = Rng(seed)
    return np.array([min(V - 1, int(rng.uniform() * V)) for _ in range(n)], np.int64)


__all__ = ["splitmix64", "normal", "gpt2_tensors", "gpt2_safetensors", "Rng", "prompt_ids", "C", "MAX_T", "V"]
