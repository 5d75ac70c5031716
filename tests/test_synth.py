"""The synthetic-input generator's K-quant helpers against the oracle's
GGUF decoder (gguf.mojo:178-297): the 12-byte scale / min packing decodes to
the sub-block scales and mins it was given, and centered Q4_K / Q5_K blocks
dequantize to weights of mean ~0."""
import numpy as np


def test_k_scales_bytes_decode(orc):
    from llm_mojo_amd import synth

    rng = np.random.default_rng(0)
    n = 64
    sc = rng.integers(0, 64, (n, 8), dtype=np.uint8)
    m = rng.integers(0, 64, (n, 8), dtype=np.uint8)
    b = np.zeros((n, 144), np.uint8)
    one = np.array([1.0], np.float16).view(np.uint8)
    b[:, 0:2] = one
    b[:, 2:4] = one
    b[:, 4:16] = synth.k_scales_bytes(sc, m)
    b[:, 16:] = 0x11  # every code 1
    w = orc.gguf_dequant(12, b.reshape(-1), n, 256).reshape(n, 8, 32)
    want = (sc.astype(np.float32) - m.astype(np.float32))[:, :, None]  # d sc q - dmin m with q = 1
    assert np.array_equal(w, np.broadcast_to(want, w.shape))


def test_centered_blocks_have_zero_mean(orc):
    from llm_mojo_amd import synth

    for kind in (12, 13):
        plain = orc.gguf_dequant(kind, synth.gguf_blocks(kind, 64, 2048, 1, scale=1e-4), 64, 2048)
        cent = orc.gguf_dequant(kind, synth.gguf_blocks(kind, 64, 2048, 1, scale=1e-4, centered=True), 64, 2048)
        assert abs(plain.mean()) > 0.5 * plain.std()  # the offset the option removes
        assert abs(cent.mean()) < 0.01 * cent.std()
        # row means at the noise of 2048 samples (std / 45), no common offset
        assert abs(cent.mean(axis=1)).max() < 0.15 * cent.std()
