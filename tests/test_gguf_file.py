"""GGUFFile (gguf.mojo:519-636): libllmq's reader and the oracle's
restatement of the reference's reader, on files written from ggml's
published format description (tests/gguf_write.py).  Host-only: no GPU
call is made.
"""
import numpy as np
import pytest

from tests import gguf_write as gw


@pytest.fixture(scope="module")
def lm():
    import llm_mojo_amd

    llm_mojo_amd.lib()
    return llm_mojo_amd


def tensors(rng):
    """(name, ggml type, dims, bytes) of several formats and shapes."""
    out = [
        ("position_embd.weight", 0, [8, 5], gw.f32_bytes(rng.normal(0, 1, (5, 8)))),
        ("blk.0.attn_norm.bias", 0, [8], gw.f32_bytes(rng.normal(0, 1, 8))),
        ("token_embd.weight", 1, [32, 3], gw.f16_bytes(rng.normal(0, 1, (3, 32)))),
        ("blk.0.ffn_up.weight", 2, [64, 4], rng.integers(0, 256, 4 * 2 * 18, dtype=np.uint8).tobytes()),
        ("blk.0.attn_qkv.weight", 8, [32, 6], rng.integers(0, 256, 6 * 34, dtype=np.uint8).tobytes()),
        ("output.weight", 14, [256, 2, 3], rng.integers(0, 256, 6 * 210, dtype=np.uint8).tobytes()),
        ("blk.1.ffn_down.weight", 12, [512, 3], rng.integers(0, 256, 3 * 2 * 144, dtype=np.uint8).tobytes()),
    ]
    return out


METADATA = [
    ("general.architecture", gw.STRING, "gpt2"),
    ("general.name", gw.STRING, "tiny ünïcode"),
    ("gpt2.context_length", gw.U32, 1024),
    ("gpt2.block_count", gw.U64, 12),
    ("some.i8", gw.I8, -3), ("some.u16", gw.U16, 7), ("some.i16", gw.I16, -9), ("some.i32", gw.I32, -1),
    ("some.f32", gw.F32, 1.5), ("some.bool", gw.BOOL, True), ("some.i64", gw.I64, -5), ("some.f64", gw.F64, 2.25),
    ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["a", "bc", "", "def"])),
    ("tokenizer.ggml.scores", gw.ARRAY, (gw.F32, [0.5, -1.0, 2.0])),
    ("nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2, 3]), (gw.STRING, ["x"])])),
]


@pytest.mark.parametrize("version,alignment", [(3, None), (2, 64), (3, 256)])
def test_reader_matches_the_written_layout(lm, orc, tmp_path, version, alignment):
    rng = np.random.default_rng(version * 1000 + (alignment or 0))
    ts = tensors(rng)
    path = tmp_path / "t.gguf"
    start, offsets = gw.write(path, ts, METADATA, version=version, alignment=alignment)
    g = lm.GGUFFile(path)
    ostart, oidx = orc.gguf_index(path)
    assert ostart == start
    assert g.names() == [t[0] for t in ts]
    for (name, gt, dims, data), off in zip(ts, offsets):
        rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
        assert g.info(name) == (gt, rows, dims[0], off)
        assert oidx[name] == (gt, dims[0], rows, off)
        assert g.tensor_bytes(name).tobytes() == data
        assert g.has(name)
    assert not g.has("missing.weight")
    pe = g.f32("position_embd.weight")
    assert pe.shape == (5, 8) and pe.tobytes() == ts[0][3]
    with pytest.raises(ValueError, match="expected F32"):
        g.f32("token_embd.weight")
    g.close()


def test_reader_errors(lm, tmp_path):
    rng = np.random.default_rng(3)
    ts = tensors(rng)
    good = tmp_path / "good.gguf"
    gw.write(good, ts, METADATA)
    data = good.read_bytes()
    cases = {
        "magic": (b"GGML" + data[4:], "not a GGUF file"),
        "version": (data[:4] + (1).to_bytes(4, "little") + data[8:], "version 1 is not supported"),
        "metadata": (data[:200], "corrupt or truncated"),
        "type": (None, "corrupt or truncated GGUF metadata"),
    }
    # an unknown metadata value type (13) in the first entry
    klen = len("general.architecture")
    at = 24 + 8 + klen
    cases["type"] = (data[:at] + (13).to_bytes(4, "little") + data[at + 4:], cases["type"][1])
    for name, (blob, msg) in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(blob)
        with pytest.raises(lm.LlmqError, match=msg):
            lm.GGUFFile(p)
    # the index is whole but the last tensor's data is cut off
    p = tmp_path / "short.gguf"
    p.write_bytes(data[:-100])
    g = lm.GGUFFile(p)
    with pytest.raises(lm.LlmqError, match="past the end"):
        g.tensor_bytes("blk.1.ffn_down.weight")
    assert g.tensor_bytes("position_embd.weight").size == 160
    with pytest.raises(KeyError):
        g.info("nope")


def test_reader_refuses_overflowing_fields(lm, tmp_path):
    """Index fields whose arithmetic would wrap are refused with LLMQ_EINVAL
    (-1), never read through: a tensor offset of 2^63 - 16 (the end of its
    data would wrap past 2^63) and dimensions whose product exceeds 2^63."""
    data = bytes(34)  # one Q8_0 block
    p = tmp_path / "offset.gguf"
    gw.write(p, [("t", 8, [32, 1], data)])
    blob = bytearray(p.read_bytes())
    at = 24 + 8 + 1 + 4 + 2 * 8 + 4  # header, name "t", n_dims, two dims, type: the u64 offset
    assert int.from_bytes(blob[at:at + 8], "little") == 0
    blob[at:at + 8] = (2 ** 63 - 16).to_bytes(8, "little")
    p.write_bytes(bytes(blob))
    g = lm.GGUFFile(p)
    with pytest.raises(lm.LlmqError, match=r"error -1: .*past the end"):
        g.tensor_bytes("t")
    g.close()
    p = tmp_path / "dims.gguf"
    gw.write(p, [("t", 8, [32, 2 ** 33, 2 ** 33], data)])  # 2^66 rows
    with pytest.raises(lm.LlmqError, match=r"error -1: .*impossible shape"):
        lm.GGUFFile(p)
    p = tmp_path / "dims2.gguf"
    gw.write(p, [("t", 8, [32, 2 ** 40, 2 ** 40, 3], data)])
    with pytest.raises(lm.LlmqError, match=r"error -1: .*impossible shape"):
        lm.GGUFFile(p)
