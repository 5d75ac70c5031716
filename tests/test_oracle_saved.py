"""Pins the oracle's restatement of the saved-model file (gpt2t.mojo:612-698,
serialize.mojo, QuantMatrix.save tensor.mojo:634-644).  The reference
commits no saved files, so the writer is checked against what its text
fixes: the header bytes, the size (header + per matrix 24 bytes + nbytes(),
tensor.mojo:629-632, + the small floats, which is Model.weight_bytes,
gpt2t.mojo:312-319, plus the framing), and a read back of every matrix and
of the small tensors in Model.small's order.
"""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def model(orc):
    from llm_mojo_amd import gpt2, synth

    params = gpt2.params_list(synth.gpt2_tensors(seed=1337))
    return orc.GPT2(params), params


def test_saved_file_layout(orc, model, tmp_path):
    m, params = model
    path = tmp_path / "gpt2.bin"
    orc.save_model(m, params, path)
    b = path.read_bytes()
    # magic (27 bytes), version 1, "int4-g32-a16", "int8-ch-a16"
    head = (bytes([27]) + bytes(7) + b"llm_mojo GPT-2 124M weights" + bytes([1]) + bytes(7)
            + bytes([12]) + bytes(7) + b"int4-g32-a16" + bytes([11]) + bytes(7) + b"int8-ch-a16")
    assert b[:len(head)] == head
    # wte: rows 50257, cols 768, group 768 (one group per row)
    assert b[len(head):len(head) + 24] == (50257).to_bytes(8, "little") + (768).to_bytes(8, "little") * 2
    mats = [m.mat(-1)] + [m.mat(i) for i in range(48)]
    nbytes = sum(q.n * q.k * q.bits // 8 + 3 * (q.n * q.k // q.group) for q in mats)
    small = 12 * 13 * 768 + 1024 * 768 + 2 * 768  # SMALL_FLOATS, gpt2t.mojo:576
    assert nbytes + 4 * small == 92809203  # Model.weight_bytes of int4-g32-a16 + HEAD8_A16
    assert len(b) == len(head) + 49 * 24 + nbytes + 8 + 4 * small


def test_saved_file_reads_back(orc, model, tmp_path):
    m, params = model
    path = tmp_path / "gpt2.bin"
    orc.save_model(m, params, path)
    r = orc.read_saved(path)
    assert r["end"] and r["layers"] == "int4-g32-a16" and r["head"] == "int8-ch-a16"
    q = m.mat(5)  # layer 1's proj (load_model's order: qkv, proj, fc, fcproj)
    rows, cols, group, codes, scales, zps = r["mats"][6]
    assert (rows, cols, group) == (768, 768, 32)
    import ctypes

    assert codes.tobytes() == ctypes.string_at(q.data, 768 * 768 // 2)
    assert scales.tobytes() == ctypes.string_at(q.scale, 2 * 768 * 24)
    # Model.small: layer 0's ln_1.weight first, layer 11's mlp.c_proj.bias
    # before wpe, then ln_f.weight and ln_f.bias last
    s = r["small"]
    assert np.array_equal(s[:768], params[4])
    off = 12 * 13 * 768
    assert np.array_equal(s[off - 768:off], params[4 + 12 * 11 + 11])
    assert np.array_equal(s[off:off + 1024 * 768], params[1].ravel())
    assert np.array_equal(s[-1536:-768], params[2]) and np.array_equal(s[-768:], params[3])


def test_read_saved_rejects_other_files(orc, tmp_path):
    p = tmp_path / "x.bin"
    p.write_bytes(b"GGUF" + bytes(60))
    with pytest.raises(ValueError, match="not a saved llm_mojo model"):
        orc.read_saved(p)
