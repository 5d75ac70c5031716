"""Saved models and QuantMatrix.restore on the GPU (gpt2t.mojo:612-698,
tensor.mojo:634-656): the device model's file is byte-identical to the
oracle's restatement of save_model, a model loaded from it computes exactly
what the original does, and restore() rebuilds matrices from the
reference's own code layout for every format.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def note(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("bits,group,sym", [(4, 32, False), (4, 128, False), (8, 32, False), (8, 0, False),
                                            (4, 64, True)])
def test_mat_restore_from_reference_layout(gpu, orc, bits, group, sym):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(bits * 100 + group)
    K, N = 512, 80
    w = rng.normal(0, 0.05, (K, N)).astype(np.float32)
    note("restore", bits, group, sym)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    r = lm.HipQuantMatrix.restore(ctx, bits, group, sym, True, o.n, o.k, o.data, o.scale, o.zp)
    codes, scales, zps = r.export()
    assert np.array_equal(codes, o.data) and np.array_equal(scales, o.scale) and np.array_equal(zps, o.zp)
    q = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, True)
    x = torch.from_numpy(rng.normal(0, 1, (3, K)).astype(np.float32)).cuda()
    a = torch.zeros((3, N), device="cuda")
    b = torch.zeros((3, N), device="cuda")
    lm.linear(ctx, a, x, r)
    lm.linear(ctx, b, x, q)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    r.free()
    q.free()


@pytest.fixture(scope="module")
def weights():
    from llm_mojo_amd import synth

    return synth.gpt2_tensors(seed=1337)


@pytest.mark.parametrize("bits", [4, 8])
def test_gpt2_save_is_the_reference_file(gpu, orc, weights, tmp_path, bits):
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2

    note("gpt2 save", bits)
    model = lm.GPT2(ctx, weights, bits=bits, group=32)
    p1, p2 = tmp_path / "dev.bin", tmp_path / "orc.bin"
    model.save(p1)
    params = gpt2.params_list(weights)
    orc.save_model(orc.GPT2(params, bits=bits, group=32), params, p2)
    b1, b2 = p1.read_bytes(), p2.read_bytes()
    assert len(b1) == len(b2)
    if b1 != b2:
        i = next(i for i in range(len(b1)) if b1[i] != b2[i])
        raise AssertionError(f"files differ first at byte {i} of {len(b1)}")
    assert gpt2.saved_formats(p1) == (f"int{bits}-g32-a16", "int8-ch-a16")
    model.free()


def test_gpt2_load_computes_the_same(gpu, orc, weights, tmp_path):
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    prompt = synth.prompt_ids(5, 20)
    model = lm.GPT2(ctx, weights)
    path = tmp_path / "m.bin"
    model.save(path)
    note("gpt2 load")
    loaded = lm.GPT2.load(ctx, path)
    assert loaded.name() == model.name() and loaded.weight_bytes() == model.weight_bytes()
    a = model.forward(prompt, 0)
    b = loaded.forward(prompt, 0)
    assert np.array_equal(a, b)
    ta, _, _ = model.generate(prompt, 16)
    tb, _, _ = loaded.generate(prompt, 16)
    assert np.array_equal(ta, tb)
    li = lm.GPT2.load(ctx, path, attention="int")
    assert li.name().endswith("kv-int8-intattn")
    li.forward(prompt, 0)
    for m in (model, loaded, li):
        m.free()


def test_saved_file_errors(gpu, weights, tmp_path):
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2

    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"GGUF" + bytes(100))
    with pytest.raises(lm.LlmqError, match="not a saved llm_mojo model"):
        lm.GPT2.load(ctx, bad)
    model = lm.GPT2(ctx, weights)
    path = tmp_path / "m.bin"
    model.save(path)
    model.free()
    data = path.read_bytes()
    cut = tmp_path / "cut.bin"
    cut.write_bytes(data[:len(data) // 2])
    with pytest.raises(lm.LlmqError, match="unexpected end"):
        lm.GPT2.load(ctx, cut)
    # a float-activation format (QuantMatrix A16=False) has no device model
    other = tmp_path / "other.bin"
    name = b"int4-g32"
    other.write_bytes(data[:8 + 27 + 8] + len(name).to_bytes(8, "little") + name + data[8 + 27 + 8 + 8 + 12:])
    assert gpt2.saved_formats(other) == ("int4-g32", "int8-ch-a16")
    with pytest.raises(lm.LlmqError, match="device model runs"):
        lm.GPT2.load(ctx, other)
