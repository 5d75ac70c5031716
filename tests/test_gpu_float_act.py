"""QuantMatrix with float activations (A16 = False) on the GPU: gpt2t.mojo's
ten non -a16 --dtype formats (1315-1334) and the HEAD8 head (1231-1232),
through kernels.linear's matmul_rows branch (kernels.mojo:670-671, 285-349)
and the model built on them, against the oracle's restatement
(oracle.matmul_rows, oracle.GPT2 with a16=False).

Bars: codes bit-exact; float32 outputs within 1e-5 of max |out| (the
reference's own kernel tolerance, tests/a16_kernels.mojo:70; the GPU sums
in a different float32 order); the model's logits within 1e-3 of
max |logit| with the top-1 token per teacher-forced step (no int16 codes
here, so the error is float32 summation order carried through 12 layers).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REL = 1e-5
FLOAT_ACT = [(8, 0, False), (8, 0, True), (4, 0, False), (4, 0, True), (4, 128, False), (4, 128, True),
             (4, 64, False), (4, 64, True), (4, 32, False), (4, 32, True)]


def note(*a):
    print(*a, flush=True)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30)


@pytest.mark.parametrize("fmt", FLOAT_ACT)
def test_float_act_codes_bit_exact(gpu, orc, fmt):
    torch, lm, ctx = gpu
    bits, group, sym = fmt
    rng = np.random.default_rng(bits + group + sym)
    w = rng.normal(0, 0.02, (768, 70)).astype(np.float32)
    note("codes", fmt)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, False)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, False)
    codes, scales, zps = g.export()
    assert np.array_equal(codes, o.data) and np.array_equal(scales, o.scale) and np.array_equal(zps, o.zp)
    assert g.nbytes() == o.nbytes() and g.has_i16() is False
    g.free()


CASES = [  # (fmt index, T, IN, OUT): decode GEMVs of GPT-2 shapes, ragged rows, several tokens
    *[(i, 1, 768, 2304) for i in range(len(FLOAT_ACT))],
    *[(i, 1, 3072, 768) for i in (0, 3, 5, 8)],
    *[(i, 1, 768, 70) for i in (1, 6, 9)],
    *[(i, T, 768, 70) for i in (0, 4, 9) for T in (3, 17)],
    *[(i, 40, 3072, 768) for i in (2, 7)],
    (8, 1, 4096, 11008), (0, 1, 11008, 4096),
]


@pytest.mark.parametrize("fi,T,IN,OUT", CASES)
def test_float_act_linear_vs_oracle(gpu, orc, fi, T, IN, OUT):
    torch, lm, ctx = gpu
    bits, group, sym = FLOAT_ACT[fi]
    rng = np.random.default_rng(T * 131 + IN + OUT + fi)
    w = rng.uniform(-0.1, 0.1, (IN, OUT)).astype(np.float32)
    x = rng.uniform(-1, 1, (T, IN)).astype(np.float32)
    b = rng.uniform(-1, 1, OUT).astype(np.float32)
    note("linear", FLOAT_ACT[fi], T, IN, OUT)
    g = lm.HipQuantMatrix.from_f32(ctx, w, bits, group, sym, False)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, False)
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert rel_err(got, orc.matmul_rows(x, o, b)) < REL
    assert rel_err(got, x.astype(np.float64) @ o.dequant().astype(np.float64).T + b) < REL
    g.free()


@pytest.mark.parametrize("T", [1, 6])
def test_float_act_epilogues_and_layernorm(gpu, orc, T):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(40 + T)
    IN, OUT = 768, 3072
    w = rng.normal(0, 0.05, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (T, IN)).astype(np.float32)
    b = rng.normal(0, 1, OUT).astype(np.float32)
    lw = rng.uniform(0.5, 1.5, IN).astype(np.float32)
    lb = rng.normal(0, 0.1, IN).astype(np.float32)
    base = rng.normal(0, 1, (T, OUT)).astype(np.float32)
    note("epilogues", T)
    g = lm.HipQuantMatrix.from_f32(ctx, w, 4, 128, False, False)
    o = orc.QuantMatrix.from_f32(w, 4, 128, False, False)
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), gelu=True)
    torch.cuda.synchronize()
    assert rel_err(out.cpu().numpy(), orc.matmul_rows(x, o, b, orc.EPI_BIAS | orc.EPI_GELU)) < REL
    out = dev(torch, base)
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), resid=True)
    torch.cuda.synchronize()
    want = orc.matmul_rows(x, o, b, orc.EPI_BIAS | orc.EPI_RESID, out=base.copy())
    assert rel_err(out.cpu().numpy(), want) < REL
    out = torch.zeros((T, OUT), dtype=torch.float32, device="cuda")
    lm.linear(ctx, out, dev(torch, x), g, dev(torch, b), ln=(dev(torch, lw), dev(torch, lb)))
    torch.cuda.synchronize()
    assert rel_err(out.cpu().numpy(), orc.matmul_rows(orc.layernorm(x, lw, lb), o, b)) < REL
    g.free()


@pytest.mark.parametrize("T", [1, 3])
def test_head8_float_activations(gpu, orc, T):
    """HEAD8 = QuantMatrix[8, 0, False] over the GPT-2 vocabulary (50257 rows:
    a partial last row tile) through llmq_head."""
    torch, lm, ctx = gpu
    rng = np.random.default_rng(9 + T)
    V, C = 50257, 768
    wte = rng.normal(0, 0.02, (V, C)).astype(np.float32)
    h = rng.normal(0, 1, (T, C)).astype(np.float32)
    note("head8", T)
    g = lm.HipQuantMatrix.from_f32(ctx, wte, 8, 0, False, False, reduce_rows=False)
    o = orc.QuantMatrix.from_f32(wte, 8, 0, False, False, reduce_rows=False)
    logits = torch.zeros((T, V), dtype=torch.float32, device="cuda")
    lm.head(ctx, logits, dev(torch, h), g)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    want = orc.matmul_rows(h, o, None, 0)
    assert rel_err(got, want) < REL
    assert [int(np.argmax(r)) for r in got] == [orc.argmax(r) for r in want]
    g.free()


@pytest.fixture(scope="module")
def weights():
    from llm_mojo_amd import synth

    return synth.gpt2_tensors(seed=1337)


MODELS = [  # (--dtype, --head, oracle head format or None for int8-ch)
    ("int4-g128", "int8", None),
    ("int8-ch-sym", "same", (8, 0, True, False)),
    ("int4-g32", "int8", None),
]


@pytest.mark.parametrize("dtype,head,ehead", MODELS)
def test_gpt2_float_act_teacher_forced(gpu, orc, weights, dtype, head, ehead):
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2, synth

    bits = int(dtype[3])
    g = dtype.split("-")[1]
    group = 0 if g == "ch" else int(g[1:])
    sym = "-sym" in dtype
    note("gpt2 float act", dtype, head)
    model = lm.GPT2(ctx, weights, dtype=dtype, head=head)
    want_name = dtype + ("" if head == "same" else "+head-int8-ch") + "+kv-int8"
    assert model.name() == want_name
    ref = orc.GPT2(gpt2.params_list(weights), bits=bits, group=group, sym=sym, a16=False, head=ehead)
    prompt = synth.prompt_ids(77, 10)
    lg = model.forward(prompt, 0)
    lo = ref.forward(prompt, 0)
    errs = [rel_err(lg, lo)]
    agree = [int(np.argmax(lg) == orc.argmax(lo))]
    pos = len(prompt)
    for i in range(6):
        nxt = orc.argmax(lo)
        note("decode step", i)
        lg = model.forward([nxt], pos)
        lo = ref.forward([nxt], pos)
        pos += 1
        errs.append(rel_err(lg, lo))
        agree.append(int(np.argmax(lg) == orc.argmax(lo)))
    note("max logit rel err", max(errs), "top-1", sum(agree), "/", len(agree))
    assert max(errs) < 1e-3
    assert sum(agree) >= len(agree) - 1
    model.free()


def test_gpt2_float_act_generate_save_load(gpu, orc, weights, tmp_path):
    """The device-driven greedy loop over a float-activation head (its argmax
    partials) equals teacher forcing of its own picks; the saved file is the
    oracle's save_model byte for byte and loads back to the same logits."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2, synth

    prompt = synth.prompt_ids(12, 8)
    note("gpt2 float act generate")
    model = lm.GPT2(ctx, weights, dtype="int4-g64-sym", head="int8")
    toks, _, _ = model.generate(prompt, 6)
    want = []
    lg = model.forward(prompt, 0)
    for i in range(6):
        nxt = int(np.argmax(lg))
        if nxt == 50256:
            break
        want.append(nxt)
        lg = model.forward([nxt], len(prompt) + i)
    assert toks.tolist() == want
    note("gpt2 float act save")
    p1, p2 = tmp_path / "dev.bin", tmp_path / "orc.bin"
    model.save(p1)
    params = gpt2.params_list(weights)
    orc.save_model(orc.GPT2(params, bits=4, group=64, sym=True, a16=False), params, p2)
    assert p1.read_bytes() == p2.read_bytes()
    assert gpt2.saved_formats(p1) == ("int4-g64-sym", "int8-ch")
    loaded = lm.GPT2.load(ctx, p1)
    assert loaded.name() == model.name()
    assert np.array_equal(loaded.forward(prompt, 0), model.forward(prompt, 0))
    loaded.free()
    model.free()
