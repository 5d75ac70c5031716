"""The CPU baseline (oracle/llmq_oracle.c, orc_cpu_*): the reference's team
decode (gpt2t.mojo:350-447) with VPDPWSSD dots, vector int16 quantization
and attention, against the scalar oracle it restates: bit-identical logits
at several team sizes and the same greedy tokens.  On a CPU without AVX-512
VNNI the same entry points run the scalar code (cpu_vnni() == 0)."""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def params():
    from llm_mojo_amd import gpt2, synth

    return gpt2.params_list(synth.gpt2_tensors(seed=1337))


def test_team_decode_bit_identical(orc, params):
    from llm_mojo_amd import synth

    orc.set_threads(8)
    print("VPDPWSSD path:", bool(orc.cpu_vnni()), flush=True)
    m = orc.GPT2(params)
    prompt = [int(v) for v in synth.prompt_ids(1001, 12)]
    tok = orc.argmax(m.forward(prompt, 0))
    for pos, nt in ((12, 1), (12, 3), (12, 8)):
        want = m.forward([tok], pos)  # rewrites the same cache slot with the same values
        got = m.cpu_decode(tok, pos, nt)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (pos, nt)
    # a longer context (positions 13 .. 40), team of 4
    for pos in range(13, 41):
        want = m.forward([tok], pos)
        got = m.cpu_decode(tok, pos, 4)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos
        tok = orc.argmax(got)


def test_team_generate_same_tokens(orc, params):
    from llm_mojo_amd import synth

    prompt = [int(v) for v in synth.prompt_ids(1002, 12)]
    want = orc.GPT2(params).generate(prompt, 40)
    toks, prompt_s, decode_s = orc.GPT2(params).cpu_generate(prompt, 40, 3)
    assert list(toks) == list(want)
    assert prompt_s > 0 and decode_s > 0
    with pytest.raises(ValueError):
        orc.GPT2(params).cpu_generate(prompt, 40, 0)


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


def test_prompt_vnni_tiles_bit_identical(orc, params):
    """The prompt forward on VPDPWSSD tiles, vector quantizer and attention
    (the config-3 CPU baseline) gives the scalar oracle's logits bit for bit,
    and the fast forms switch off again afterwards."""
    from llm_mojo_amd import synth

    prompt = [int(v) for v in synth.prompt_ids(1003, 45)]
    orc.set_threads(8)
    want = orc.GPT2(params).forward(prompt, 0)
    got, secs = orc.GPT2(params).cpu_prompt(prompt, 8)
    assert secs > 0
    assert bits_equal(got, want)
    assert orc.cpu_set_fast(False) is False


@pytest.mark.parametrize("bits,group,sym", [(4, 32, False), (8, 0, False), (4, 64, False), (4, 128, True),
                                            (8, 32, False), (8, 128, False), (4, 0, False)])
@pytest.mark.parametrize("T", [1, 5, 37])
def test_matmul_vnni_forms_bit_identical(orc, bits, group, sym, T):
    """Every A16 format through matmul_rows_a16 with the baseline's forms on
    (one-token rows by branch, the 32-row VNNI tiles, rows_i16's tail)."""
    rng = np.random.default_rng(bits * 100 + group + T)
    IN, OUT = 768, 70  # 70 rows: two tiles and a 6-row tail
    w = rng.normal(0, 0.02, (IN, OUT)).astype(np.float32)
    x = rng.normal(0, 1, (T, IN)).astype(np.float32)
    b = rng.normal(0, 0.1, OUT).astype(np.float32)
    o = orc.QuantMatrix.from_f32(w, bits, group, sym, True)
    flags = orc.EPI_BIAS | orc.EPI_GELU
    want = orc.matmul_rows_a16(x, o, b, flags)
    assert orc.cpu_set_fast(True) == bool(orc.cpu_vnni())
    try:
        got = orc.matmul_rows_a16(x, o, b, flags)
    finally:
        orc.cpu_set_fast(False)
    assert bits_equal(got, want)


@pytest.mark.parametrize("t", [2, 3, 8, 12, 13, 14])
def test_gguf_avx512_rows_bit_identical(orc, t):
    """The baseline's AVX-512 GGUF decoders (config-2 CPU GEMVs) equal the
    scalar GGUFMatrix.dot_row restatement row by row."""
    from llm_mojo_amd import synth

    rows, cols = 24, 2048
    blocks = synth.gguf_blocks(t, rows, cols, seed=t)
    rb = cols // synth.GGUF_BLOCK[t][0] * synth.GGUF_BLOCK[t][1]
    x = np.random.default_rng(t).normal(0, 1, cols).astype(np.float32)
    for r in range(rows):
        row = blocks[r * rb:(r + 1) * rb]
        assert bits_equal(orc.cpu_gguf_dot_row(t, row, cols, x), orc.gguf_dot_row(t, row, cols, x)), r
    secs, out = orc.cpu_gguf_gemv_seconds(t, [blocks, blocks.copy()], rows, cols, x, 2, reps=3)
    assert secs > 0
    want = np.array([orc.gguf_dot_row(t, blocks[r * rb:(r + 1) * rb], cols, x) for r in range(rows)], np.float32)
    assert bits_equal(out, want)


def test_gemv_seconds_team(orc):
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, (768, 2304)).astype(np.float32)
    x = rng.normal(0, 1, (1, 768)).astype(np.float32)
    mats = [orc.QuantMatrix.from_f32(w, 4, 64, False, True) for _ in range(2)]
    secs, out = orc.cpu_gemv_seconds(mats, x, 3, reps=5)
    assert secs > 0
    assert bits_equal(out, orc.matmul_rows_a16(x, mats[0], None, 0)[0])
