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
