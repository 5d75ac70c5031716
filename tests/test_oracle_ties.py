"""Exact .5 ties in config 0: the codes whose value the tie rule of Mojo's
round() decides (tensor.mojo:377,381; kernels.mojo:415; kvcache.mojo:330).
The oracle and the GPU round half away from zero.  The reference's own
evidence on the rule is textual: PLAN.md:394-397 reports that its NumPy
restatement (tests/reference.py --act16, whose np.round is half to even)
matches the Mojo run to 5 digits, "the remaining difference is rounding of
exact .5 ties", so Mojo's round() is not half to even; half away from zero
is the other rule in use (and LLVM's llvm.round, which a SIMD round lowers
to, is defined that way).  No run of Mojo here can settle it beyond that
text.  On the synthetic checkpoint the weights meet 136 ties and the int16
activation codes about 31 per forward, so the rule is not moot: these tests
pin the counts and show what half to even would change: the same greedy
tokens, logits within 3e-3 of max |logit|.
"""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def params():
    from llm_mojo_amd import gpt2, synth

    return gpt2.params_list(synth.gpt2_tensors(seed=1337))


def decode(orc, model, steps=20):
    from llm_mojo_amd import synth

    prompt = [int(v) for v in synth.prompt_ids(1000, 12)]
    lo = model.forward(prompt, 0)
    toks, logits = [], [lo]
    for i in range(steps):
        toks.append(orc.argmax(lo))
        lo = model.forward([toks[-1]], 12 + i)
        logits.append(lo)
    return toks, logits


def test_config0_tie_counts_and_the_other_rule(orc, params):
    orc.set_threads(8)
    orc.set_round_half_even(False)
    orc.ties(reset=True)
    away = orc.GPT2(params)
    t = orc.ties(reset=True)
    assert t == {"weights": 136, "activations": 0, "kv": 0, "other": 0}, t
    toks_a, lg_a = decode(orc, away)
    t = orc.ties(reset=True)
    print("ties in a 12-token prompt + 20 decode forwards:", t, flush=True)
    assert t["weights"] == 0 and t["other"] == 0
    assert 21 * 10 < t["activations"] < 21 * 60 and t["kv"] >= 0
    try:
        orc.set_round_half_even(True)
        even = orc.GPT2(params)
        toks_e, lg_e = decode(orc, even)
    finally:
        orc.set_round_half_even(False)
    assert toks_a == toks_e
    worst = max(float(np.max(np.abs(a - e)) / np.max(np.abs(a))) for a, e in zip(lg_a, lg_e))
    print(f"half-even vs half-away: max rel logit difference {worst:.2e}", flush=True)
    assert 0 < worst < 3e-3
