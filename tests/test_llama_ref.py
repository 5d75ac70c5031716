"""The config-4 NumPy statement (tests/llama_ref.py) is the GPU decoder's
only check, so its block form (a whole prompt at once, causal mask) is held
to its one-token-at-a-time form on the CPU: the same logits at the end of a
prompt and after decode positions on the same cache, the same cache codes,
and a planted missing mask lands far outside that bar."""
import numpy as np

from tests.llama_ref import NumpyLlama

CFG = dict(n_layer=2, dim=512, n_head=8, n_kv=2, head_dim=64, ffn=512, vocab=1000, max_t=80, batch=1,
           layer_type=12, head_type=14, embd_type=12, eps=1e-5, theta=10000.0)


def rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_block_equals_token_at_a_time(orc):
    from llm_mojo_amd import synth

    tensors = synth.llama_tensors(CFG, 3)
    toks = synth.llama_prompts(3, 1, 40, CFG["vocab"])[0]
    blk = NumpyLlama(CFG, tensors)
    one = NumpyLlama(CFG, tensors)
    a = blk.forward(0, toks[:37], 0)
    for i in range(37):
        b = one.forward(0, toks[i:i + 1], i)
    assert rel(a, b) <= 1e-5
    assert np.array_equal(blk.cache[0].k, one.cache[0].k) and np.array_equal(blk.cache[0].v, one.cache[0].v)
    assert np.array_equal(blk.cache[0].ks, one.cache[0].ks) and np.array_equal(blk.cache[0].vs, one.cache[0].vs)
    a = blk.forward(0, toks[37:], 37)
    b = one.forward(0, toks[37:], 37)
    assert rel(a, b) <= 1e-5


def test_block_without_mask_differs(orc):
    from llm_mojo_amd import synth

    tensors = synth.llama_tensors(CFG, 4)
    toks = synth.llama_prompts(4, 1, 30, CFG["vocab"])[0]
    good = NumpyLlama(CFG, tensors).block(0, toks, 0)
    bad_model = NumpyLlama(CFG, tensors)
    bad_model.causal = False
    bad = bad_model.block(0, toks, 0)
    # the last row sees every position either way; earlier rows must not
    assert rel(bad[-1], good[-1]) <= 1e-6
    assert rel(bad[10], good[10]) > 1e-3  # 100x the bar above
