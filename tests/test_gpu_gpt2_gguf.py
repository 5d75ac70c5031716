"""GPT-2 124M from a GGUF file on the GPU (load_gguf, gpt2t.mojo:728-760)
against its CPU statement on the oracle's parts (tests/gpt2_gguf_ref.py),
on synthetic files: Q8_0 layers with the head tied to a Q8_0 token_embd
(head_i16), and Q4_K layers with a separate Q6_K output and a Q4_0
embedding.  Bars as for the QuantMatrix model: logits within 2e-3 of
max |logit| and top-1 per teacher-forced step (int16 head codes can flip
by one between float summation orders).
"""
import numpy as np
import pytest

from tests.gpt2_gguf_ref import GGUFGPT2Ref, write_gpt2_gguf

pytestmark = pytest.mark.gpu

STEPS = 6
LOGIT_REL = 2e-3


def note(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("layer_type,embd_type,head_type", [(8, 8, None), (12, 2, 14)])
def test_gpt2_gguf_forward_and_decode(gpu, orc, tmp_path, layer_type, embd_type, head_type):
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    path = tmp_path / "gpt2.gguf"
    note("write gguf", layer_type, embd_type, head_type)
    t = write_gpt2_gguf(path, 3, layer_type, embd_type, head_type)
    model = lm.GPT2.from_gguf(ctx, path)
    assert model.name() == "gguf+kv-int8"
    nb = sum(v[3].nbytes if v[0] == 0 else len(v[3]) for k, v in t.items() if v[0] != 0)
    assert model.weight_bytes() == nb + 4 * (12 * 13 * 768 + 1024 * 768 + 2 * 768)
    ref = GGUFGPT2Ref(t)
    prompt = synth.prompt_ids(9, 8)
    note("prefill")
    lg = model.forward(prompt, 0)
    lo = ref.forward(prompt, 0)
    errs = [np.max(np.abs(lg - lo)) / np.max(np.abs(lo))]
    agree = [int(np.argmax(lg) == orc.argmax(lo))]
    pos = len(prompt)
    for i in range(STEPS):
        nxt = orc.argmax(lo)
        note("decode step", i)
        lg = model.forward([nxt], pos)
        lo = ref.forward([nxt], pos)
        pos += 1
        errs.append(np.max(np.abs(lg - lo)) / np.max(np.abs(lo)))
        agree.append(int(np.argmax(lg) == orc.argmax(lo)))
    note("max logit rel err", max(errs), "top-1", sum(agree), "/", len(agree))
    assert max(errs) < LOGIT_REL
    assert sum(agree) >= len(agree) - 1
    # greedy generation on a fresh model equals teacher forcing of its own picks
    m2 = lm.GPT2.from_gguf(ctx, path)
    toks, pre_ms, dec_ms = m2.generate(prompt, 5)
    want, p = [], list(prompt)
    lg = model.forward(prompt, 0)  # the first model's cache is rewritten from position 0
    for i in range(5):
        nxt = int(np.argmax(lg))
        if nxt == 50256:
            break
        want.append(nxt)
        lg = model.forward([nxt], len(prompt) + i)
    assert toks.tolist() == want
    model.free()
    m2.free()


def test_gpt2_gguf_errors(gpu, tmp_path):
    torch, lm, ctx = gpu
    from tests import gguf_write as gw

    p = tmp_path / "empty.gguf"
    gw.write(p, [("position_embd.weight", 0, [768, 1024], bytes(768 * 1024 * 4))])
    with pytest.raises(lm.LlmqError, match="tensor not in GGUF file: token_embd.weight"):
        lm.GPT2.from_gguf(ctx, p)
