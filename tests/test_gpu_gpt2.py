"""End-to-end GPT-2 124M int4-g32-a16 (+ int8-ch head, int8 KV) on the GPU
against the CPU oracle's restatement of gpt2t.mojo, on the seeded synthetic
checkpoint (seeded N(0, 0.02) weights): config 0 as generate runs it, a
12-token prompt then 100 greedy tokens (99 decode forwards,
gpt2t.mojo:969-980), for 10 seeded prompts.

Every float operation on the GPU's decode path follows the reference's
order (tests/test_gpu_exact.py pins each kernel bit for bit), so the bar
is exact: at every step (teacher-forced: both sides are fed the oracle's
greedy token) the logits are bit-identical and every int16 activation code
of every linear's input equals the oracle's (the code-flip rate, counted
per layer and matrix, is zero), and the device-driven greedy loop emits the
oracle's tokens.
"""
import numpy as np
import pytest

from tests.gpt2_exact import bits_equal, check_decode_exact

pytestmark = pytest.mark.gpu

STEPS = 100  # generated tokens per prompt (99 decode forwards)
PROMPTS = 10


@pytest.fixture(scope="module")
def weights():
    from llm_mojo_amd import synth

    return synth.gpt2_tensors(seed=1337)


@pytest.fixture(scope="module")
def models(gpu, orc, weights):
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2

    orc.set_threads(16)
    print("gpt2 load", flush=True)
    model = lm.GPT2(ctx, weights)
    ref = orc.GPT2(gpt2.params_list(weights))
    assert model.weight_bytes() == 50429952 + 38748147 + 4 * (12 * 13 * 768 + 1024 * 768 + 2 * 768)
    yield model, ref
    model.free()


@pytest.mark.parametrize("seed", range(PROMPTS))
def test_gpt2_decode_matches_oracle_exactly(gpu, orc, models, seed):
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    model, ref = models
    prompt = [int(v) for v in synth.prompt_ids(1000 + seed, 12)]
    check_decode_exact(torch, orc, model, ref, prompt, STEPS, f"prompt {seed}")


def test_gpt2_embed_fold_same_tokens(gpu, orc, models, weights, monkeypatch):
    """The decode step's embed step (the pick from the head's argmax
    partials, the embedding and position rows) runs in the first qkv GEMV's
    prologue by default, with embed_kernel under LLMQ_EMBED_FOLD=0: both
    loops emit the oracle's greedy tokens, for 1, 2 and 30 tokens (the first
    has no decode forward, the second one), twice in a row on one model (the
    captured step graph replayed from a new prompt's state)."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    model, ref = models
    monkeypatch.setenv("LLMQ_EMBED_FOLD", "0")
    plain = lm.GPT2(ctx, weights)
    for seed, steps in ((7, 1), (8, 2), (9, 30), (10, 30)):
        prompt = [int(v) for v in synth.prompt_ids(3000 + seed, 12)]
        want = list(ref.generate(prompt, steps))
        want = want[:next((i for i, t in enumerate(want) if t == 50256), len(want))]
        print("embed fold: prompt", seed, "steps", steps, flush=True)
        monkeypatch.setenv("LLMQ_EMBED_FOLD", "0")
        a, _, _ = plain.generate(prompt, steps)
        monkeypatch.delenv("LLMQ_EMBED_FOLD")
        b, _, _ = model.generate(prompt, steps)
        assert a.tolist() == want and b.tolist() == want, (a.tolist(), b.tolist(), want)
    plain.free()


@pytest.mark.parametrize("n_prompt,steps", [(1, 20), (1000, 30)])
def test_gpt2_generate_edges(gpu, orc, models, n_prompt, steps):
    """generate at the edges of its range: a one-token prompt (its forward
    takes the one-token kernels; the decode graph starts at position 1), and
    a 1000-token prompt asked for 30 tokens, which gpt2t.mojo:945 clamps to
    the 24 that fit the 1024 positions (the last decode step writes the
    cache's last slot).  The tokens are the oracle's greedy ones."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    model, ref = models
    prompt = [int(v) for v in synth.prompt_ids(5000 + n_prompt, n_prompt)]
    want = list(ref.generate(prompt, min(steps, 1024 - n_prompt)))  # the oracle takes the clamped count
    print("generate edges", n_prompt, steps, flush=True)
    got, _, _ = model.generate(prompt, steps)
    assert got.tolist() == want


@pytest.mark.parametrize("k", [1, 3, 64])
def test_gpt2_steps_per_graph_same_tokens(gpu, orc, models, monkeypatch, k):
    """k decode steps captured as one graph (LLMQ_GRAPH_STEPS; the remainder
    below k as one-step graphs): 30 tokens are 29 decode steps, so k = 3
    replays the 3-step graph 9 times and the one-step graph twice, k = 64
    only the one-step graph.  The tokens are the oracle's greedy ones."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    model, ref = models
    prompt = [int(v) for v in synth.prompt_ids(3100 + k, 12)]
    want = list(ref.generate(prompt, 30))
    monkeypatch.setenv("LLMQ_GRAPH_STEPS", str(k))
    print("steps per graph", k, flush=True)
    got, _, _ = model.generate(prompt, 30)
    assert got.tolist() == want


@pytest.mark.parametrize("bits", [4, 8])
def test_gpt2_prompt_kv_store_in_gemm(gpu, orc, weights, monkeypatch, bits):
    """A prompt's keys and values go to the int8 cache from the qkv GEMM's
    epilogue (the workgroups whose 64 rows are one head's keys or values)
    instead of kv_store_kernel (LLMQ_KV_FOLD=0): after a 40-token prompt
    (a partial last token tile) and two decode tokens, both models' logits
    are the same bits at every step.  The prompt's logits are the oracle's
    bits for both formats; so are the decode steps' for int4-g32 (int8-g32's
    one-token GEMV runs in free order: its int16 codes can flip, so its bar
    is the code-flip spread, 2e-3 of max |logit|, and top-1)."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2, synth

    prompt = [int(v) for v in synth.prompt_ids(4040 + bits, 40)]
    monkeypatch.setenv("LLMQ_KV_FOLD", "0")
    plain = lm.GPT2(ctx, weights, bits=bits, group=32)
    monkeypatch.delenv("LLMQ_KV_FOLD")
    fold = lm.GPT2(ctx, weights, bits=bits, group=32)
    ref = orc.GPT2(gpt2.params_list(weights), bits=bits, group=32)
    print("kv store in gemm: prompt", bits, flush=True)
    monkeypatch.setenv("LLMQ_KV_FOLD", "0")
    la = plain.forward(prompt, 0)
    monkeypatch.delenv("LLMQ_KV_FOLD")
    lb, lo = fold.forward(prompt, 0), ref.forward(prompt, 0)
    assert bits_equal(la, lb) and bits_equal(lb, lo)
    pos = len(prompt)
    for i in range(2):
        nxt = orc.argmax(lo)
        la, lb, lo = plain.forward([nxt], pos), fold.forward([nxt], pos), ref.forward([nxt], pos)
        pos += 1
        assert bits_equal(la, lb), i
        if bits == 4:
            assert bits_equal(lb, lo), i
        else:
            assert np.max(np.abs(lb - lo)) / np.max(np.abs(lo)) < 2e-3 and int(np.argmax(lb)) == orc.argmax(lo), i
    plain.free()
    fold.free()


def test_gpt2_fused_qkv_attention(gpu, orc, weights, monkeypatch):
    """Decode tokens through the fused qkv + attention kernel (a faster form
    for long contexts, whose attention sums run in another order: not the
    default while exact order is on; forced here) against the oracle and the
    two-kernel path, after a 300-token prompt, teacher-forced and on the
    device.  Its bar is the code-flip spread: 2e-3 of max |logit|, top-1."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2, synth

    prompt = synth.prompt_ids(4, 300)
    monkeypatch.setenv("LLMQ_DECODE_FUSION", "1")
    mf = lm.GPT2(ctx, weights)
    monkeypatch.setenv("LLMQ_DECODE_FUSION", "0")
    mu = lm.GPT2(ctx, weights)
    ref = orc.GPT2(gpt2.params_list(weights))
    print("fused prefill", flush=True)
    lf, lu, lo = mf.forward(prompt, 0), mu.forward(prompt, 0), ref.forward(prompt, 0)
    assert bits_equal(lu, lo) and bits_equal(lf, lo)  # the prompt runs the same kernels
    pos, errs, agree, exact = len(prompt), [], 0, 0
    for i in range(8):
        nxt = orc.argmax(lo)
        print("fused decode step", i, flush=True)
        lf, lu, lo = mf.forward([nxt], pos), mu.forward([nxt], pos), ref.forward([nxt], pos)
        pos += 1
        errs.append(np.max(np.abs(lf - lo)) / np.max(np.abs(lo)))
        agree += int(np.argmax(lf) == orc.argmax(lo))
        exact += int(bits_equal(lu, lo))
    print("fused max rel err", max(errs), "top-1", agree, "/ 8; two-kernel bit-exact", exact, "/ 8", flush=True)
    assert max(errs) < 2e-3 and agree >= 7 and exact == 8
    tf, _, _ = mf.generate(prompt, 12)
    tu, _, _ = mu.generate(prompt, 12)
    n = min(len(tf), len(tu))
    assert next((i for i in range(n) if tf[i] != tu[i]), n) >= n - 2, (tf.tolist(), tu.tolist())
    mf.free()
    mu.free()


def test_gpt2_int4_same_head_exact(gpu, orc, weights):
    """--dtype int4-g32-a16 --head same (run[W, W], gpt2t.mojo:1289-1290):
    the head is a BLOCKED int4-g32 matrix, whose exact GEMV leaves the argmax
    partials the device-driven loop picks from.  Teacher-forced logits are
    bit-identical to the oracle's with the same head, and the device's
    greedy tokens are the oracle's."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2, synth

    print("gpt2 int4 head: load", flush=True)
    model = lm.GPT2(ctx, weights, dtype="int4-g32-a16", head="same")
    assert model.name() == "int4-g32-a16+kv-int8"
    ref = orc.GPT2(gpt2.params_list(weights), head=(4, 32, False, True))
    prompt = [int(v) for v in synth.prompt_ids(2024, 12)]
    lg, lo = model.forward(prompt, 0), ref.forward(prompt, 0)
    exact = [bits_equal(lg, lo)]
    toks, pos = [], len(prompt)
    for i in range(39):
        nxt = orc.argmax(lo)
        toks.append(nxt)
        lg, lo = model.forward([nxt], pos), ref.forward([nxt], pos)
        pos += 1
        exact.append(bits_equal(lg, lo))
    toks.append(orc.argmax(lo))
    print(f"gpt2 int4 head: {sum(exact)} / {len(exact)} steps bit-identical", flush=True)
    assert all(exact)
    gen, _, _ = model.generate(prompt, 40)
    want = toks[:next((i for i, t in enumerate(toks) if t == 50256), len(toks))]
    assert gen.tolist() == want
    model.free()
