"""IntAttnKV (int_attention.mojo) on the GPU against the CPU oracle.

The cache store and the attention are integer arithmetic up to one float
step per 256-position segment and a final float multiply, which the kernels
perform in the reference's order, so codes, scales and outputs must match
the oracle bit for bit.  Cases: tests/int_attention_check.mojo's context
lengths and token counts, a 476-token prompt, the last positions of the
cache, head_dim 128, and a cache too long to stage in LDS.  The GPT-2 model
with --attention int is held to the float-attention model's exact bar
(bit-identical logits, no int16 code flips, the device's greedy tokens).
"""
import numpy as np
import pytest

from tests.gpt2_exact import check_decode_exact

pytestmark = pytest.mark.gpu


def note(*a):
    print(*a, flush=True)


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


CASES = [
    # (T, pos0, max_t, n_head, head_dim, spread)
    (1, 0, 1024, 12, 64, 0.5), (5, 0, 1024, 12, 64, 2.0), (1, 15, 1024, 12, 64, 0.5),
    (1, 16, 1024, 12, 64, 2.0), (1, 99, 1024, 12, 64, 0.5), (7, 200, 1024, 12, 64, 2.0),
    (1, 511, 1024, 12, 64, 0.5), (3, 1000, 1024, 12, 64, 2.0), (476, 0, 1024, 12, 64, 1.0),
    (4, 1020, 1024, 12, 64, 1.0), (9, 100, 256, 4, 128, 1.0), (2, 3000, 4096, 2, 64, 1.0),
]


@pytest.mark.parametrize("T,pos0,MT,NH,HS,spread", CASES)
def test_ikv_store_and_attend_bit_exact(gpu, orc, T, pos0, MT, NH, HS, spread):
    torch, lm, ctx = gpu
    C = NH * HS
    NL, layer = 2, 1
    rng = np.random.default_rng(1000 * T + pos0 + HS)
    n = pos0 + T
    qkv_all = np.concatenate([rng.normal(0, spread, (n, 2 * C)), rng.normal(0, 1, (n, C))], 1).astype(np.float32)
    qkv_all[min(3, n - 1), C:C + HS] = 0.0  # an all-zero key head: scale 1
    note("ikv store/attend", T, pos0, MT, NH, HS, spread)
    kv = lm.IntAttnKV(ctx, NL, MT, NH, HS)
    okv = orc.IntAttnKV(NL, MT, NH, HS)
    if pos0:
        kv.store(layer, 0, dev(torch, qkv_all[:pos0]))
    q1 = dev(torch, qkv_all[pos0:])
    kv.store(layer, pos0, q1)
    out = torch.zeros((T, C), dtype=torch.float32, device="cuda")
    kv.attend(out, q1, layer, pos0)
    torch.cuda.synchronize()
    for p in range(n):
        okv.store(layer, p, qkv_all[p, C:2 * C], qkv_all[p, 2 * C:])
    k, v, kq, vq = kv.export()
    assert np.array_equal(k, okv.k) and np.array_equal(v, okv.v)
    assert np.array_equal(kq, okv.kq) and np.array_equal(vq, okv.vq)
    want = okv.attend(qkv_all[pos0:], layer, T, pos0)
    got = out.cpu().numpy()
    bad = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
    assert len(bad) == 0, (len(bad), bad[:4].tolist(), got[tuple(bad[0])], want[tuple(bad[0])])


def test_ikv_shape_checks(gpu):
    torch, lm, ctx = gpu
    with pytest.raises(lm.LlmqError, match="max_t % 16"):
        lm.IntAttnKV(ctx, 1, 100, 12, 64)
    with pytest.raises(lm.LlmqError, match="head_dim % 32"):
        lm.IntAttnKV(ctx, 1, 128, 12, 48)
    with pytest.raises(lm.LlmqError, match="head_dim 96"):
        lm.IntAttnKV(ctx, 1, 128, 12, 96)
    kv = lm.IntAttnKV(ctx, 1, 64, 2, 64)
    assert kv.nbytes() == 2 * 64 * 2 * (64 + 4)  # IntAttnKV.nbytes, int_attention.mojo:272-274
    with pytest.raises(lm.LlmqError, match="integer scales"):
        lm.QuantKV8.export(kv)


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
    note("gpt2 int attention: load")
    model = lm.GPT2(ctx, weights, attention="int")
    assert model.name().endswith("+kv-int8-intattn")
    ref = orc.GPT2(gpt2.params_list(weights), attention="int")
    yield model, ref
    model.free()


@pytest.mark.parametrize("seed", range(PROMPTS))
def test_gpt2_int_attention_exact(gpu, orc, models, seed):
    """GPT-2 int4-g32-a16 with --attention int (run_with[..., IntAttnKV],
    gpt2t.mojo:1251-1257; int_attention.mojo:170-269) held to config 0's
    bar: 12-token prompt, 100 greedy tokens, logits bit-identical at every
    step, zero int16 code flips, device greedy tokens equal."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    model, ref = models
    prompt = [int(v) for v in synth.prompt_ids(1000 + seed, 12)]
    check_decode_exact(torch, orc, model, ref, prompt, 100, f"int attention prompt {seed}")


def test_gpt2_int_attention_long_prompt_exact(gpu, orc, models):
    """The same bar after a 476-token prompt (the README's long-context
    decode), 24 generated tokens: prompt attention and decode attention over
    two 256-position segments."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import synth

    model, ref = models
    prompt = [int(v) for v in synth.prompt_ids(1337, 476)]
    check_decode_exact(torch, orc, model, ref, prompt, 24, "int attention 476-token prompt")
