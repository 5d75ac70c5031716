"""The accuracy harness on the GPU (gpt2t.mojo:448-459, 1016-1201):
forward_all against the oracle's, score_rows against the oracle's, and the
window loop against the same statistics recomputed from forward_all's
logits on the host."""
import numpy as np
import pytest

from tests.gpt2_exact import bits_equal

pytestmark = pytest.mark.gpu


def note(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def weights():
    from llm_mojo_amd import synth

    return synth.gpt2_tensors(seed=1337)


def test_score_rows_matches_oracle(gpu, orc):
    torch, lm, ctx = gpu
    rng = np.random.default_rng(8)
    R, V = 37, 50257
    a = rng.normal(0, 3, (R, V)).astype(np.float32)
    b = (a + rng.normal(0, 0.2, (R, V))).astype(np.float32)
    targets = rng.integers(0, V, R)
    note("score rows")
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    tt = torch.from_numpy(targets).cuda()
    for base in (None, tb):
        st = torch.zeros((6, R), dtype=torch.float64, device="cuda")
        lm.lib().llmq_score_rows(ctx.h, ta.data_ptr(), None if base is None else base.data_ptr(), tt.data_ptr(), 3,
                                 R - 2, V, st.data_ptr(), R)
        torch.cuda.synchronize()
        got = st.cpu().numpy()
        want = orc.score_rows(a, targets, 3, R - 2, base=None if base is None else b)
        # float64 sums of 50257 float32 exps in another order, each exp
        # within an ulp of libm's: ~1e-8 absolute on NLL and KL
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
        assert np.array_equal(got[2], want[2])  # top-1 agreement is exact


@pytest.mark.parametrize("T", [40, 476])
def test_forward_all_matches_oracle(gpu, orc, weights, T):
    """Model.forward_all (gpt2t.mojo:448-459): every row's logits bit for
    bit the oracle's (the prompt's exact GEMMs and attention, LN_f on every
    row, the head as a T-token GEMM in tile_i16's / rows_i16's order), and
    its last row equal to forward's."""
    torch, lm, ctx = gpu
    from llm_mojo_amd import gpt2, synth

    orc.set_threads(16)
    ids = synth.prompt_ids(21, T)
    model = lm.GPT2(ctx, weights)
    ref = orc.GPT2(gpt2.params_list(weights))
    out = torch.zeros((T, 50257), device="cuda")
    note("forward_all", T)
    model.forward_all(ids, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = ref.forward_all(ids)
    rows_equal = int(sum(bits_equal(got[t], want[t]) for t in range(T)))
    rel = np.abs(got - want).max(axis=1) / np.abs(want).max(axis=1)
    note("forward_all", T, "rows bit-identical", rows_equal, "max rel err", rel.max())
    assert rows_equal == T
    # forward's head is the one-token dot_row_i16 (another float order than
    # the T-token GEMM's, in the reference too)
    last = model.forward(ids, 0)
    assert bits_equal(last, ref.forward(ids, 0))
    assert np.abs(last - got[-1]).max() / np.abs(got[-1]).max() < 1e-4
    model.free()


def test_eval_loop_windows(gpu, weights):
    torch, lm, ctx = gpu
    from llm_mojo_amd import evaluate, synth

    ids = synth.prompt_ids(33, 1100)
    m4 = lm.GPT2(ctx, weights)
    m8 = lm.GPT2(ctx, weights, bits=8, group=32)
    note("eval loop")
    res = evaluate.eval_loop(m4, ids, base=m8)
    note(res)
    assert res["scored"] == 1099 and res["windows"] == 2
    # the same numbers from forward_all's logits, scored on the host
    nll, nll_b, agree = 0.0, 0.0, 0
    out = torch.zeros((1024, 50257), device="cuda")
    outb = torch.zeros((1024, 50257), device="cuda")
    for begin, end, r0, r1 in evaluate.windows(len(ids)):
        w = ids[begin:end]
        m4.forward_all(w, out[:end - begin])
        m8.forward_all(w, outb[:end - begin])
        torch.cuda.synchronize()
        lg = out[r0:r1].double()
        lb = outb[r0:r1].double()
        tg = torch.from_numpy(ids[begin + r0 + 1:begin + r1 + 1]).cuda()
        nll += float(-(torch.log_softmax(lg, 1).gather(1, tg[:, None])).sum())
        nll_b += float(-(torch.log_softmax(lb, 1).gather(1, tg[:, None])).sum())
        agree += int((lg.argmax(1) == lb.argmax(1)).sum())
    assert abs(res["mean_nll"] - nll / 1099) < 1e-6
    assert abs(np.log(res["ppl_base"]) - nll_b / 1099) < 1e-6
    assert abs(res["agree"] - agree / 1099) < 1e-9
    assert 0 <= res["mean_kl"] < 1 and res["diff_max"] > 0
    m4.free()
    m8.free()
