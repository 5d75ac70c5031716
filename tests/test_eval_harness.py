"""The accuracy harness (gpt2t.mojo:1016-1201) on the CPU: the oracle's
score_rows against float64 closed forms (log-softmax NLL, KL of the two
softmaxes, top-1 with first-maximum ties), and the window bookkeeping of
eval_loop against brute force."""
import numpy as np
import pytest

from llm_mojo_amd import evaluate


def closed_form(lm, lb, targets):
    def log_softmax(x):
        x = x.astype(np.float64)
        m = x.max(axis=1, keepdims=True)
        return x - m - np.log(np.exp(x - m).sum(axis=1, keepdims=True))

    lp, lpb = log_softmax(lm), log_softmax(lb)
    r = np.arange(len(lm))
    return np.stack([-lp[r, targets], -lpb[r, targets], (lm.argmax(1) == lb.argmax(1)).astype(float),
                     (np.exp(lpb) * (lpb - lp)).sum(1), np.abs(lm.astype(np.float64) - lb).max(1),
                     np.abs(lm.astype(np.float64) - lb).sum(1)])


def test_score_rows_closed_form(orc):
    rng = np.random.default_rng(4)
    R, V = 9, 5003
    lm = rng.normal(0, 3, (R, V)).astype(np.float32)
    lb = (lm + rng.normal(0, 0.3, (R, V))).astype(np.float32)
    lm[2, 17] = lm[2, 40] = lm[2].max() + 1  # a tie: the first maximum counts
    lb[2, 40] = lb[2].max() + 1
    targets = rng.integers(0, V, R)
    st = orc.score_rows(lm, targets, 1, R - 1, base=lb)
    want = closed_form(lm, lb, targets)
    assert np.all(st[:, 0] == 0) and np.all(st[:, R - 1] == 0)
    # log_sum_exp takes exp in float32 (gpt2t.mojo:1035): ~6e-8 relative per
    # term, so NLL and KL agree with float64 to ~1e-8 absolute
    np.testing.assert_allclose(st[:, 1:R - 1], want[:, 1:R - 1], rtol=1e-6, atol=1e-7)
    assert st[2, 2] == 0.0  # model picks 17 (first maximum), base picks 40
    only = orc.score_rows(lm, targets, 0, R)
    np.testing.assert_allclose(only[0], want[0], rtol=1e-6, atol=1e-7)
    assert np.all(only[1:] == 0)


@pytest.mark.parametrize("n", [2, 100, 1024, 1025, 1536, 1537, 5000])
def test_windows_score_each_token_once(n):
    seen = np.zeros(n, int)
    ctx_min = []
    for k, (begin, end, r0, r1) in enumerate(evaluate.windows(n)):
        assert begin == 512 * k and end == min(begin + 1024, n)
        for r in range(r0, r1):
            seen[begin + r + 1] += 1  # row r predicts ids[begin + r + 1]
            if k:
                ctx_min.append(r + 1)  # tokens of context before the target
    assert seen[0] == 0 and np.all(seen[1:] == 1)
    assert not ctx_min or min(ctx_min) >= 1024 - 512
