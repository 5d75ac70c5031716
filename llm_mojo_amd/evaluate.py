"""The accuracy harness (gpt2t.mojo:1016-1201): perplexity over sliding
windows, and with a baseline model, top-1 agreement, KL and logit
differences position by position.

Windows are EVAL_WINDOW tokens long and start every EVAL_STRIDE tokens; each
token after the first is scored once, in the first window where it is not
yet scored (eval_loop, gpt2t.mojo:1098-1185).  A window runs
Model.forward_all on the device (logits [T, V] stay in HBM) and score_rows
on the device; only the six per-row float64 statistics come back.  The
reference's baseline is its float32 DenseMatrix model, which this build does
not have: `base` is any second model with forward_all (for example another
weight format).  Tokenization is out of scope: ids are given.
"""
import ctypes

import numpy as np

from ._lib import DeviceBuffer, check, lib

EVAL_WINDOW, EVAL_STRIDE = 1024, 512
NLL, NLL_BASE, AGREE, KL, DIFF_MAX, DIFF_SUM, N_STATS = range(7)
V = 50257


def windows(n, window=EVAL_WINDOW, stride=EVAL_STRIDE):
    """eval_loop's windows over n ids: (begin, end, r0, r1), rows r0..r1-1 of
    window [begin, end) scored (row r predicts ids[begin + r + 1])."""
    out, scored_until, begin = [], 0, 0
    while True:
        end = min(begin + window, n)
        r0, r1 = max(0, scored_until - begin), end - begin - 1
        out.append((begin, end, r0, r1))
        scored_until = end - 1
        if end == n:
            return out
        begin += stride


def eval_loop(model, ids, base=None, window=EVAL_WINDOW, stride=EVAL_STRIDE):
    """Scores every token of ids after the first; returns the totals the
    reference prints (perplexity, mean NLL, and with base: the base's
    perplexity, top-1 agreement, mean KL(base || model), mean and max
    |logit difference|)."""
    ids = np.ascontiguousarray(ids, np.int64)
    n = len(ids)
    if n < 2:
        raise ValueError("need at least 2 tokens")
    ctx = model.ctx
    logits = DeviceBuffer(ctx, window * V * 4)
    blog = DeviceBuffer(ctx, window * V * 4) if base is not None else None
    stats = DeviceBuffer(ctx, N_STATS * window * 8)
    tgt = DeviceBuffer(ctx, window * 8)
    totals = np.zeros(N_STATS)
    diff_max, scored, nwin = 0.0, 0, 0
    host = np.zeros((N_STATS, window))
    for begin, end, r0, r1 in windows(n, window, stride):
        w = ids[begin:end]
        targets = np.zeros(window, np.int64)
        targets[:end - begin - 1] = ids[begin + 1:end]
        tgt.upload(targets)
        model.forward_all(w, logits.ptr)
        if base is not None:
            base.forward_all(w, blog.ptr)
        check(lib().llmq_score_rows(ctx.h, logits.ptr, blog.ptr if blog else None, tgt.ptr, r0, r1, V, stats.ptr,
                                    window))
        stats.download(host)
        rows = host[:, r0:r1]
        totals += rows.sum(axis=1) if base is not None else np.array([rows[0].sum()] + [0.0] * (N_STATS - 1))
        if base is not None and r1 > r0:
            diff_max = max(diff_max, rows[DIFF_MAX].max())
        scored += r1 - r0
        nwin += 1
    for b in (logits, blog, stats, tgt):
        if b is not None:
            b.free()
    cnt = float(scored)
    out = {"scored": scored, "windows": nwin, "ppl": float(np.exp(totals[NLL] / cnt)),
           "mean_nll": totals[NLL] / cnt}
    if base is not None:
        ppl_b = float(np.exp(totals[NLL_BASE] / cnt))
        out.update(ppl_base=ppl_b, ppl_change_pct=(out["ppl"] / ppl_b - 1) * 100, agree=totals[AGREE] / cnt,
                   mean_kl=totals[KL] / cnt, diff_mean=totals[DIFF_SUM] / (cnt * V), diff_max=diff_max)
    return out
