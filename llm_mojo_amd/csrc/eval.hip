// The evaluation harness's per-position scoring (score_rows,
// gpt2t.mojo:1040-1095): for each window row r, whose logits predict
// targets[r],
//   NLL      = logsumexp(logits) - logits[target]
// and with a baseline's logits (compare mode)
//   NLL_BASE = the same under the baseline,
//   AGREE    = 1 if both top-1 predictions (first maximum) are equal,
//   KL       = sum_v p_base(v) (log p_base(v) - log p(v)),
//   DIFF_MAX / DIFF_SUM = max / sum of |logit difference|.
// logsumexp is the reference's: the row maximum, then sum exp(l - max) in
// float32 accumulated in float64.  One workgroup per row; the sums are over
// 50257 values in a different order than the reference's loop (float64, so
// the results agree to ~1e-12 relative).
#include "common.h"

namespace {

constexpr int kThreads = 256;

template <typename T, typename Op>
__device__ T block_reduce(T v, T *red, Op op) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o));
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    T r = red[0];
    for (int i = 1; i < kThreads / 64; i++) r = op(r, red[i]);
    return r;
}

// First maximum of a row: (value, index), ties to the lower index.
struct Best {
    float v;
    int i;
};
__device__ __forceinline__ Best better(Best a, Best b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

template <bool COMPARE>
__global__ __launch_bounds__(kThreads) void score_rows_kernel(const float *__restrict__ logits,
                                                              const float *__restrict__ base,
                                                              const int64_t *__restrict__ targets, int r0, int V,
                                                              double *__restrict__ stats, int64_t ld) {
    __shared__ double redd[kThreads / 64];
    __shared__ float redi_v[kThreads / 64];
    __shared__ int redi_i[kThreads / 64];
    const int r = r0 + blockIdx.x, tid = threadIdx.x;
    const float *lm = logits + (int64_t)r * V;
    const float *lb = COMPARE ? base + (int64_t)r * V : nullptr;
    auto max_op = [](double a, double b) { return fmax(a, b); };
    auto add_op = [](double a, double b) { return a + b; };
    // row maxima and first-maximum positions
    Best bm{-INFINITY, V}, bb{-INFINITY, V};
    for (int v = tid; v < V; v += kThreads) {
        bm = better(bm, Best{lm[v], v});
        if (COMPARE) bb = better(bb, Best{lb[v], v});
    }
    auto best_reduce = [&](Best b) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            Best c{__shfl_xor(b.v, o), __shfl_xor(b.i, o)};
            b = better(b, c);
        }
        const int lane = tid & 63, wid = tid >> 6;
        __syncthreads();
        if (lane == 0) {
            redi_v[wid] = b.v;
            redi_i[wid] = b.i;
        }
        __syncthreads();
        Best out{redi_v[0], redi_i[0]};
        for (int i = 1; i < kThreads / 64; i++) out = better(out, Best{redi_v[i], redi_i[i]});
        return out;
    };
    bm = best_reduce(bm);
    const float mx = bm.v;
    float mxb = 0.0f;
    if (COMPARE) {
        bb = best_reduce(bb);
        mxb = bb.v;
    }
    double s = 0.0, sb = 0.0;
    for (int v = tid; v < V; v += kThreads) {
        s += (double)expf(lm[v] - mx);
        if (COMPARE) sb += (double)expf(lb[v] - mxb);
    }
    s = block_reduce(s, redd, add_op);
    const double lse = (double)mx + log(s);
    const int64_t target = targets[r];
    const bool ok = target >= 0 && target < V;  // an id outside the vocabulary scores NaN
    if (tid == 0) stats[r] = ok ? lse - (double)lm[target] : NAN;  // NLL
    if (!COMPARE) return;
    sb = block_reduce(sb, redd, add_op);
    const double lse_b = (double)mxb + log(sb);
    double kl = 0.0, dsum = 0.0, dmax = 0.0;
    for (int v = tid; v < V; v += kThreads) {
        const double lpb = (double)lb[v] - lse_b;
        kl += exp(lpb) * (lpb - ((double)lm[v] - lse));
        const double d = fabs((double)lm[v] - (double)lb[v]);
        dmax = fmax(dmax, d);
        dsum += d;
    }
    kl = block_reduce(kl, redd, add_op);
    dsum = block_reduce(dsum, redd, add_op);
    dmax = block_reduce(dmax, redd, max_op);
    if (tid == 0) {
        stats[1 * ld + r] = ok ? lse_b - (double)lb[target] : NAN;  // NLL_BASE
        stats[2 * ld + r] = bm.i == bb.i ? 1.0 : 0.0;       // AGREE
        stats[3 * ld + r] = kl;                             // KL
        stats[4 * ld + r] = dmax;                           // DIFF_MAX
        stats[5 * ld + r] = dsum;                           // DIFF_SUM
    }
}

}  // namespace

extern "C" int llmq_score_rows(llmq_ctx *ctx, const float *logits, const float *base, const int64_t *targets, int r0,
                               int r1, int V, double *stats, int64_t ld) {
    LLMQ_REQUIRE(ctx && logits && targets && stats, "score_rows: bad arguments");
    LLMQ_REQUIRE(r0 >= 0 && r1 >= r0 && r1 <= ld && V > 0, "score_rows: rows %d..%d (ld %lld)", r0, r1, (long long)ld);
    if (r1 == r0) return LLMQ_OK;
    if (base)
        hipLaunchKernelGGL(score_rows_kernel<true>, dim3(r1 - r0), dim3(kThreads), 0, ctx->stream, logits, base,
                           targets, r0, V, stats, ld);
    else
        hipLaunchKernelGGL(score_rows_kernel<false>, dim3(r1 - r0), dim3(kThreads), 0, ctx->stream, logits, base,
                           targets, r0, V, stats, ld);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
