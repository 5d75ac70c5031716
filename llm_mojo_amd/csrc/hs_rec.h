// The "h16s" activation record of the several-token Q4_K matmul
// (gguf_gemm16.hip) and its writer, shared by the kernels that produce one.
#pragma once
#include "common.h"

namespace {

// The "h16s" record, which the batch-decode chain's matmul epilogues write:
// the h16 record with a scale per half sub-block (16 inputs) of a token
// instead of one per superblock, so that a workgroup owning 16 consecutive
// outputs of one matmul writes its part of the next one's input.  Per token
// and half h (inputs 16h .. 16h + 15) a power of two s_h = 2^e_h with
// max |x s_h| < 2^10; the planes hold x s_h as hi / lo in the h16 layout;
//   sums  fp16 [T16 / 16][NSB][4 groups][16 tokens][8]: groups 0 and 1 the
//         hi of s_h X_h for the superblock's halves 0..7 and 8..15, groups
//         2 and 3 their lo (X_h the half's sum of x);
//   exps  int8 [T16 / 16][NSB][16 tokens][16]: e_h;
//   ssq   float [T16][K / 16]: the half's sum of x^2, for an RMSNorm of the
//         row that the reading matmul applies to its outputs (a factor per
//         token: W (x r g) = r W (x g)).
// The reader brings each superblock of a token to the common scale 2^c,
// c = min e_h (its largest half's), multiplying each half's planes and sums
// by 2^(c - e_h) in fp16: exact wherever the products stay normal, and then
// equal to the h16 record's x 2^c.
struct HSRec {
    uint8_t *planes;
    _Float16 *sums;
    int8_t *exps;
    float *ssq;
    int KB, NSB, NH;
};

inline HSRec hs_parts(void *rec, int64_t T, int64_t K) {
    const int64_t T16 = (T + 15) / 16 * 16, KB = K / 32, NSB = K / 256;
    uint8_t *p = static_cast<uint8_t *>(rec);
    HSRec r{};
    if (!p) return r;
    r.planes = p;
    r.sums = reinterpret_cast<_Float16 *>(p + T16 * KB * 128);
    r.exps = reinterpret_cast<int8_t *>(p + T16 * KB * 128 + T16 * NSB * 64);
    r.ssq = reinterpret_cast<float *>(p + T16 * KB * 128 + T16 * NSB * 80);
    r.KB = (int)KB;
    r.NSB = (int)NSB;
    r.NH = (int)(K / 16);
    return r;
}

// Every lane of a 16-lane row gets the row's maximum / sum (the same bits
// in each lane: the pairings are symmetric).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, llmq_dppf<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, llmq_dppf<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, llmq_dppf<0x141>(v));  // row_half_mirror
    return fmaxf(v, llmq_dppf<0x140>(v));  // row_mirror
}
__device__ __forceinline__ float row16_sum(float v) {
    v = v + llmq_dppf<0xB1>(v);
    v = v + llmq_dppf<0x4E>(v);
    v = v + llmq_dppf<0x141>(v);
    return v + llmq_dppf<0x140>(v);
}

// Half hb (inputs 16 hb .. 16 hb + 15) of token t of an h16s record, by the
// 16 lanes of a row of the wave, lane i % 16 holding input 16 hb + i % 16
// in v; with o.ssq, the half's sum of xn^2 goes there (xn: the row before
// the RMSNorm gain that v carries).
__device__ __forceinline__ void hs_store_half(const HSRec &o, int t, int hb, float v, float xn) {
    const int i = threadIdx.x & 15;
    const float m = row16_max(fabsf(v));
    int ex = 0;
    frexpf(m, &ex);  // m < 2^ex
    const int e = min(126, max(-126, 10 - ex));
    const float s = ldexpf(1.0f, e);
    const float xs = v * s, X = row16_sum(v) * s;
    const float sq = o.ssq ? row16_sum(xn * xn) : 0.0f;
    const _Float16 hi = (_Float16)xs, lo = (_Float16)(xs - (float)hi);
    const _Float16 shi = (_Float16)X, slo = (_Float16)(X - (float)shi);
    const int64_t tt = t >> 4, c = t & 15;
    const int j = hb >> 1, kk = (hb & 1) * 16 + i, g = kk >> 3, ii = kk & 7;
    const int pos = (ii & 1) ? 4 + (ii >> 1) : (ii >> 1);
    _Float16 *p = reinterpret_cast<_Float16 *>(o.planes) + ((tt * o.KB + j) * 1024 + (g * 16 + c) * 8 + pos);
    p[0] = hi;
    p[512] = lo;
    if (i == 0) {
        const int sb = hb >> 4, hs = hb & 15;
        _Float16 *ps = o.sums + ((tt * o.NSB + sb) * 4 + (hs >> 3)) * 128 + c * 8 + (hs & 7);
        ps[0] = shi;
        ps[256] = slo;
        o.exps[((tt * o.NSB + sb) * 16 + c) * 16 + hs] = (int8_t)e;
        if (o.ssq) o.ssq[t * (int64_t)o.NH + hb] = sq;
    }
}

}  // namespace
