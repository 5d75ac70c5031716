// QuantKV[8] store and float attention over the int8 cache
// (kvcache.mojo:248-385, attend_float_one 113-150), LayerNorm
// (kernels.mojo:179-197) and the token embedding with the greedy argmax of
// the previous step (gpt2t.mojo:378-385, 495-502, 792-797).
#include "common.h"

namespace {

// max over the wave (order-free, so exact in any pairing), without LDS
__device__ __forceinline__ float wave_max(float v) { return llmq_wave_max_all(v); }

// QuantKV.store (kvcache.mojo:333-342) for token t = blockIdx.y, head h =
// blockIdx.x: per head s = max|x| / 127 (1 if zero), codes round(x / s).
// One wave per (token, head); head_dim is a multiple of 64.
__global__ __launch_bounds__(64) void kv_store_kernel(const float *__restrict__ qkv, int64_t ld, int C, int pos0,
                                                      const int *__restrict__ pos_dev, int layer, int max_t,
                                                      int n_head, int hd, int8_t *__restrict__ K8,
                                                      int8_t *__restrict__ V8, float *__restrict__ KS,
                                                      float *__restrict__ VS) {
    const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos = (pos_dev ? *pos_dev : pos0) + t;
    const int64_t sl = ((int64_t)layer * max_t + pos) * n_head + h;
    for (int kv = 0; kv < 2; kv++) {
        const float *src = qkv + (int64_t)t * ld + (int64_t)(1 + kv) * C + (int64_t)h * hd;
        float m = 0.0f;
        for (int i = lane; i < hd; i += 64) m = fmaxf(m, fabsf(src[i]));
        m = wave_max(m);
        float s = m / 127.0f;
        if (s == 0.0f) s = 1.0f;
        const float inv = 1.0f / s;
        int8_t *dst = (kv ? V8 : K8) + sl * hd;
        for (int i = lane; i < hd; i += 64) dst[i] = (int8_t)llmq_to_int(roundf(src[i] * inv));
        if (lane == 0) (kv ? VS : KS)[sl] = s;
    }
}

// attend_float_one (kvcache.mojo:113-150) through QuantKV.score / add_value
// (344-370) for token t = blockIdx.y (position pos0 + t), head h = blockIdx.x.
// Scores: q . k over head_dim, times the key's scale, times 1/sqrt(hd); softmax
// with the running maximum; out = sum_s (p_s * vs_s) * v_s, every float
// operation in the reference's order: the score's 16 lane partials and
// halving tree, the total added position by position, and each output
// dimension's fma chain over positions (one thread per dimension).
//
// The thread that scores position s also copies that position's value row
// and scale into LDS (STAGE), so the value pass reads no global memory.  With
// STORE (one token per launch: decode) the workgroup first quantizes its
// head's new key and value (QuantKV.store, kvcache.mojo:333-342), writes them
// to the cache, and uses them from LDS for the current position.
constexpr int kAttnThreads = 256;
typedef int v4i __attribute__((ext_vector_type(4)));

// Workgroup barrier ordering LDS only (global loads stay in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int HD, bool STAGE, bool STORE>
__global__ __launch_bounds__(kAttnThreads) void kv_attend_kernel(const float *__restrict__ qkv, int64_t ld, int C,
                                                                 int pos0, const int *__restrict__ pos_dev,
                                                                 int layer, int max_t, int n_head,
                                                                 int8_t *__restrict__ K8, int8_t *__restrict__ V8,
                                                                 float *__restrict__ KS, float *__restrict__ VS,
                                                                 float *__restrict__ out, int64_t ldo) {
    constexpr int NV = HD / 16;  // 16-byte pieces of a row
    extern __shared__ __align__(16) float sm[];
    float *q = sm;                // [HD]
    float *scores = q + HD;       // [max_t]
    float *vsc = scores + max_t;  // [max_t]  value scales (STAGE)
    // [max_t][HD] value codes (STAGE), 16-byte aligned for the int4 copies
    int8_t *vrow = reinterpret_cast<int8_t *>((reinterpret_cast<uintptr_t>(vsc + max_t) + 15) & ~(uintptr_t)15);
    __shared__ float red[kAttnThreads];
    __shared__ __align__(16) int8_t knew[HD], vnew[HD];
    __shared__ float kscale_new, vscale_new;
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int npos = (pos_dev ? *pos_dev : pos0) + t + 1;
    const int cur = npos - 1;
    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t base = (int64_t)layer * max_t * n_head + h;  // slot of position 0

    // The rows of this thread's first position, requested before anything
    // else (positions past the end re-read the last one and are not used).
    v4i kr[NV], vr[NV];  // native vectors: HIP's int4 struct copies kept vr in scratch
    float ksr, vsr;
    auto load_row = [&](int s) {
        const int64_t sl = base + (int64_t)s * n_head;
        const v4i *kp = reinterpret_cast<const v4i *>(K8 + sl * HD);
        const v4i *vp = reinterpret_cast<const v4i *>(V8 + sl * HD);
#pragma unroll
        for (int i = 0; i < NV; i++) {
            kr[i] = kp[i];
            if (STAGE) vr[i] = vp[i];
        }
        ksr = KS[sl];
        if (STAGE) vsr = VS[sl];
    };
    load_row(tid < npos ? tid : cur);
    __builtin_amdgcn_sched_barrier(0);

    for (int i = tid; i < HD; i += kAttnThreads) q[i] = qkv[(int64_t)t * ld + (int64_t)h * HD + i];
    if (STORE && (wid == 1 || wid == 2)) {
        // QuantKV.store for this head (kvcache.mojo:320-342)
        const int kv = wid - 1;
        const float *src = qkv + (int64_t)t * ld + (int64_t)(1 + kv) * C + (int64_t)h * HD;
        float xs[HD / 64];
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < HD / 64; e++) {
            xs[e] = src[lane + 64 * e];
            m = fmaxf(m, fabsf(xs[e]));
        }
        m = wave_max(m);
        float sc = m / 127.0f;
        if (sc == 0.0f) sc = 1.0f;
        const float inv = 1.0f / sc;
        const int64_t sl = base + (int64_t)cur * n_head;
#pragma unroll
        for (int e = 0; e < HD / 64; e++) {
            const int i = lane + 64 * e;
            const int8_t code = (int8_t)llmq_to_int(roundf(xs[e] * inv));
            (kv ? V8 : K8)[sl * HD + i] = code;
            // LDS copies: the workgroup reads the new rows from there, not
            // back from global memory.
            if (kv == 0)
                knew[i] = code;
            else if (STAGE)
                vrow[(int64_t)cur * HD + i] = code;
            else
                vnew[i] = code;
        }
        if (lane == 0) {
            (kv ? VS : KS)[sl] = sc;
            if (kv == 0)
                kscale_new = sc;
            else if (STAGE)
                vsc[cur] = sc;
            else
                vscale_new = sc;
        }
    }
    lds_barrier();

    float mx = -INFINITY;
    for (int s = tid; s < npos; s += kAttnThreads) {
        if (s != tid) load_row(s);  // only past 256 positions
        const bool fresh = STORE && s == cur;
        if (fresh) {
#pragma unroll
            for (int i = 0; i < NV; i++) kr[i] = *reinterpret_cast<const v4i *>(knew + 16 * i);
            ksr = kscale_new;
        }
        // QuantKV.score (kvcache.mojo:344-353): 16 lanes d_l += q[16 i + l] *
        // f32(k[16 i + l]) (multiply, then add), reduce_add, times the key's
        // scale; then times 1 / sqrt(HD) (attend_float_one, 122-124).
        float dl[16];
#pragma unroll
        for (int e = 0; e < 16; e++) dl[e] = 0.0f;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const int8_t *b = reinterpret_cast<const int8_t *>(&kr[i]);
#pragma unroll
            for (int e = 0; e < 16; e++) dl[e] = dl[e] + q[16 * i + e] * (float)b[e];
        }
#pragma unroll
        for (int e = 0; e < 8; e++) dl[e] = dl[e] + dl[e + 8];
#pragma unroll
        for (int e = 0; e < 4; e++) dl[e] = dl[e] + dl[e + 4];
        dl[0] = dl[0] + dl[2];
        dl[1] = dl[1] + dl[3];
        const float d = dl[0] + dl[1];
        if (STAGE && !fresh) {
#pragma unroll
            for (int i = 0; i < NV; i++) *reinterpret_cast<v4i *>(vrow + (int64_t)s * HD + 16 * i) = vr[i];
            vsc[s] = vsr;
        }
        const float sc = (d * ksr) * scale;
        scores[s] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    lds_barrier();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int s = tid; s < npos; s += kAttnThreads) scores[s] = ref_expf(scores[s] - mx);
    lds_barrier();
    auto vscale = [&](int s) -> float {
        if (STAGE) return vsc[s];
        if (STORE && s == cur) return vscale_new;
        return VS[base + (int64_t)s * n_head];
    };
    // The total in position order (attend_float_one, 139-141): 16 scores per
    // batch of LDS reads, then their adds in order.
    auto total_of = [&]() -> float {
        float t = 0.0f;
        int s = 0;
        for (; s + 16 <= npos; s += 16) {
            float e[16];
#pragma unroll
            for (int k = 0; k < 16; k++) e[k] = scores[s + k];
#pragma unroll
            for (int k = 0; k < 16; k++) t += e[k];
        }
        for (; s < npos; s++) t += scores[s];
        return t;
    };
    // out[i] = acc_i, acc_i = fma(w_s, f32(v_s[i]), acc_i) over positions in
    // order (add_value, 367-370), w_s = (e_s / total) * vs_s: one lane per
    // dimension.
    auto value_chain = [&](int i) -> float {
        auto value = [&](int s) -> int8_t {
            if (STAGE) return vrow[(int64_t)s * HD + i];
            if (STORE && s == cur) return vnew[i];
            return V8[(base + (int64_t)s * n_head) * HD + i];
        };
        float acc = 0.0f;
        int s = 0;
        for (; s + 8 <= npos; s += 8) {  // a batch's loads, then its fma chain
            float w[8];
            int8_t v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                w[k] = scores[s + k];
                v[k] = value(s + k);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) acc = fmaf(w[k], (float)v[k], acc);
        }
        for (; s < npos; s++) acc = fmaf(scores[s], (float)value(s), acc);
        return acc;
    };
    if constexpr (HD == 64) {
        // One wave finishes: every lane forms the same total, the lanes then
        // turn positions lane, lane + 64, ... into weights, and run the 64
        // value chains (LDS operations of a wave complete in order).
        if (wid == 0) {
            const float total = total_of();
            for (int s = lane; s < npos; s += 64) scores[s] = (scores[s] / total) * vscale(s);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
            out[(int64_t)t * ldo + (int64_t)h * HD + lane] = value_chain(lane);
        }
    } else {
        if (tid == 0) red[0] = total_of();
        lds_barrier();
        const float total = red[0];
        for (int s = tid; s < npos; s += kAttnThreads) scores[s] = (scores[s] / total) * vscale(s);
        lds_barrier();
        if (tid < HD) out[(int64_t)t * ldo + (int64_t)h * HD + tid] = value_chain(tid);
    }
}

// Prompt attention in the reference's order (KVCache.attend calls
// attend_float_one for every token and head, kvcache.mojo:62-79, 113-150),
// the arithmetic of kv_attend_kernel operation by operation, for TQ tokens
// of one head per workgroup of NTH threads, which share the staged key and
// value rows (head_dim 64; the cache already holds every token of the
// prompt).  Workgroup y takes block nblk - 1 - y, then block y, so every
// workgroup has about the same causal work.  Per block:
//  1. keys staged NTH / 4 positions at a time as floats; lane (i = lane % TQ,
//     p = lane / TQ) of wave w scores token i, its query in registers,
//     against position (st NW + w) PW + p of the chunk (16 lane partials,
//     halving tree, times the key's scale, times 1/sqrt(64));
//  2. per token (NTH / TQ threads): maximum, exponentials, the total added
//     in position order by one lane, the weights (e / total) * vs;
//  3. per token and dimension the fma chain over positions in order, values
//     staged as floats: with 16 tokens and SV, 256 threads each run four
//     chains, tokens j and j + 8 times dimensions 2 d and 2 d + 1 (one read
//     of a value pair for two tokens); else 64 TQ / NTH dimensions of one
//     token a thread.
// One wave issues a VALU instruction every ~6 cycles, so the larger
// workgroup (two waves a SIMD) is the faster one.
constexpr int kKStr = 68;  // floats per staged key row (bank spread)

template <int NTH, int TQ, bool SV>
__global__ __launch_bounds__(NTH) void attend_prompt_exact_kernel(const float *__restrict__ qkv, int64_t ld, int pos0,
                                                                  int T, int layer, int max_t, int n_head,
                                                                  const int8_t *__restrict__ K8,
                                                                  const int8_t *__restrict__ V8,
                                                                  const float *__restrict__ KS,
                                                                  const float *__restrict__ VS, float *__restrict__ out,
                                                                  int64_t ldo, int NP) {
    constexpr int HD = 64, NW = NTH / 64, PW = 64 / TQ, TPT = NTH / TQ, DPT = HD / TPT, PC = NTH / 4;
    static_assert(DPT >= 1 && DPT <= 4 && TPT <= 64, "shape");
    extern __shared__ __align__(16) float sm[];
    float *kf = sm;              // [PC][kKStr] keys; phase 3: [PC][HD] values
    float *ksc = kf + PC * kKStr; // [PC]
    float *vsc = ksc + PC;        // [NP]
    float *sc = vsc + NP;         // [TQ][NP + 1] scores, then exponentials, then weights
    const int NPS = NP + 1;       // rows of different tokens on different banks
    const int h = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t base = (int64_t)layer * max_t * n_head + h;  // slot of position 0
    const float scale = 1.0f / sqrtf((float)HD);
    const int nblk = (T + TQ - 1) / TQ;
    for (int pass = 0; pass < 2; pass++) {
        const int blk = pass == 0 ? nblk - 1 - (int)blockIdx.y : (int)blockIdx.y;
        if (pass == 1 && blk >= nblk - 1 - (int)blockIdx.y) break;  // the middle block, done once
        if (pass == 1) lds_barrier();  // the first block's reads of LDS are done
        const int t0 = blk * TQ;
        const int npb = pos0 + (t0 + TQ < T ? t0 + TQ : T);  // positions the block reads

        // 16 codes of position c0 + (tid >> 2) (keys: with the key and value
        // scales): fetched into registers one chunk ahead, then committed to
        // LDS as floats
        int4 raw = make_int4(0, 0, 0, 0);
        float rks = 0.0f, rvs = 0.0f;
        auto fetch = [&](const int8_t *src, int c0, bool keys) {
            const int sl = tid >> 2, pc = tid & 3, s = c0 + sl;
            if (s < npb) {
                const int64_t slot = base + (int64_t)s * n_head;
                raw = *reinterpret_cast<const int4 *>(src + slot * HD + pc * 16);
                if (keys && pc == 0) {
                    rks = KS[slot];
                    rvs = VS[slot];
                }
            }
        };
        auto commit = [&](int c0, int stride, bool keys) {
            const int sl = tid >> 2, pc = tid & 3, s = c0 + sl;
            if (s < npb) {
                const int8_t *bb = reinterpret_cast<const int8_t *>(&raw);
                float4 *dst = reinterpret_cast<float4 *>(kf + sl * stride + pc * 16);
#pragma unroll
                for (int k = 0; k < 4; k++)
                    dst[k] = make_float4((float)bb[4 * k], (float)bb[4 * k + 1], (float)bb[4 * k + 2],
                                         (float)bb[4 * k + 3]);
                if (keys && pc == 0) {
                    ksc[sl] = rks;
                    vsc[s] = rvs;
                }
            }
        };
        fetch(K8, 0, true);

        // 1. scores
        const int qi = lane % TQ, qp = lane / TQ;
        const bool qok = t0 + qi < T;
        const int qpos = pos0 + t0 + qi;
        float q[HD];
        {
            const float4 *src =
                reinterpret_cast<const float4 *>(qkv + (int64_t)(qok ? t0 + qi : t0) * ld + (int64_t)h * HD);
#pragma unroll
            for (int k = 0; k < HD / 4; k++) {
                const float4 v = src[k];
                q[4 * k] = v.x;
                q[4 * k + 1] = v.y;
                q[4 * k + 2] = v.z;
                q[4 * k + 3] = v.w;
            }
        }
        for (int c0 = 0; c0 < npb; c0 += PC) {
            commit(c0, kKStr, true);
            lds_barrier();
            if (c0 + PC < npb) fetch(K8, c0 + PC, true);  // in flight while this chunk is scored
#pragma unroll 1
            for (int st = 0; st < PC / (NW * PW); st++) {
                const int sl = (st * NW + w) * PW + qp, s = c0 + sl;
                if (s < npb) {
                    const float4 *kr = reinterpret_cast<const float4 *>(kf + sl * kKStr);
                    float dl[16];
#pragma unroll
                    for (int e = 0; e < 16; e++) dl[e] = 0.0f;
#pragma unroll
                    for (int i = 0; i < HD / 16; i++) {
                        const float4 k0 = kr[4 * i], k1 = kr[4 * i + 1], k2 = kr[4 * i + 2], k3 = kr[4 * i + 3];
                        const float kk[16] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w,
                                              k2.x, k2.y, k2.z, k2.w, k3.x, k3.y, k3.z, k3.w};
#pragma unroll
                        for (int e = 0; e < 16; e++) dl[e] = dl[e] + q[16 * i + e] * kk[e];
                    }
#pragma unroll
                    for (int e = 0; e < 8; e++) dl[e] = dl[e] + dl[e + 8];
#pragma unroll
                    for (int e = 0; e < 4; e++) dl[e] = dl[e] + dl[e + 4];
                    dl[0] = dl[0] + dl[2];
                    dl[1] = dl[1] + dl[3];
                    const float d = dl[0] + dl[1];
                    if (qok && s <= qpos) sc[qi * NPS + s] = (d * ksc[sl]) * scale;
                }
            }
            lds_barrier();
        }

        fetch(V8, 0, false);  // the first value chunk, in flight during step 2

        // 2. per token: maximum, exponentials, total in order, weights
        {
            const int ti = tid / TPT, tl = tid % TPT;
            const bool tok = t0 + ti < T;
            const int tpos = tok ? pos0 + t0 + ti : -1;
            float *row = sc + ti * NPS;
            float mx = -INFINITY;
            for (int s = tl; s <= tpos; s += TPT) mx = fmaxf(mx, row[s]);
#pragma unroll
            for (int off = TPT / 2; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
#pragma unroll 4
            for (int s = tl; s <= tpos; s += TPT) row[s] = ref_expf(row[s] - mx);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
            float total = 0.0f;
            if (tl == 0 && tok) {
                int s = 0;
                for (; s + 16 <= tpos + 1; s += 16) {
                    float e[16];
#pragma unroll
                    for (int k = 0; k < 16; k++) e[k] = row[s + k];
#pragma unroll
                    for (int k = 0; k < 16; k++) total += e[k];
                }
                for (; s <= tpos; s++) total += row[s];
            }
            total = __shfl(total, (lane / TPT) * TPT);
#pragma unroll 4
            for (int s = tl; s <= tpos; s += TPT) row[s] = (row[s] / total) * vsc[s];
        }
        lds_barrier();

        // 3. the value chains
        if constexpr (SV && TQ == 16) {
            // thread (tokens j, j + 8; dimensions 2 d, 2 d + 1), j = tid / 32, d = tid % 32
            const bool act = tid < 256;
            const int ja = (tid >> 5) & 7, jb = ja + 8, dd = 2 * (tid & 31);
            const int pa = act && t0 + ja < T ? pos0 + t0 + ja : -1, pb = act && t0 + jb < T ? pos0 + t0 + jb : -1;
            const float *wa = sc + ja * NPS, *wb = sc + jb * NPS;
            float aa0 = 0.0f, aa1 = 0.0f, ab0 = 0.0f, ab1 = 0.0f;
            for (int c0 = 0; c0 < npb; c0 += PC) {
                commit(c0, HD, false);
                lds_barrier();
                if (c0 + PC < npb) fetch(V8, c0 + PC, false);
                // this chunk's positions of each token (pb >= pa)
                const int ca = pa + 1 - c0 < PC ? pa + 1 - c0 : PC, cb = pb + 1 - c0 < PC ? pb + 1 - c0 : PC;
                int sl = 0;
                for (; sl + 8 <= ca; sl += 8) {  // both tokens: a batch's reads, then the fmas in order
                    float xa[8], xb[8];
                    float2 v[8];
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        xa[k] = wa[c0 + sl + k];
                        xb[k] = wb[c0 + sl + k];
                        v[k] = *reinterpret_cast<const float2 *>(kf + (sl + k) * HD + dd);
                    }
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        aa0 = fmaf(xa[k], v[k].x, aa0);
                        aa1 = fmaf(xa[k], v[k].y, aa1);
                        ab0 = fmaf(xb[k], v[k].x, ab0);
                        ab1 = fmaf(xb[k], v[k].y, ab1);
                    }
                }
                for (; sl < ca; sl++) {
                    const float2 v = *reinterpret_cast<const float2 *>(kf + sl * HD + dd);
                    const float xa = wa[c0 + sl], xb = wb[c0 + sl];
                    aa0 = fmaf(xa, v.x, aa0);
                    aa1 = fmaf(xa, v.y, aa1);
                    ab0 = fmaf(xb, v.x, ab0);
                    ab1 = fmaf(xb, v.y, ab1);
                }
                for (; sl + 8 <= cb; sl += 8) {  // token j + 8's further positions
                    float xb[8];
                    float2 v[8];
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        xb[k] = wb[c0 + sl + k];
                        v[k] = *reinterpret_cast<const float2 *>(kf + (sl + k) * HD + dd);
                    }
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        ab0 = fmaf(xb[k], v[k].x, ab0);
                        ab1 = fmaf(xb[k], v[k].y, ab1);
                    }
                }
                for (; sl < cb; sl++) {
                    const float2 v = *reinterpret_cast<const float2 *>(kf + sl * HD + dd);
                    const float xb = wb[c0 + sl];
                    ab0 = fmaf(xb, v.x, ab0);
                    ab1 = fmaf(xb, v.y, ab1);
                }
                lds_barrier();
            }
            if (pa >= 0) {
                float *o = out + (int64_t)(t0 + ja) * ldo + (int64_t)h * HD + dd;
                o[0] = aa0;
                o[1] = aa1;
            }
            if (pb >= 0) {
                float *o = out + (int64_t)(t0 + jb) * ldo + (int64_t)h * HD + dd;
                o[0] = ab0;
                o[1] = ab1;
            }
        } else {
            // thread (token ti, dimensions DPT dg ..)
            const int ti = tid / TPT, dg = tid % TPT;
            const int ipos = t0 + ti < T ? pos0 + t0 + ti : -1;
            const float *wr = sc + ti * NPS;
            float acc[DPT];
#pragma unroll
            for (int k = 0; k < DPT; k++) acc[k] = 0.0f;
            auto step = [&](float wv, const float *vp) {
#pragma unroll
                for (int k = 0; k < DPT; k++) acc[k] = fmaf(wv, vp[k], acc[k]);
            };
            for (int c0 = 0; c0 < npb; c0 += PC) {
                commit(c0, HD, false);
                lds_barrier();
                if (c0 + PC < npb) fetch(V8, c0 + PC, false);
                const int cn = ipos + 1 - c0 < PC ? ipos + 1 - c0 : PC;  // this token's positions here
                int sl = 0;
                for (; sl + 8 <= cn; sl += 8) {  // a batch's reads, then its fmas in order
                    float wv[8], v[8][DPT];
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        wv[k] = wr[c0 + sl + k];
#pragma unroll
                        for (int m = 0; m < DPT; m++) v[k][m] = kf[(sl + k) * HD + dg * DPT + m];
                    }
#pragma unroll
                    for (int k = 0; k < 8; k++)
#pragma unroll
                        for (int m = 0; m < DPT; m++) acc[m] = fmaf(wv[k], v[k][m], acc[m]);
                }
                for (; sl < cn; sl++) step(wr[c0 + sl], kf + sl * HD + dg * DPT);
                lds_barrier();
            }
            if (ipos >= 0) {
                float *o = out + (int64_t)(t0 + ti) * ldo + (int64_t)h * HD + dg * DPT;
#pragma unroll
                for (int k = 0; k < DPT; k++) o[k] = acc[k];
            }
        }
    }
}

// LayerNorm over rows of C (kernels.mojo:179-197), one workgroup per row,
// with the statistics in the reference's order (16 lane partials, halving
// tree) and the output as (x - mean) * rstd * w + b, each operation rounded.
__global__ __launch_bounds__(256) void layernorm_kernel(float *__restrict__ out, const float *__restrict__ x,
                                                        const float *__restrict__ w, const float *__restrict__ b,
                                                        int64_t C) {
    extern __shared__ float xs[];  // [C]
    __shared__ float bc[2];
    const float *xr = x + (int64_t)blockIdx.x * C;
    float *o = out + (int64_t)blockIdx.x * C;
    const int tid = threadIdx.x;
    for (int64_t i = tid; i < C; i += 256) xs[i] = xr[i];
    llmq_lds_barrier();
    float mean, rstd;
    llmq_ln_stats(xs, (int)C, bc, mean, rstd);
    for (int64_t i = tid; i < C; i += 256) {
        const float nn = (xs[i] - mean) * rstd;
        o[i] = nn * w[i] + b[i];
    }
}

// Embedding rows of E (any QuantMatrix in the row-tile layout), plus wpe.
// In decode mode (parts != nullptr) the token is first picked as the argmax
// over the previous head's per-workgroup partials (ties: smaller index), is
// recorded in gen[step], and state = {pos, step} advances by one.
__global__ __launch_bounds__(256) void embed_kernel(const uint4 *__restrict__ codes,
                                                    const uint16_t *__restrict__ scales,
                                                    const uint8_t *__restrict__ zps, int bits, int64_t CK,
                                                    int64_t NG, int64_t CPG, const float *__restrict__ wpe,
                                                    const int64_t *__restrict__ tokens, int pos0, int C,
                                                    float *__restrict__ x, const ArgmaxPart *__restrict__ parts,
                                                    int nparts, int64_t *__restrict__ gen, int *__restrict__ state,
                                                    int do_embed, int64_t n_rows) {
    __shared__ float bv[4];  // per wave (256 threads)
    __shared__ int bi[4];
    __shared__ int64_t s_tok;
    __shared__ int s_pos;
    const int tid = threadIdx.x, t = blockIdx.x;
    if (parts) {
        float v = -INFINITY;
        int idx = 0x7fffffff;
        // Sixteen partials a thread per round (one round for 4096), all
        // loads issued before the compares; indices past the end re-read
        // the last partial, which cannot change the result.
        for (int p0 = tid; p0 < nparts; p0 += 256 * 16) {
            ArgmaxPart c[16];
#pragma unroll
            for (int k = 0; k < 16; k++) c[k] = parts[min(p0 + 256 * k, nparts - 1)];
#pragma unroll
            for (int k = 0; k < 16; k++)
                if (c[k].v > v || (c[k].v == v && c[k].idx < idx)) {
                    v = c[k].v;
                    idx = c[k].idx;
                }
        }
        // Within each wave by shuffles, then over the four waves in order
        // (the larger value wins, equal values keep the smaller index).
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(v, off);
            const int oi = __shfl_xor(idx, off);
            if (ov > v || (ov == v && oi < idx)) {
                v = ov;
                idx = oi;
            }
        }
        if ((tid & 63) == 0) {
            bv[tid >> 6] = v;
            bi[tid >> 6] = idx;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < 4; w++)
                if (bv[w] > bv[0] || (bv[w] == bv[0] && bi[w] < bi[0])) {
                    bv[0] = bv[w];
                    bi[0] = bi[w];
                }
            const int step = state[1] + 1;
            const int pos = state[0] + 1;
            gen[step] = bi[0];
            state[0] = pos;
            state[1] = step;
            s_tok = bi[0];
            s_pos = pos;
        }
        __syncthreads();
    } else {
        if (tid == 0) {
            s_tok = tokens[t];
            s_pos = pos0 + t;
        }
        __syncthreads();
    }
    if (!do_embed) return;
    // An argmax over logits that are all NaN has no index: embed token 0
    // rather than read outside the table.
    const int64_t row = (s_tok >= 0 && s_tok < n_rows) ? s_tok : 0;
    const int pos = s_pos;
    const int64_t tile = row / LLMQ_TILE_ROWS, r = row % LLMQ_TILE_ROWS;
    const int wpc = bits == 4 ? 32 : 16;
    for (int k = tid; k < C; k += 256) {
        const int64_t c = k / wpc, e = k % wpc;
        const uint8_t *chunk = reinterpret_cast<const uint8_t *>(codes + (tile * CK + c) * LLMQ_TILE_ROWS + r);
        int u = bits == 4 ? ((chunk[e >> 1] >> (4 * (e & 1))) & 15) : chunk[e];
        const int64_t gi = (tile * NG + c / CPG) * LLMQ_TILE_ROWS + r;
        const float s = __half2float(__ushort_as_half(scales[gi]));
        const float v = ((float)u - (float)zps[gi]) * s;  // row_op (tensor.mojo:463-473)
        x[(int64_t)t * C + k] = v + wpe[(int64_t)pos * C + k];
    }
}


// Prompt attention (T > 1, positions known on the host): attend_float_one
// (kvcache.mojo:113-150) for a block of 16 consecutive queries of one head per
// workgroup, causal over the int8 cache after QuantKV.store of the prompt.
// Key and value rows are staged 64 at a time in LDS and shared by the 16
// queries; each query's scores live in LDS (sized by the prompt's last
// position), then the softmax (16-lane DPP reductions) and the value pass in
// position order.  Per element the arithmetic is that of kv_attend_kernel:
// score = (q . k) * ks / sqrt(hd), e = exp(score - max), p = e / total,
// out = sum_s fma(p * vs, v, .).
constexpr int kQB = 16;   // queries per workgroup
constexpr int kPB = 64;   // key / value rows per staged block

template <int CTRL>
__device__ __forceinline__ float dpp_row(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Over each row of 16 lanes; every lane of the row gets the same bits.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_row<0xB1>(v));
    v = fmaxf(v, dpp_row<0x4E>(v));
    v = fmaxf(v, dpp_row<0x141>(v));
    return fmaxf(v, dpp_row<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_row<0xB1>(v);
    v += dpp_row<0x4E>(v);
    v += dpp_row<0x141>(v);
    return v + dpp_row<0x140>(v);
}

typedef float v4f __attribute__((ext_vector_type(4)));

// Prompt attention for one query head and 16 queries on the fp32 matrix cores
// (its key / value head h / group of n_kv cached heads)
// (v_mfma_f32_16x16x4f32; lane l holds A[l % 16][l / 16], B[l / 16][l % 16]
// and D[4 (l / 16) + i][l % 16]).  KVCache.attend over QuantKV[8]
// (kvcache.mojo:62-79, 113-150, 344-370): per query and position
//   score = (sum_d q_d * f32(k_d)) * ks * (1 / sqrt(64)),  causal,
//   e = exp(score - max),  p = e / total,  out = sum_s (p * vs) * f32(v_s)
// with the sums over d and s taken by the matrix cores (float32 products
// and accumulation, in their own order).
//
// Key / value rows are staged 64 at a time.  Scores: wave w takes keys
// 16w..16w+15 of the block; MFMA step t covers dims 16k + t (k = lane / 16),
// so a lane's 16 key bytes are one contiguous 16-byte read.  Values: wave w
// takes dims 16w..16w+15; step t covers block keys 16k + t, so a lane reads
// 16 consecutive weights of its query and 16 consecutive bytes of the
// transposed value block.
template <int HD>
__global__ __launch_bounds__(256) void attend_prompt_kernel(const float *__restrict__ qkv, int64_t ld, int pos0, int T,
                                                            int layer, int max_t, int n_kv, int group,
                                                            const int8_t *__restrict__ K8,
                                                            const int8_t *__restrict__ V8,
                                                            const float *__restrict__ KS,
                                                            const float *__restrict__ VS, float *__restrict__ out,
                                                            int64_t ldo, int LT, int hm) {
    static_assert(HD == 64, "prompt attention: head_dim 64");
    extern __shared__ __align__(16) float smp[];
    float *S = smp;                                      // [kQB][LT] scores, then e
    float *RS = S + kQB * LT;                            // [kPB] row scales of the staged block
    int8_t *R8 = reinterpret_cast<int8_t *>(RS + kPB);   // [kPB][HD] staged key rows / [HD][kPB] value columns
    __shared__ float tot[kQB];
    const int h = blockIdx.x, q0 = blockIdx.y * kQB, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, c16 = lane & 15, k4 = lane >> 4;
    const int nq = min(kQB, T - q0);
    const int npos = pos0 + q0 + nq;  // positions any query of the block sees
    const float scale = 1.0f / sqrtf((float)HD);
    // the query head's key / value head: its position 0 and position stride (rows)
    const int64_t base = hm ? ((int64_t)layer * n_kv + h / group) * max_t : (int64_t)layer * max_t * n_kv + h / group;
    const int64_t pstr = hm ? 1 : n_kv;

    // A operand of the scores: query c16, dims 16 k4 + t
    float qa[16];
    {
        const float *qr = qkv + (int64_t)(q0 + c16) * ld + (int64_t)h * HD + 16 * k4;
#pragma unroll
        for (int t = 0; t < 16; t += 4) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (c16 < nq) v = *reinterpret_cast<const float4 *>(qr + t);
            qa[t] = v.x;
            qa[t + 1] = v.y;
            qa[t + 2] = v.z;
            qa[t + 3] = v.w;
        }
    }
    // One 16-byte piece of row s0 + row (64 rows x 4 pieces) and the row scale.
    auto load_piece = [&](const int8_t *src, const float *sc, int s0, int4 &v, float &f) {
        const int row = tid >> 2, piece = tid & 3;
        const int s = s0 + row;
        v = make_int4(0, 0, 0, 0);
        f = 0.0f;
        if (s < npos) {
            const int64_t sl = base + (int64_t)s * pstr;
            v = *reinterpret_cast<const int4 *>(src + sl * HD + 16 * piece);
            f = sc[sl];
        }
    };
    // Scores.
    for (int s0 = 0; s0 < npos; s0 += kPB) {
        int4 v;
        float f;
        load_piece(K8, KS, s0, v, f);
        __syncthreads();
        *reinterpret_cast<int4 *>(R8 + (tid >> 2) * HD + 16 * (tid & 3)) = v;
        if ((tid & 3) == 0) RS[tid >> 2] = f;
        __syncthreads();
        if (s0 + 16 * w < npos) {
            const int key = 16 * w + c16;  // this lane's key of the block (B column)
            const int4 kb = *reinterpret_cast<const int4 *>(R8 + key * HD + 16 * k4);
            const uint32_t kw[4] = {(uint32_t)kb.x, (uint32_t)kb.y, (uint32_t)kb.z, (uint32_t)kb.w};
            v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 16; t++) {
                const float kf = (float)(int8_t)((kw[t >> 2] >> (8 * (t & 3))) & 255u);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[t], kf, acc, 0, 0, 0);
            }
            const float ks = RS[key];
#pragma unroll
            for (int i = 0; i < 4; i++) S[(4 * k4 + i) * LT + s0 + key] = acc[i] * ks * scale;
        }
    }
    __syncthreads();
    // Softmax per query (16 lanes a row): e in place, the total aside.
    {
        const int qi = tid >> 4, li = tid & 15;
        const int qlast = pos0 + q0 + qi;
        float mx = -INFINITY;
        for (int s = li; s <= qlast && qi < nq; s += 16) mx = fmaxf(mx, S[qi * LT + s]);
        mx = row16_max(mx);
        float t = 0.0f;
        for (int s = li; s <= qlast && qi < nq; s += 16) {
            const float e = ref_expf(S[qi * LT + s] - mx);
            S[qi * LT + s] = e;
            t += e;
        }
        t = row16_sum(t);
        if (li == 0) tot[qi] = t;
    }
    // Values: wave w owns dims 16w..16w+15 of the 16 queries.
    const int qlast_a = pos0 + q0 + c16;  // the A row's query sees positions <= this
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < npos; s0 += kPB) {
        int4 v;
        float f;
        load_piece(V8, VS, s0, v, f);
        __syncthreads();  // also orders the softmax writes before the first reads
        {   // transposed: R8[d * kPB + row]
            const int row = tid >> 2, d0 = 16 * (tid & 3);
            const uint32_t vw[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
            for (int j = 0; j < 16; j++) R8[(d0 + j) * kPB + row] = (int8_t)((vw[j >> 2] >> (8 * (j & 3))) & 255u);
        }
        if ((tid & 3) == 0) RS[tid >> 2] = f;
        __syncthreads();
        const float total = tot[c16];
        const int d = 16 * w + c16;  // this lane's dim (B column)
        const int4 vb = *reinterpret_cast<const int4 *>(R8 + d * kPB + 16 * k4);
        const uint32_t vw[4] = {(uint32_t)vb.x, (uint32_t)vb.y, (uint32_t)vb.z, (uint32_t)vb.w};
        const float *er = S + c16 * LT + s0 + 16 * k4;
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const int s = s0 + 16 * k4 + t;
            float a = 0.0f;
            if (s <= qlast_a && c16 < nq) a = (er[t] / total) * RS[16 * k4 + t];  // p * vs
            const float vf = (float)(int8_t)((vw[t >> 2] >> (8 * (t & 3))) & 255u);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vf, acc, 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = 4 * k4 + i;
        if (q < nq) out[(int64_t)(q0 + q) * ldo + (int64_t)h * HD + 16 * w + c16] = acc[i];
    }
}
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// 8 signed int8 codes (a, b) as exact fp16 values: (c ^ 0x80) = c + 128 as a
// byte, 0x6400 | byte = 1024 + byte, minus 1152.
__device__ __forceinline__ v8h s8x8_f16(uint32_t a, uint32_t b) {
    a ^= 0x80808080u;
    b ^= 0x80808080u;
    const uint32_t d[4] = {__builtin_amdgcn_perm(0x64646464u, a, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)};
    const v2h k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    v8h r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const v2h h = __builtin_bit_cast(v2h, d[i]) - k1152;
        r[2 * i] = h[0];
        r[2 * i + 1] = h[1];
    }
    return r;
}
__device__ __forceinline__ float rows4_max_p(float v) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ float rows4_sum_p(float v) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// attend_prompt_kernel's attention for the 8 query heads of key / value head
// blockIdx.x and queries q0 .. q0 + 15 (q0 = 16 blockIdx.y) at once, on the
// fp16 matrix cores: each staged block of 64 key / value rows serves all 8
// heads.  Scores k . q with the int8 codes exact in fp16 and q as hi / lo
// planes; a first pass over the keys finds each query's maximum and the
// largest value scale, the second forms e = exp(s - max), the weights
// e vs sigma as hi / lo planes (sigma a power of two, max vs sigma < 2^10)
// and their products with the value codes.  Wave w owns heads 2w and 2w + 1:
// in the scores lane l holds query l % 16 and keys 4 (l / 16) + i of each
// 16-key tile, which is the operand layout of the value products, so the
// weights never leave registers.  Sums are in the matrix cores' order (float
// rounding, not attend_prompt_kernel's bits).
__global__ __launch_bounds__(256) void attend_prompt_gqa_kernel(const float *__restrict__ qkv, int64_t ld, int pos0,
                                                                int T, int layer, int max_t, int n_kv,
                                                                const int8_t *__restrict__ K8,
                                                                const int8_t *__restrict__ V8,
                                                                const float *__restrict__ KS,
                                                                const float *__restrict__ VS, float *__restrict__ out,
                                                                int64_t ldo, int hm) {
    constexpr int HD = 64, G = 8, KR = HD + 8, VR = kPB + 4;  // head dim, heads; LDS row strides (bytes)
    __shared__ __align__(16) int8_t kr[kPB][KR];
    __shared__ __align__(16) int8_t vt[HD][VR];
    __shared__ float ksb[kPB], vsb[kPB], vmx[4], tfin[4][2][16];
    const int kvh = blockIdx.x, q0 = blockIdx.y * kQB, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6, c16 = lane & 15, g = lane >> 4;
    const int nq = min(kQB, T - q0);
    const int npos = pos0 + q0 + nq;  // positions any query of the block sees
    const int64_t base = hm ? ((int64_t)layer * n_kv + kvh) * max_t : (int64_t)layer * max_t * n_kv + kvh;
    const int64_t pstr = hm ? 1 : n_kv;  // rows between positions
    const int qpos = pos0 + q0 + c16;  // the lane's query sees positions <= qpos
    const bool qok = c16 < nq;
    // the query operand of head 8 kvh + 2w + r: dims 32 kb + 8 g .., hi and lo planes
    v8h bq[2][2][2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const float *qr = qkv + (int64_t)(q0 + c16) * ld + (int64_t)(kvh * G + 2 * w + r) * HD;
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; e += 4) {
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (qok) v = *reinterpret_cast<const float4 *>(qr + 32 * kb + 8 * g + e);
                x[e] = v.x;
                x[e + 1] = v.y;
                x[e + 2] = v.z;
                x[e + 3] = v.w;
            }
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const _Float16 hi = (_Float16)x[e];
                bq[r][kb][0][e] = hi;
                bq[r][kb][1][e] = (_Float16)(x[e] - (float)hi);
            }
        }
    }
    // Block s0's rows: thread (key tid / 4, piece tid % 4) loads 16 bytes of the
    // key row (and of the value row), lane 0 of the key the scales; rows past
    // npos are zero.  fetch() issues the loads (the next block's go out before
    // this block's products), commit() writes them to LDS, values transposed.
    struct Rows {
        int4 kv, vv;
        float ks, vs;
    };
    auto fetch = [&](int s0, bool values) {
        Rows x{make_int4(0, 0, 0, 0), make_int4(0, 0, 0, 0), 0.0f, 0.0f};
        const int row = tid >> 2, piece = tid & 3, sidx = s0 + row;
        if (sidx < npos) {
            const int64_t sl = base + (int64_t)sidx * pstr;
            x.kv = *reinterpret_cast<const int4 *>(K8 + sl * HD + 16 * piece);
            x.ks = KS[sl];
            x.vs = VS[sl];
            if (values) x.vv = *reinterpret_cast<const int4 *>(V8 + sl * HD + 16 * piece);
        }
        return x;
    };
    auto commit = [&](const Rows &x, bool values) {
        const int row = tid >> 2, piece = tid & 3;
        __syncthreads();  // the previous block's reads are done
        *reinterpret_cast<int4 *>(&kr[row][16 * piece]) = x.kv;
        if (piece == 0) {
            ksb[row] = x.ks;
            vsb[row] = x.vs;
        }
        if (values) {
            const uint32_t vw[4] = {(uint32_t)x.vv.x, (uint32_t)x.vv.y, (uint32_t)x.vv.z, (uint32_t)x.vv.w};
#pragma unroll
            for (int j = 0; j < 16; j++) vt[16 * piece + j][row] = (int8_t)((vw[j >> 2] >> (8 * (j & 3))) & 255u);
        }
        __syncthreads();
    };
    // scores of key tile kt of the staged block for head row tiles r: D[key 4 g + i][query c16]
    auto scores = [&](int kt, v4f (&d)[2]) {
#pragma unroll
        for (int r = 0; r < 2; r++) d[r] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const uint2 kk = *reinterpret_cast<const uint2 *>(&kr[16 * kt + c16][32 * kb + 8 * g]);
            const v8h ak = s8x8_f16(kk.x, kk.y);
#pragma unroll
            for (int r = 0; r < 2; r++) {
                d[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bq[r][kb][0], d[r], 0, 0, 0);
                d[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bq[r][kb][1], d[r], 0, 0, 0);
            }
        }
    };
    const float scale = 1.0f / sqrtf((float)HD);
    // pass 1: each query's maximum, and the largest value scale
    float mx[2] = {-INFINITY, -INFINITY}, vm = 0.0f;
    Rows nx = fetch(0, false);
    for (int s0 = 0; s0 < npos; s0 += kPB) {
        commit(nx, false);
        vm = fmaxf(vm, nx.vs);
        if (s0 + kPB < npos) nx = fetch(s0 + kPB, false);
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            v4f d[2];
            scores(kt, d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = s0 + 16 * kt + 4 * g + i;
                const float ks = ksb[16 * kt + 4 * g + i];
#pragma unroll
                for (int r = 0; r < 2; r++)
                    if (qok && p <= qpos) mx[r] = fmaxf(mx[r], d[r][i] * ks * scale);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 2; r++) mx[r] = rows4_max_p(mx[r]);
    vm = wave_max(vm);
    if (lane == 0) vmx[w] = vm;
    __syncthreads();
    int ex = 0;
    frexpf(fmaxf(fmaxf(vmx[0], vmx[1]), fmaxf(vmx[2], vmx[3])), &ex);
    const int sig_e = min(126, max(-126, 10 - ex));
    const float sigma = ldexpf(1.0f, sig_e);
    // pass 2: weights and value sums; o[r][dt]: D[query 4 g + i][dim 16 dt + c16]
    v4f o[2][4];
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[r][dt] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    float te[2] = {0.0f, 0.0f};
    nx = fetch(0, true);
    for (int s0 = 0; s0 < npos; s0 += kPB) {
        commit(nx, true);
        if (s0 + kPB < npos) nx = fetch(s0 + kPB, true);
        v8h ph[2][2], pl[2][2];  // [r][key half]: element e is key 32 c + 16 (e / 4) + 4 g + e % 4
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            v4f d[2];
            scores(kt, d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = s0 + 16 * kt + 4 * g + i;
                const float ks = ksb[16 * kt + 4 * g + i], vs = vsb[16 * kt + 4 * g + i];
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const bool ok = qok && p <= qpos;
                    const float e = ok ? expf(d[r][i] * ks * scale - mx[r]) : 0.0f;
                    te[r] += e;
                    const float x = e * vs * sigma;
                    const _Float16 hi = (_Float16)x;
                    ph[r][kt >> 1][4 * (kt & 1) + i] = hi;
                    pl[r][kt >> 1][4 * (kt & 1) + i] = (_Float16)(x - (float)hi);
                }
            }
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t v0 = *reinterpret_cast<const uint32_t *>(&vt[16 * dt + c16][32 * c + 4 * g]);
                const uint32_t v1 = *reinterpret_cast<const uint32_t *>(&vt[16 * dt + c16][32 * c + 16 + 4 * g]);
                const v8h bv = s8x8_f16(v0, v1);
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    o[r][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[r][c], bv, o[r][dt], 0, 0, 0);
                    o[r][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[r][c], bv, o[r][dt], 0, 0, 0);
                }
            }
    }
    // each query's total, from the score layout (lane = query) to the value layout (4 g + i)
#pragma unroll
    for (int r = 0; r < 2; r++) {
        te[r] = rows4_sum_p(te[r]);
        if (g == 0) tfin[w][r][c16] = te[r];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's own LDS writes are in
    const float isig = ldexpf(1.0f, -sig_e);
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = 4 * g + i;
            if (q < nq) {
                const float t = tfin[w][r][q];
#pragma unroll
                for (int dt = 0; dt < 4; dt++)
                    out[(int64_t)(q0 + q) * ldo + (int64_t)(kvh * G + 2 * w + r) * HD + 16 * dt + c16] =
                        o[r][dt][i] * isig / t;
            }
        }
}

}  // namespace

int launch_attend_prompt(llmq_ctx *ctx, const int8_t *K8, const int8_t *V8, const float *KS, const float *VS,
                         int layer, int max_t, int n_head, int n_kv, const float *qkv, int64_t ld, int pos0, int T,
                         float *out, int64_t ldo, bool head_major) {
    LLMQ_REQUIRE(n_kv > 0 && n_head % n_kv == 0, "attend: %d query heads over %d key / value heads", n_head, n_kv);
    LLMQ_REQUIRE(T >= 1 && pos0 >= 0 && pos0 + T <= max_t, "attend: positions %d..%d beyond %d", pos0, pos0 + T - 1,
                 max_t);
    const int LT = ((pos0 + T) + 63) & ~63;
    const size_t lds = sizeof(float) * ((size_t)kQB * LT + kPB) + (size_t)kPB * 64;
    static size_t granted = 64 * 1024;
    if (lds > granted) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&attend_prompt_kernel<64>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    if (n_head == 8 * n_kv) {  // grouped queries: the 8 heads of a key / value head share each staged block
        hipLaunchKernelGGL(attend_prompt_gqa_kernel, dim3(n_kv, (T + kQB - 1) / kQB), dim3(256), 0, ctx->stream, qkv,
                           ld, pos0, T, layer, max_t, n_kv, K8, V8, KS, VS, out, ldo, (int)head_major);
        LLMQ_HIP(hipGetLastError());
        return LLMQ_OK;
    }
    hipLaunchKernelGGL(attend_prompt_kernel<64>, dim3(n_head, (T + kQB - 1) / kQB), dim3(256), lds, ctx->stream, qkv,
                       ld, pos0, T, layer, max_t, n_kv, n_head / n_kv, K8, V8, KS, VS, out, ldo, LT, (int)head_major);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_kv_store(llmq_ctx *ctx, llmq_kv *kv, int layer, int pos0, const int *pos_dev, const float *qkv, int T,
                    int64_t ld) {
    LLMQ_REQUIRE(kv && qkv && T >= 1, "kv_store: bad arguments");
    LLMQ_REQUIRE(layer >= 0 && layer < kv->n_layer, "kv_store: layer %d out of range", layer);
    LLMQ_REQUIRE(pos_dev || (pos0 >= 0 && pos0 + T <= kv->max_t), "kv_store: positions %d..%d beyond max_t %d", pos0,
                 pos0 + T - 1, kv->max_t);
    if (kv->integer) return launch_ikv_store(ctx, kv, layer, pos0, pos_dev, qkv, T, ld);
    const int C = kv->n_head * kv->head_dim;
    hipLaunchKernelGGL(kv_store_kernel, dim3(kv->n_head, T), dim3(64), 0, ctx->stream, qkv, ld ? ld : 3 * C, C, pos0,
                       pos_dev, layer, kv->max_t, kv->n_head, kv->head_dim, kv->k, kv->v, kv->ks, kv->vs);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

template <int HD, bool STAGE, bool STORE>
static int attend_launch(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
                         const int *pos_dev, int64_t ld, size_t lds) {
    const int C = kv->n_head * kv->head_dim;
    hipLaunchKernelGGL((kv_attend_kernel<HD, STAGE, STORE>), dim3(kv->n_head, T), dim3(kAttnThreads), lds, ctx->stream,
                       qkv, ld ? ld : 3 * C, C, pos0, pos_dev, layer, kv->max_t, kv->n_head, kv->k, kv->v, kv->ks,
                       kv->vs, out, (int64_t)C);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

// Raises a kernel's dynamic LDS limit to `bytes` once; false if the device
// does not allow that much.
template <int HD, bool STAGE, bool STORE>
static bool allow_lds(size_t bytes) {
    static size_t granted = 64 * 1024;
    if (bytes <= granted) return true;
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(&kv_attend_kernel<HD, STAGE, STORE>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    granted = bytes;
    return true;
}

template <int HD>
static int attend_hd(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
                     const int *pos_dev, int64_t ld, bool store) {
    const size_t base = sizeof(float) * ((size_t)HD + kv->max_t);
    const size_t staged = base + (size_t)kv->max_t * (sizeof(float) + HD) + 16;
    if (store && allow_lds<HD, true, true>(staged))
        return attend_launch<HD, true, true>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, staged);
    if (!store && allow_lds<HD, true, false>(staged))
        return attend_launch<HD, true, false>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, staged);
    return store ? attend_launch<HD, false, true>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, base)
                 : attend_launch<HD, false, false>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, base);
}

// The exact-order prompt attention (head_dim 64); LLMQ_PROMPT_NTH /
// LLMQ_PROMPT_TQ choose other workgroup shapes, for measurement.
template <int NTH, int TQ, bool SV = false>
static int prompt_exact_launch(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T,
                               int pos0, int64_t ld) {
    const int C = kv->n_head * 64;
    const int PC = NTH / 4;
    const int NP = (pos0 + T + PC - 1) / PC * PC;
    const size_t lds = sizeof(float) * ((size_t)PC * kKStr + PC + NP + (size_t)TQ * (NP + 1));
    static size_t granted = 64 * 1024;
    if (lds > granted) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&attend_prompt_exact_kernel<NTH, TQ, SV>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    const int nblk = (T + TQ - 1) / TQ;
    hipLaunchKernelGGL((attend_prompt_exact_kernel<NTH, TQ, SV>), dim3(kv->n_head, (nblk + 1) / 2), dim3(NTH), lds,
                       ctx->stream, qkv, ld ? ld : 3 * C, pos0, T, layer, kv->max_t, kv->n_head, kv->k, kv->v, kv->ks,
                       kv->vs, out, (int64_t)C, NP);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_kv_attend(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
                     const int *pos_dev, int64_t ld, bool store) {
    LLMQ_REQUIRE(kv && qkv && out && T >= 1, "kv_attend: bad arguments");
    LLMQ_REQUIRE(layer >= 0 && layer < kv->n_layer, "kv_attend: layer %d out of range", layer);
    LLMQ_REQUIRE(pos_dev || (pos0 >= 0 && pos0 + T <= kv->max_t), "kv_attend: positions beyond max_t");
    LLMQ_REQUIRE(!store || T == 1, "kv_attend: the fused store takes one token");
    if (kv->integer) return launch_ikv_attend(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, store);
    if (!store && !pos_dev && T > 1 && kv->head_dim == 64 && !exact_order()) {
        // Prompt: query blocks of 16 per head, scores in LDS up to the last position
        const int C = kv->n_head * kv->head_dim;
        return launch_attend_prompt(ctx, kv->k, kv->v, kv->ks, kv->vs, layer, kv->max_t, kv->n_head, kv->n_head, qkv,
                                    ld ? ld : 3 * C, pos0, T, out, (int64_t)C);
    }
    if (!store && !pos_dev && T > 1 && kv->head_dim == 64 && (ld ? ld : 3 * kv->n_head * 64) % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(qkv) & 15) == 0) {
        const char *e = getenv("LLMQ_PROMPT_TQ"), *n = getenv("LLMQ_PROMPT_NTH");
        // 512 threads, 16 tokens: 44 us a layer at 476 tokens (256 / 8, 256 / 16: 48-51 us)
        const int tq = e ? atoi(e) : 16, nth = n ? atoi(n) : 512;
        if (nth == 256) return tq == 8 ? prompt_exact_launch<256, 8>(ctx, kv, out, qkv, layer, T, pos0, ld)
                                       : prompt_exact_launch<256, 16>(ctx, kv, out, qkv, layer, T, pos0, ld);
        if (tq == 8) return prompt_exact_launch<512, 8>(ctx, kv, out, qkv, layer, T, pos0, ld);
        // value chains four a thread (LLMQ_PROMPT_SV=0: two a thread): 476
        // tokens, same box, 1.50 / 1.62 ms against 1.51 / 1.64 (int4 / int8
        // prefill); two queries a lane in the scores measured slower (1.58)
        const char *sv = getenv("LLMQ_PROMPT_SV");
        if (sv && sv[0] == '0') return prompt_exact_launch<512, 16, false>(ctx, kv, out, qkv, layer, T, pos0, ld);
        return prompt_exact_launch<512, 16, true>(ctx, kv, out, qkv, layer, T, pos0, ld);
    }
    if (kv->head_dim == 64) return attend_hd<64>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, store);
    if (kv->head_dim == 128) return attend_hd<128>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, store);
    return llmq_set_error(LLMQ_EUNSUPPORTED, "kv_attend: head_dim %d (64 or 128)", kv->head_dim);
}

int launch_layernorm(llmq_ctx *ctx, float *out, const float *x, const float *w, const float *b, int64_t T, int64_t C) {
    LLMQ_REQUIRE(T >= 1 && C >= 1 && out && x && w && b, "layernorm: bad arguments");
    LLMQ_REQUIRE(C % 16 == 0 && C <= 16384, "layernorm: C must be a multiple of 16, at most 16384");
    hipLaunchKernelGGL(layernorm_kernel, dim3((unsigned)T), dim3(256), (size_t)C * 4, ctx->stream, out, x, w, b, C);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_embed(llmq_ctx *ctx, const llmq_mat *E, const float *wpe, const int64_t *tokens, int T, int pos0,
                 float *x, const ArgmaxPart *parts, int nparts, int64_t *gen, int *state, int do_embed) {
    LLMQ_REQUIRE(E && E->kind == MAT_QUANT, "embed: the embedding must be a QuantMatrix");
    LLMQ_REQUIRE(parts ? nparts > 0 && gen && state : tokens && T >= 1,
                 "embed: tokens, or argmax partials with the decode state");
    const int64_t cpg = E->group / (E->bits == 4 ? 32 : 16);
    hipLaunchKernelGGL(embed_kernel, dim3(parts ? 1 : T), dim3(256), 0, ctx->stream,
                       reinterpret_cast<const uint4 *>(E->codes), E->scales, E->zps, E->bits, E->CK, E->NG, cpg, wpe,
                       tokens, pos0, (int)E->k, x, parts, nparts, gen, state, do_embed, E->n);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
