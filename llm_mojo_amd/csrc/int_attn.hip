// IntAttnKV (int_attention.mojo:62-269): an int8 key / value cache with
// per-(position, head) scales held as integers (scale * 2^24), and attention
// computed in integers with intmath.masked_exp (intmath.mojo:48-123).
//
// Layout in HBM: the int8 cache's [layer, pos, head, head_dim] codes and
// [layer, pos, head] int32 scales (the reference's VNNI blocking is a CPU
// layout for VPDPWSSD; the arithmetic does not depend on it).
//
// Every step is integer arithmetic except the final float multiply, which
// follows the reference: per 256-position segment the exact int32 value sums
// become float and add in segment order, then out = sums * f32(vmax 2^15 /
// (2^24 total)).  The integer sums are exact in any order, so the kernels
// reproduce the reference's results bit for bit.
#include "common.h"

namespace {

constexpr int kKS = 24;  // fraction bits of the key / value scales (int_attention.mojo:54)
constexpr int kSF = 16;  // fraction bits of the fixed-point scores (:55)
constexpr int kFB = 16;  // fraction bits of the base-2 exponent (intmath.mojo:31)
constexpr int kMB = 24;  // extra fraction bits of the multiplier (:32)
constexpr int64_t kDCap = (int64_t)1 << 31;  // :35
constexpr int kThreads = 256;

// A native vector (not HIP's int4 struct, whose copies kept the value rows
// in scratch memory).
typedef int v4i __attribute__((ext_vector_type(4)));

// maxima over the wave (order-free), without LDS
__device__ __forceinline__ float wave_max_f(float v) { return llmq_wave_max_all(v); }
__device__ __forceinline__ int wave_max_i(int v) { return llmq_wave_max_all(v); }
__device__ __forceinline__ int64_t wave_sum_l(int64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// exp2_neg (intmath.mojo:53-65): 2^(-d scale log2 e) in Q30 for d >= 0, the
// integer part of the exponent as a shift and the fraction by a degree-3
// polynomial; exponents >= 31 give 0.
__device__ __forceinline__ int64_t exp2_neg(int64_t d, int64_t mult) {
    constexpr int64_t C0 = 1073741824, C1 = -742598100, C2 = 248207216, C3 = -42480028;  // :40-43
    const int64_t y = ((d < kDCap ? d : kDCap) * mult) >> kMB;
    const int64_t q = y >> kFB;
    const int64_t r = y & (((int64_t)1 << kFB) - 1);
    int64_t p = C3;
    p = ((p * r) >> kFB) + C2;
    p = ((p * r) >> kFB) + C1;
    p = ((p * r) >> kFB) + C0;
    return q >= 31 ? 0 : p >> q;
}

// IntAttnKV.quantize_head (int_attention.mojo:140-168) with one wave:
// s = max|x| / 127 (1 if zero), codes round(x * (1 / s)); returns s * 2^24
// rounded, as int32.  Codes go to dst (global) and, when given, lds_copy.
template <int HD>
__device__ __forceinline__ int32_t quantize_head(const float *__restrict__ src, int8_t *__restrict__ dst,
                                                 int8_t *lds_copy, int lane) {
    float xs[HD / 64];
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < HD / 64; e++) {
        xs[e] = src[lane + 64 * e];
        m = fmaxf(m, fabsf(xs[e]));
    }
    m = wave_max_f(m);
    float s = m / 127.0f;
    if (s == 0.0f) s = 1.0f;
    const float inv = 1.0f / s;
#pragma unroll
    for (int e = 0; e < HD / 64; e++) {
        const int8_t c = (int8_t)llmq_to_int(roundf(xs[e] * inv));
        dst[lane + 64 * e] = c;
        if (lds_copy) lds_copy[lane + 64 * e] = c;
    }
    return (int32_t)(int64_t)round((double)s * (double)(1 << kKS));
}

// IntAttnKV.store (int_attention.mojo:132-138) for token t = blockIdx.y at
// position pos0 + t, head h = blockIdx.x; keys and values are columns C..
// and 2C.. of qkv row t.
template <int HD>
__global__ __launch_bounds__(64) void ikv_store_kernel(const float *__restrict__ qkv, int64_t ld, int C, int pos0,
                                                       const int *__restrict__ pos_dev, int layer, int max_t,
                                                       int n_head, int8_t *__restrict__ K8, int8_t *__restrict__ V8,
                                                       int32_t *__restrict__ KQ, int32_t *__restrict__ VQ) {
    const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int pos = (pos_dev ? *pos_dev : pos0) + t;
    const int64_t sl = ((int64_t)layer * max_t + pos) * n_head + h;
    const float *row = qkv + (int64_t)t * ld + (int64_t)h * HD;
    const int32_t kq = quantize_head<HD>(row + C, K8 + sl * HD, nullptr, lane);
    const int32_t vq = quantize_head<HD>(row + 2 * C, V8 + sl * HD, nullptr, lane);
    if (lane == 0) {
        KQ[sl] = kq;
        VQ[sl] = vq;
    }
}

// IntAttnKV.attend_one (int_attention.mojo:170-269) for token t = blockIdx.y
// (position pos0 + t, or state[0] + t on the device-driven decode path) and
// head h = blockIdx.x, 256 threads:
//   1. query -> int16 (wave 0) and the score multiplier qm = sq / sqrt(HD) 2^40;
//   2-3. thread i scores positions i, i + 256, ...: the int32 dot product of
//      the int16 query with the int8 key, rescaled to 16 fraction bits
//      ((dot kq + 2^23) >> 24, then (. qm + 2^23) >> 24);
//   4. masked_exp over the scores (maximum, exp2_neg, int64 total);
//   5. int16 weights w = min((e r16 + 2^30) >> 31, 32767) with r16 the value
//      scale relative to the largest, Q16; per 256-position segment the
//      int32 sums of w v (exact) become float and add in segment order;
//   6. out = sums * f32(vmax 2^15 / (2^24 total)).
// STAGE copies each position's value row into LDS while scoring, so the
// value pass reads no global memory.  STORE (one token: decode) quantizes the
// head's new key and value first (IntAttnKV.store) and uses them from LDS.
template <int HD, bool STAGE, bool STORE>
__global__ __launch_bounds__(kThreads) void ikv_attend_kernel(const float *__restrict__ qkv, int64_t ld, int C,
                                                              int pos0, const int *__restrict__ pos_dev, int layer,
                                                              int max_t, int n_head, int8_t *__restrict__ K8,
                                                              int8_t *__restrict__ V8, int32_t *__restrict__ KQ,
                                                              int32_t *__restrict__ VQ, float *__restrict__ out,
                                                              int64_t ldo, int64_t mult, double sqrt_hd) {
    constexpr int NV = HD / 16;         // 16-byte pieces of a row
    constexpr int DG = HD / 4;          // value pass: dimension groups of 4
    constexpr int SLICES = kThreads / DG;  // and position slices
    extern __shared__ __align__(16) int32_t ism[];
    int32_t *scores = ism;             // [max_t]
    int32_t *vqs = scores + max_t;     // [max_t] value scales
    int16_t *w = reinterpret_cast<int16_t *>(vqs + max_t);  // [max_t] weights
    int8_t *vrow = reinterpret_cast<int8_t *>(w + ((max_t + 7) & ~7));  // [max_t][HD] (STAGE)
    __shared__ __align__(16) int16_t qi[HD];
    __shared__ __align__(16) int8_t knew[HD], vnew[HD];
    __shared__ __align__(16) int32_t part[SLICES * HD];
    __shared__ int64_t qm_s, red64[4];
    __shared__ int32_t red_m[4], red_v[4], kq_new;
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int npos = (pos_dev ? *pos_dev : pos0) + t + 1;
    const int cur = npos - 1;
    const int64_t base = (int64_t)layer * max_t * n_head + h;  // slot of position 0
    const float *qrow = qkv + (int64_t)t * ld + (int64_t)h * HD;

    // This thread's first rows, requested before anything else (positions
    // past the end re-read the last one and are not used).
    v4i kr[NV], vr[NV];
    int32_t kqr, vqr;
    auto load_row = [&](int s) {
        const int64_t sl = base + (int64_t)s * n_head;
        const v4i *kp = reinterpret_cast<const v4i *>(K8 + sl * HD);
        const v4i *vp = reinterpret_cast<const v4i *>(V8 + sl * HD);
#pragma unroll
        for (int i = 0; i < NV; i++) {
            kr[i] = kp[i];
            if (STAGE) vr[i] = vp[i];
        }
        kqr = KQ[sl];
        vqr = VQ[sl];
    };
    load_row(tid < npos ? tid : cur);
    __builtin_amdgcn_sched_barrier(0);

    if (wid == 0) {
        // 1. Query -> int16, symmetric (int_attention.mojo:183-197).
        float qv[HD / 64];
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < HD / 64; e++) {
            qv[e] = qrow[lane + 64 * e];
            m = fmaxf(m, fabsf(qv[e]));
        }
        m = wave_max_f(m);
        float sq = m / 32767.0f;
        if (sq == 0.0f) sq = 1.0f;
        const float invq = 1.0f / sq;
#pragma unroll
        for (int e = 0; e < HD / 64; e++) qi[lane + 64 * e] = (int16_t)llmq_to_int(roundf(qv[e] * invq));
        if (lane == 0) qm_s = (int64_t)round((double)sq / sqrt_hd * (double)((int64_t)1 << (kSF + kKS)));
    } else if (STORE && (wid == 1 || wid == 2)) {
        // IntAttnKV.store for this head's new key (wave 1) and value (wave 2).
        const int kv = wid - 1;
        const int64_t sl = base + (int64_t)cur * n_head;
        // LDS copies: the workgroup reads the new rows from there, not back
        // from global memory.
        int8_t *copy = kv == 0 ? knew : (STAGE ? vrow + (int64_t)cur * HD : vnew);
        const int32_t q = quantize_head<HD>(qrow + (int64_t)(1 + kv) * C, (kv ? V8 : K8) + sl * HD, copy, lane);
        if (lane == 0) {
            (kv ? VQ : KQ)[sl] = q;
            if (kv == 0)
                kq_new = q;
            else
                vqs[cur] = q;
        }
    }
    lds_barrier();

    // 2-3. Scores in 16 fraction bits; the maxima of the scores and scales.
    uint32_t qpair[HD / 2];  // the int16 query, two dimensions a word
#pragma unroll
    for (int i = 0; i < HD / 8; i++) {
        const int4 q4 = reinterpret_cast<const int4 *>(qi)[i];
        qpair[4 * i] = (uint32_t)q4.x;
        qpair[4 * i + 1] = (uint32_t)q4.y;
        qpair[4 * i + 2] = (uint32_t)q4.z;
        qpair[4 * i + 3] = (uint32_t)q4.w;
    }
    const int64_t qm = qm_s;
    int smax = INT32_MIN, vmax = 0;
    for (int s = tid; s < npos; s += kThreads) {
        if (s != tid) load_row(s);  // only past 256 positions
        const bool fresh = STORE && s == cur;
        if (fresh) {
#pragma unroll
            for (int i = 0; i < NV; i++) kr[i] = reinterpret_cast<const v4i *>(knew)[i];
            kqr = kq_new;
            vqr = vqs[cur];
        }
        // int32 dot product (at most HD 32767 127: no overflow for HD <= 512)
        int32_t acc = 0;
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t kw[4] = {(uint32_t)kr[i].x, (uint32_t)kr[i].y, (uint32_t)kr[i].z, (uint32_t)kr[i].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t q01 = qpair[8 * i + 2 * j], q23 = qpair[8 * i + 2 * j + 1];
                acc += (int32_t)(int16_t)q01 * (int32_t)(int8_t)kw[j];
                acc += (int32_t)(int16_t)(q01 >> 16) * (int32_t)(int8_t)(kw[j] >> 8);
                acc += (int32_t)(int16_t)q23 * (int32_t)(int8_t)(kw[j] >> 16);
                acc += (int32_t)(int16_t)(q23 >> 16) * (int32_t)(int8_t)(kw[j] >> 24);
            }
        }
        const int64_t t1 = ((int64_t)acc * kqr + ((int64_t)1 << (kKS - 1))) >> kKS;
        const int32_t sc = (int32_t)((t1 * qm + ((int64_t)1 << (kKS - 1))) >> kKS);
        scores[s] = sc;
        smax = max(smax, sc);
        vmax = max(vmax, vqr);
        if (!fresh) {
            vqs[s] = vqr;
            if (STAGE) {
#pragma unroll
                for (int i = 0; i < NV; i++) *reinterpret_cast<v4i *>(vrow + (int64_t)s * HD + 16 * i) = vr[i];
            }
        }
    }
    smax = wave_max_i(smax);
    vmax = wave_max_i(vmax);
    if (lane == 0) {
        red_m[wid] = smax;
        red_v[wid] = vmax;
    }
    lds_barrier();
    const int64_t m = max(max(red_m[0], red_m[1]), max(red_m[2], red_m[3]));
    vmax = max(max(red_v[0], red_v[1]), max(red_v[2], red_v[3]));

    // 4-5. e = exp2_neg(m - score) in Q30, the total, the int16 weights.
    const int64_t inv47 = vmax > 0 ? ((int64_t)1 << 47) / vmax : 0;
    int64_t tot = 0;
    for (int s = tid; s < npos; s += kThreads) {
        const int64_t e = exp2_neg(m - scores[s], mult);
        tot += e;
        const int64_t r16 = ((int64_t)vqs[s] * inv47) >> 31;
        const int64_t ww = min((e * r16 + ((int64_t)1 << 30)) >> 31, (int64_t)32767);
        w[s] = e == 0 ? 0 : (int16_t)ww;
    }
    tot = wave_sum_l(tot);
    if (lane == 0) red64[wid] = tot;
    lds_barrier();
    const int64_t total = red64[0] + red64[1] + red64[2] + red64[3];
    float *o = out + (int64_t)t * ldo + (int64_t)h * HD;
    if (vmax == 0 || total == 0) {
        for (int i = tid; i < HD; i += kThreads) o[i] = 0.0f;
        return;
    }

    // Weighted value sums: thread (dg, slice) takes dimensions 4dg..4dg+3 of
    // positions slice, slice + SLICES, ... of each 256-position segment.
    const int dg = tid % DG, slice = tid / DG;
    float accf = 0.0f;  // dimension tid (tid < HD)
    for (int seg = 0; seg < npos; seg += 256) {
        const int end = min(seg + 256, npos);
        int32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
        for (int s = seg + slice; s < end; s += SLICES) {
            const int32_t ws = w[s];
            uint32_t vw;
            if (STAGE)
                vw = *reinterpret_cast<const uint32_t *>(vrow + (int64_t)s * HD + 4 * dg);
            else if (STORE && s == cur)
                vw = *reinterpret_cast<const uint32_t *>(vnew + 4 * dg);
            else
                vw = *reinterpret_cast<const uint32_t *>(V8 + (base + (int64_t)s * n_head) * HD + 4 * dg);
            a0 += ws * (int32_t)(int8_t)(vw);
            a1 += ws * (int32_t)(int8_t)(vw >> 8);
            a2 += ws * (int32_t)(int8_t)(vw >> 16);
            a3 += ws * (int32_t)(int8_t)(vw >> 24);
        }
        *reinterpret_cast<int4 *>(part + slice * HD + 4 * dg) = make_int4(a0, a1, a2, a3);
        lds_barrier();
        if (tid < HD) {
            int32_t v = 0;
#pragma unroll
            for (int p = 0; p < SLICES; p++) v += part[p * HD + tid];
            accf += (float)v;
        }
        lds_barrier();
    }
    // 6. Back to float: * (vmax / 2^24) * 2^15 / total.
    const float fs = (float)((double)vmax * (double)(1 << 15) / ((double)(1 << kKS) * (double)total));
    if (tid < HD) o[tid] = accf * fs;
}

template <int HD, bool STAGE, bool STORE>
int attend_launch(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
                  const int *pos_dev, int64_t ld, size_t lds, int64_t mult) {
    static size_t granted = 64 * 1024;
    if (lds > granted) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&ikv_attend_kernel<HD, STAGE, STORE>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    const int C = kv->n_head * kv->head_dim;
    hipLaunchKernelGGL((ikv_attend_kernel<HD, STAGE, STORE>), dim3(kv->n_head, T), dim3(kThreads), lds, ctx->stream,
                       qkv, ld ? ld : 3 * C, C, pos0, pos_dev, layer, kv->max_t, kv->n_head, kv->k, kv->v, kv->kq,
                       kv->vq, out, (int64_t)C, mult, sqrt((double)HD));
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

template <int HD>
int attend_hd(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
              const int *pos_dev, int64_t ld, bool store) {
    // exp_multiplier(1 / 2^16) (intmath.mojo:48-50, int_attention.mojo:174)
    const int64_t mult = (int64_t)(1.0 / (double)(1 << kSF) * 1.4426950408889634 *
                                       (double)((int64_t)1 << (kFB + kMB)) + 0.5);
    const size_t base = (size_t)kv->max_t * 8 + (size_t)((kv->max_t + 7) & ~7) * 2;
    const size_t staged = base + (size_t)kv->max_t * HD;
    // Staged values fit the 160 KB of LDS up to max_t = 1920 at HD 64.
    if (staged <= 150 * 1024)
        return store ? attend_launch<HD, true, true>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, staged, mult)
                     : attend_launch<HD, true, false>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, staged, mult);
    LLMQ_REQUIRE(base <= 150 * 1024, "int attention: max_t %d needs more LDS than a workgroup has", kv->max_t);
    return store ? attend_launch<HD, false, true>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, base, mult)
                 : attend_launch<HD, false, false>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, base, mult);
}

}  // namespace

int launch_ikv_store(llmq_ctx *ctx, llmq_kv *kv, int layer, int pos0, const int *pos_dev, const float *qkv, int T,
                     int64_t ld) {
    const int C = kv->n_head * kv->head_dim;
    if (kv->head_dim == 64)
        hipLaunchKernelGGL(ikv_store_kernel<64>, dim3(kv->n_head, T), dim3(64), 0, ctx->stream, qkv, ld ? ld : 3 * C,
                           C, pos0, pos_dev, layer, kv->max_t, kv->n_head, kv->k, kv->v, kv->kq, kv->vq);
    else if (kv->head_dim == 128)
        hipLaunchKernelGGL(ikv_store_kernel<128>, dim3(kv->n_head, T), dim3(64), 0, ctx->stream, qkv, ld ? ld : 3 * C,
                           C, pos0, pos_dev, layer, kv->max_t, kv->n_head, kv->k, kv->v, kv->kq, kv->vq);
    else
        return llmq_set_error(LLMQ_EUNSUPPORTED, "int attention: head_dim %d (64 or 128)", kv->head_dim);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_ikv_attend(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
                      const int *pos_dev, int64_t ld, bool store) {
    if (kv->head_dim == 64) return attend_hd<64>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, store);
    if (kv->head_dim == 128) return attend_hd<128>(ctx, kv, out, qkv, layer, T, pos0, pos_dev, ld, store);
    return llmq_set_error(LLMQ_EUNSUPPORTED, "int attention: head_dim %d (64 or 128)", kv->head_dim);
}
