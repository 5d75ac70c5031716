// One GPT-2 decode token's qkv projection and attention, fused per head:
// LayerNorm (kernels.mojo:179-197), quantize_rows (400-416) and the int4 A16
// GEMV of the head's 192 qkv rows (QuantMatrix.dot_row_i16, tensor.mojo:
// 518-577, + bias), then QuantKV.store of the new key and value
// (kvcache.mojo:320-342) and attend_float_one (113-150) over the head's
// cached positions.  One 1024-thread workgroup per head: the cached key and
// value rows (one position per thread, max_t <= 1024), the activation row
// and the head's weight rows are all requested at kernel start, so their
// latency overlaps the prologue; the attention needs no kernel boundary
// after the projection.
//
// Arithmetic is the two-kernel path's: the same int16 codes and exact
// per-chunk integer sums G = sum xq (u - zp), acc += G * scale, y = acc * sx
// + b; the attention's float sums run in a different order (1e-5 bar).
#include "common.h"

namespace {

constexpr int kNT = 1024, kNW = 16, kHD = 64;
constexpr int kMaxCK = 48;  // chunks of 32 inputs per row (C <= 1536)

typedef int v4i __attribute__((ext_vector_type(4)));

struct QkvAttnArgs {
    const uint4 *codes;      // qkv matrix, device row tiles (int4)
    const uint16_t *scales;  // [tile][group][16] float16 bits
    const uint8_t *zps;
    int CK, NG, cpg_shift;
    const float *x, *ln_w, *ln_b, *bias;  // residual row [C], LN_1, qkv bias [3C]
    int C;
    int8_t *K8, *V8;
    float *KS, *VS;
    int layer, max_t, n_head;
    const int *pos_dev;  // device position (decode graph) or nullptr
    int pos0;
    float *qkv_out;  // [3C]: this head's q, k, v columns
    float *att;      // [C]: this head's 64 outputs
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < kNW; i++) s += red[i];
    lds_barrier();  // red is reused by the next reduction
    return s;
}
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < kNW; i++) s = fmaxf(s, red[i]);
    lds_barrier();
    return s;
}
// Buffer loads: an offset at or past the extent returns zeros without a
// memory access, so lanes and waves with nothing to load need no branch
// (a branch around a load makes the join wait for it).
constexpr uint32_t kOOB = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

__device__ __forceinline__ int round_to_int(float v) {
    float r = roundf(v);
    r = r != r ? 0.0f : r;
    r = fminf(fmaxf(r, -1.0e9f), 1.0e9f);
    return (int)r;
}

template <int S>  // code steps of 4 chunks per row: CK = 4 S
__global__ __launch_bounds__(kNT) void qkv_attn_kernel(QkvAttnArgs a) {
    extern __shared__ __align__(16) float dyn[];
    float *scores = dyn;                // [max_t]
    float *vsc = scores + a.max_t;      // [max_t]
    int8_t *vrow = reinterpret_cast<int8_t *>(vsc + a.max_t);  // [max_t][64], 16-byte aligned
    int8_t *krow = vrow + (int64_t)a.max_t * kHD;               // [max_t][64]
    __shared__ __align__(16) uint32_t planes[kMaxCK * 16];      // [chunk][dword i][plane p]
    __shared__ int xsum[kMaxCK];
    __shared__ float red[kNW];
    __shared__ float head[3][kHD];  // q, k, v of this head
    __shared__ float kscale_new;
    __shared__ float part[kNW][kHD];

    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int C = a.C, nunits = C / 4;
    const int npos = (a.pos_dev ? *a.pos_dev : a.pos0) + 1;
    const int cur = npos - 1;
    const int64_t base = (int64_t)a.layer * a.max_t * a.n_head + h;  // cache slot of position 0

    // 1. Every load that does not depend on this kernel's results, first, in
    //    the order they are needed (loads complete in order): the activation
    //    row, the wave's weight rows, scales, zero points and biases, then
    //    this thread's cached key / value row.
    const bool has = tid < nunits;
    const uint32_t xo = has ? (uint32_t)tid * 16u : kOOB;
    const auto rx = rsrc(a.x, (uint32_t)C * 4u), rlw = rsrc(a.ln_w, (uint32_t)C * 4u),
               rlb = rsrc(a.ln_b, (uint32_t)C * 4u);
    const v4i xi = bload16(rx, xo), lwi = bload16(rlw, xo), lbi = bload16(rlb, xo);
    __builtin_amdgcn_sched_barrier(0);
    // wave w < 12: block b = w / 4 (q, k, v), row tile w % 4 of the head
    const int r = lane & 15, j = lane >> 4;
    const bool gemv_wave = wid < 12;
    const int blk = wid >> 2;
    const int tile = blk * (C / 16) + h * (kHD / 16) + (wid & 3);
    const int row = tile * 16 + r;  // row of the [3C] output
    const int ntiles = 3 * C / 16;
    const auto rc = rsrc(a.codes, (uint32_t)ntiles * a.CK * 256u);
    const auto rs = rsrc(a.scales, (uint32_t)ntiles * a.NG * 32u);
    const auto rz = rsrc(a.zps, (uint32_t)ntiles * a.NG * 16u);
    const auto rbias = rsrc(a.bias, (uint32_t)(3 * C) * 4u);
    v4i wc[S];
    uint32_t wsc[S], wzp[S];  // raw float16 bits / zero points, converted where used
#pragma unroll
    for (int s = 0; s < S; s++) {
        const int c = 4 * s + j;
        const uint32_t gi = (uint32_t)((tile * a.NG + (c >> a.cpg_shift)) * 16 + r);
        wc[s] = bload16(rc, gemv_wave ? (uint32_t)(((tile * a.CK + c) * 16 + r) * 16) : kOOB);
        wsc[s] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)(gemv_wave ? gi * 2u : kOOB), 0, 0);
        wzp[s] = __builtin_amdgcn_raw_buffer_load_b8(rz, (int)(gemv_wave ? gi : kOOB), 0, 0);
    }
    const float brow = __uint_as_float(bload4(rbias, gemv_wave ? (uint32_t)row * 4u : kOOB));
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t cache_bytes = (uint32_t)((int64_t)(a.layer + 1) * a.max_t * a.n_head * kHD);
    const auto rk = rsrc(a.K8, cache_bytes), rv = rsrc(a.V8, cache_bytes);
    const auto rks = rsrc(a.KS, cache_bytes / kHD * 4), rvs = rsrc(a.VS, cache_bytes / kHD * 4);
    const bool past = tid < cur;
    const uint32_t slot = (uint32_t)(base + (int64_t)tid * a.n_head);
    v4i kr[4], vr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        kr[i] = bload16(rk, past ? slot * kHD + 16u * i : kOOB);
        vr[i] = bload16(rv, past ? slot * kHD + 16u * i : kOOB);
    }
    float ksr = __uint_as_float(bload4(rks, past ? slot * 4u : kOOB));
    const float vsr = __uint_as_float(bload4(rvs, past ? slot * 4u : kOOB));
    const float4 xv = make_float4(__int_as_float(xi[0]), __int_as_float(xi[1]), __int_as_float(xi[2]),
                                  __int_as_float(xi[3]));
    const float4 lw = make_float4(__int_as_float(lwi[0]), __int_as_float(lwi[1]), __int_as_float(lwi[2]),
                                  __int_as_float(lwi[3]));
    const float4 lb = make_float4(__int_as_float(lbi[0]), __int_as_float(lbi[1]), __int_as_float(lbi[2]),
                                  __int_as_float(lbi[3]));
    __builtin_amdgcn_sched_barrier(0);

    // 2. LayerNorm and int16 codes of the row; nibble planes of
    //    X = xq + 32768 and per-chunk sums of xq into LDS.
    const float mean = block_sum((xv.x + xv.y) + (xv.z + xv.w), red) / (float)C;
    float sq = 0.0f;
    if (has) {
        const float d0 = xv.x - mean, d1 = xv.y - mean, d2 = xv.z - mean, d3 = xv.w - mean;
        sq = (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
    const float var = block_sum(sq, red) / (float)C;
    const float rstd = 1.0f / sqrtf(var + 1e-5f);
    float xn[4] = {((xv.x - mean) * rstd) * lw.x + lb.x, ((xv.y - mean) * rstd) * lw.y + lb.y,
                   ((xv.z - mean) * rstd) * lw.z + lb.z, ((xv.w - mean) * rstd) * lw.w + lb.w};
    float m = 0.0f;
    if (has) m = fmaxf(fmaxf(fabsf(xn[0]), fabsf(xn[1])), fmaxf(fabsf(xn[2]), fabsf(xn[3])));
    m = block_max(m, red);
    float sx = m / 32767.0f;
    if (sx == 0.0f) sx = 1.0f;
    const float inv = 1.0f / sx;
    int qs = 0;
    uint32_t pl[4] = {0, 0, 0, 0};  // 16-bit halves of the four plane dwords
    if (has) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int q = round_to_int(xn[e] * inv);
            qs += q;
            const uint32_t X = (uint32_t)(q + 32768);
#pragma unroll
            for (int p = 0; p < 4; p++) pl[p] |= ((X >> (4 * p)) & 15u) << (4 * e);
        }
    }
    // unit u: chunk u / 8, dword (u % 8) / 2, nibbles 4 (u % 2) .. +3
    qs += __shfl_xor(qs, 1);
    qs += __shfl_xor(qs, 2);
    qs += __shfl_xor(qs, 4);
    if (has) {
        uint16_t *p16 = reinterpret_cast<uint16_t *>(planes);
        const int c = tid >> 3, i = (tid & 7) >> 1, half = tid & 1;
#pragma unroll
        for (int p = 0; p < 4; p++) p16[((c * 4 + i) * 4 + p) * 2 + half] = (uint16_t)pl[p];
        if ((tid & 7) == 0) xsum[c] = qs;
    }
    lds_barrier();

    // 3. The head's 192 qkv rows: exact chunk sums, float accumulation.
    if (gemv_wave) {
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int c = 4 * s + j;
            const uint4 *P = reinterpret_cast<const uint4 *>(planes + c * 16);
            const uint32_t w[4] = {(uint32_t)wc[s][0], (uint32_t)wc[s][1], (uint32_t)wc[s][2], (uint32_t)wc[s][3]};
            uint32_t d0 = 0, d1 = 0, d2 = 0, d3 = 0, su = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 q = P[i];
                d0 = __builtin_amdgcn_udot8(q.x, w[i], d0, false);
                d1 = __builtin_amdgcn_udot8(q.y, w[i], d1, false);
                d2 = __builtin_amdgcn_udot8(q.z, w[i], d2, false);
                d3 = __builtin_amdgcn_udot8(q.w, w[i], d3, false);
                su = __builtin_amdgcn_udot8(0x11111111u, w[i], su, false);
            }
            // sum X u - 32768 sum u - zp sum xq, exact in int32
            const int G = (int)(d0 + (d1 << 4) + (d2 << 8) + (d3 << 12)) - (int)(su << 15) -
                          (int)wzp[s] * xsum[c];
            acc = fmaf((float)G, __half2float(__ushort_as_half((unsigned short)wsc[s])), acc);
        }
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        if (j == 0) {
            const float y = acc * sx + brow;
            head[blk][(wid & 3) * 16 + r] = y;
            a.qkv_out[row] = y;
        }
    }
    lds_barrier();

    // 4. QuantKV.store of the new key (wave 12) and value (wave 13): codes
    //    and scales to the cache, and copies in LDS for this workgroup.
    if (wid == 12 || wid == 13) {
        const int kv = wid - 12;
        const float v = head[1 + kv][lane];
        const float mx = wave_max(fabsf(v));
        float sc = mx / 127.0f;
        if (sc == 0.0f) sc = 1.0f;
        const float vinv = 1.0f / sc;
        const int8_t code = (int8_t)llmq_to_int(roundf(v * vinv));
        const int64_t sl = base + (int64_t)cur * a.n_head;
        (kv ? a.V8 : a.K8)[sl * kHD + lane] = code;
        (kv ? vrow : krow)[(int64_t)cur * kHD + lane] = code;
        if (lane == 0) {
            (kv ? a.VS : a.KS)[sl] = sc;
            if (kv == 0)
                kscale_new = sc;
            else
                vsc[cur] = sc;
        }
    }
    // cached key and value rows into LDS (position tid), as loaded: no
    // register holds unpacked codes across the projection
    if (past) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *reinterpret_cast<v4i *>(krow + (int64_t)tid * kHD + 16 * i) = kr[i];
            *reinterpret_cast<v4i *>(vrow + (int64_t)tid * kHD + 16 * i) = vr[i];
        }
        vsc[tid] = vsr;
    }
    lds_barrier();

    // 5. attend_float_one: scores q . k * ks / sqrt(64), softmax, values.
    const float scale = 1.0f / sqrtf((float)kHD);
    float sc_mine = -INFINITY;
    if (tid < npos) {
        if (tid == cur) ksr = kscale_new;  // (the load above returned 0 for it)
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const v4i k4 = *reinterpret_cast<const v4i *>(krow + (int64_t)tid * kHD + 16 * i);
            const int8_t *b8 = reinterpret_cast<const int8_t *>(&k4);
#pragma unroll
            for (int e = 0; e < 16; e++) d = fmaf(head[0][16 * i + e], (float)b8[e], d);
        }
        sc_mine = d * ksr * scale;
    }
    const float mx = block_max(sc_mine, red);
    float ex = 0.0f;
    if (tid < npos) {
        ex = ref_expf(sc_mine - mx);
        scores[tid] = ex;
    }
    const float total = block_sum(ex, red);
    // Each position's weight p * vs once (p = e / total), by its own thread.
    if (tid < npos) scores[tid] = (ex / total) * vsc[tid];
    lds_barrier();
    const int i = lane;  // output dimension
    float acc = 0.0f;
    for (int s = wid; s < npos; s += kNW) acc = fmaf(scores[s], (float)vrow[(int64_t)s * kHD + i], acc);
    part[wid][i] = acc;
    lds_barrier();
    if (tid < kHD) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kNW; w++) v += part[w][tid];
        a.att[h * kHD + tid] = v;
    }
}

template <int S>
int launch_s(llmq_ctx *ctx, const QkvAttnArgs &a, int n_head, size_t lds) {
    static size_t granted = 64 * 1024;
    if (lds > granted) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&qkv_attn_kernel<S>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    hipLaunchKernelGGL(qkv_attn_kernel<S>, dim3(n_head), dim3(kNT), lds, ctx->stream, a);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

}  // namespace

// Fused qkv GEMV + KV store + attention for one decode token, when the
// shapes allow it (int4 A16 qkv, head_dim 64, float cache, max_t <= 1024,
// C = 768); returns LLMQ_EUNSUPPORTED otherwise so the
// caller can run the two kernels instead.
int launch_qkv_attn(llmq_ctx *ctx, const llmq_mat *w, const float *x, const float *ln_w, const float *ln_b,
                    const float *bias, llmq_kv *kv, int layer, int pos0, const int *pos_dev, float *qkv_out,
                    float *att) {
    const int C = kv->n_head * kv->head_dim;
    if (w->kind != MAT_QUANT || w->bits != 4 || !w->a16 || kv->integer || kv->head_dim != kHD ||
        kv->max_t > kNT || w->k != C || w->n != 3 * C || w->CK % 4 != 0 || w->CK > kMaxCK || C / 4 > kNT)
        return LLMQ_EUNSUPPORTED;
    int cpg = (int)(w->group / 32), shift = 0;
    while ((1 << shift) < cpg) shift++;
    if ((1 << shift) != cpg) return LLMQ_EUNSUPPORTED;
    LLMQ_REQUIRE(pos_dev || (pos0 >= 0 && pos0 < kv->max_t), "qkv_attn: position %d beyond %d", pos0, kv->max_t);
    QkvAttnArgs a;
    a.codes = reinterpret_cast<const uint4 *>(w->codes);
    a.scales = w->scales;
    a.zps = w->zps;
    a.CK = (int)w->CK;
    a.NG = (int)w->NG;
    a.cpg_shift = shift;
    a.x = x;
    a.ln_w = ln_w;
    a.ln_b = ln_b;
    a.bias = bias;
    a.C = C;
    a.K8 = kv->k;
    a.V8 = kv->v;
    a.KS = kv->ks;
    a.VS = kv->vs;
    a.layer = layer;
    a.max_t = kv->max_t;
    a.n_head = kv->n_head;
    a.pos_dev = pos_dev;
    a.pos0 = pos0;
    a.qkv_out = qkv_out;
    a.att = att;
    const size_t lds = (size_t)kv->max_t * (8 + 2 * kHD);
    switch (w->CK / 4) {
    case 6: return launch_s<6>(ctx, a, kv->n_head, lds);  // C = 768 (GPT-2 124M); wider rows would spill
    default: return LLMQ_EUNSUPPORTED;
    }
}
