// W4A16 / W8A16 matmul over the row-tile layout (common.h): the integer path
// of kernels.matmul_rows_a16 / linear_team (kernels.mojo:419-509, 774-866)
// and QuantMatrix.dot_row_i16 (tensor.mojo:518-577).
//
// Per output row o and 16-byte code chunk c the kernel computes the exact
// integer partial
//     G[o, c] = sum_{k in c} xq_k * (u_{o,k} - zp_{o,g(c)})
// (a chunk never straddles a group: groups are multiples of 32 weights), adds
// G * scale_g into a float32 accumulator, and finishes with
//     y_o = act(acc_o * sx + b_o) (+ y_o for the residual).
//
// Integer sums use unsigned dot products on planes of the activations:
// X = xq + 32768 is a 16-bit unsigned value, split into four 4-bit planes
// (int4 weights, v_dot8_u32_u4 against the raw nibbles) or two 8-bit planes
// (int8 weights, v_dot4_u32_u8 against the raw bytes).  Then
//     sum X*u = sum_p 16^p * S_p   (or S_lo + 256 * S_hi)
//     sum x*u = sum X*u - 32768 * sum u
//     G       = sum x*u - zp * sum x
// with sum u from the same dot instruction against a ones pattern and sum x
// per chunk computed once per token in the prologue.  No intermediate
// exceeds 2^31: a chunk of 32 int4 or 16 int8 products stays below 2.7e8.
//
// Work mapping: a wave owns one 16-row tile and a slice of the reduction
// axis; lane (r, j) = (lane % 16, lane / 16) reads chunk 4s + j of row r at
// step s, so one 128-bit load per lane covers 1 KiB of contiguous codes.  A
// workgroup of four waves holds 4 / ks tiles, each split over ks waves whose
// partial sums meet in LDS in a fixed order (results are deterministic).
// The prologue (LayerNorm if requested, then quantize_rows) runs in every
// workgroup on its token block while the first code loads are in flight.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPrefetch = 4;  // steps of code loads kept in flight per lane

struct GemvArgs {
    const uint4 *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    int n, K, ntiles, CK, NG, CPG, T, ks, flags;
    int64_t ldx, ldo;
    const float *x, *ln_w, *ln_b, *bias;
    float *out;
    ArgmaxPart *amax;
    int32_t *dbg;
    int16_t *xq_out;
    float *sx_out;
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
// Sum / max over the 256 threads; every thread gets the same bits.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// GELU of kernels.store_out (kernels.mojo:43-45), operation by operation.
__device__ __forceinline__ float gelu_f(float r) {
    const float s = 0.7978845608028654f;
    float t = 0.044715f * r;
    t = t * r;
    t = t * r;
    float u = r + t;
    float th = tanhf(s * u);
    float h = 0.5f * r;
    return h * (1.0f + th);
}

// One token row: optional LayerNorm (kernels.mojo:179-197), quantize_rows
// (kernels.mojo:400-416), then the activation planes and per-chunk sums.
template <int BITS, bool LN>
__device__ void prep_token(const GemvArgs &a, const float *__restrict__ xr, uint32_t *xpl, int *xsum, float *red,
                           float &s_out, int16_t *xq_dbg) {
    const int K = a.K, tid = threadIdx.x;
    const float4 *x4 = reinterpret_cast<const float4 *>(xr);
    float mean = 0.0f, rstd = 1.0f;
    if (LN) {
        float sum = 0.0f;
        for (int i = tid; i < K / 4; i += kThreads) {
            float4 v = x4[i];
            sum += ((v.x + v.y) + v.z) + v.w;
        }
        mean = block_sum(sum, red) / (float)K;
        float sq = 0.0f;
        for (int i = tid; i < K / 4; i += kThreads) {
            float4 v = x4[i];
            float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
            sq += ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
        }
        float var = block_sum(sq, red) / (float)K;
        rstd = 1.0f / sqrtf(var + 1e-5f);
    }
    auto xn = [&](int i, float v) -> float {
        if (!LN) return v;
        float nn = (v - mean) * rstd;
        return nn * a.ln_w[i] + a.ln_b[i];
    };
    float m = 0.0f;
    for (int i = tid; i < K / 4; i += kThreads) {
        float4 v = x4[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xn(4 * i, v.x)), fabsf(xn(4 * i + 1, v.y))),
                           fmaxf(fabsf(xn(4 * i + 2, v.z)), fabsf(xn(4 * i + 3, v.w)))));
    }
    m = block_max(m, red);
    float s = m / 32767.0f;
    if (s == 0.0f) s = 1.0f;
    const float inv = 1.0f / s;
    s_out = s;
    constexpr int VPT = BITS == 4 ? 8 : 4;  // activations per thread per step (one plane dword)
    constexpr int PD = BITS == 4 ? 16 : 8;  // plane dwords per chunk
    for (int g = tid; g < K / VPT; g += kThreads) {
        float vals[VPT];
#pragma unroll
        for (int h = 0; h < VPT / 4; h++) {
            float4 v = x4[g * (VPT / 4) + h];
            vals[4 * h] = v.x;
            vals[4 * h + 1] = v.y;
            vals[4 * h + 2] = v.z;
            vals[4 * h + 3] = v.w;
        }
        uint32_t p[4] = {0, 0, 0, 0};
        int qs = 0;
#pragma unroll
        for (int e = 0; e < VPT; e++) {
            int q = llmq_to_int(roundf(xn(g * VPT + e, vals[e]) * inv));
            if (xq_dbg) xq_dbg[g * VPT + e] = (int16_t)q;
            qs += q;
            uint32_t X = (uint32_t)(q + 32768);
            if (BITS == 4) {
                p[0] |= (X & 15u) << (4 * e);
                p[1] |= ((X >> 4) & 15u) << (4 * e);
                p[2] |= ((X >> 8) & 15u) << (4 * e);
                p[3] |= (X >> 12) << (4 * e);
            } else {
                p[0] |= (X & 255u) << (8 * e);
                p[1] |= (X >> 8) << (8 * e);
            }
        }
        const int c = g >> 2, i = g & 3;  // four threads fill one chunk
#pragma unroll
        for (int pl = 0; pl < PD / 4; pl++) xpl[c * PD + pl * 4 + i] = p[pl];
        qs += __shfl_xor(qs, 1);
        qs += __shfl_xor(qs, 2);
        if (i == 0) xsum[c] = qs;
    }
}

template <int BITS, int MT, bool LN, bool PERCH, bool DBG>
__global__ __launch_bounds__(kThreads) void gemv_a16_kernel(GemvArgs a) {
    constexpr int PD = BITS == 4 ? 16 : 8;
    extern __shared__ uint32_t smem[];
    __shared__ float part[4 * MT * 16];
    __shared__ float pre_red[4];
    __shared__ float s_sx[MT];
    __shared__ ArgmaxPart s_best[4];

    const int CK = a.CK;
    uint32_t *xpl = smem;                                // [MT][CK][PD]
    int *xsum = reinterpret_cast<int *>(smem + MT * CK * PD);  // [MT][CK]
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int tpw = 4 / a.ks;
    const int tile = blockIdx.x * tpw + wid / a.ks;
    const int kpart = wid % a.ks;
    const int S = (CK + 3) >> 2;
    const int s0 = (S * kpart) / a.ks, s1 = (S * (kpart + 1)) / a.ks;
    const int r = lane & 15, j = lane >> 4;
    const bool tile_ok = tile < a.ntiles;
    const uint4 *cb = a.codes + (size_t)tile * CK * 16 + r;
    const size_t sbase = (size_t)tile * a.NG * 16 + r;

    uint4 buf[kPrefetch];
    uint32_t bsc[kPrefetch], bzp[kPrefetch];
    auto fetch = [&](int s, uint4 &d, uint32_t &sc, uint32_t &zp) {
        const int c = 4 * s + j;
        if (tile_ok && s < s1 && c < CK) {
            d = cb[(size_t)c * 16];
            if (!PERCH) {
                const size_t gi = sbase + (size_t)(c / a.CPG) * 16;
                sc = a.scales[gi];
                zp = a.zps[gi];
            }
        } else {
            d = make_uint4(0, 0, 0, 0);
            sc = 0;
            zp = 0;
        }
    };
#pragma unroll
    for (int u = 0; u < kPrefetch; u++) fetch(s0 + u, buf[u], bsc[u], bzp[u]);
    float psc = 0.0f;
    int pzp = 0;
    if (PERCH && tile_ok) {
        psc = __half2float(__ushort_as_half(a.scales[sbase]));
        pzp = a.zps[sbase];
    }

    // Prologue: the token block's activations, quantized, into LDS.
    const int tb = blockIdx.y;
    for (int t = 0; t < MT; t++) {
        const int tok = tb * MT + t;
        if (tok < a.T) {
            float s;
            int16_t *dbgq = (a.xq_out && blockIdx.x == 0) ? a.xq_out + (size_t)tok * a.K : nullptr;
            prep_token<BITS, LN>(a, a.x + (size_t)tok * a.ldx, xpl + t * CK * PD, xsum + t * CK, pre_red, s, dbgq);
            if (tid == 0) {
                s_sx[t] = s;
                if (a.sx_out && blockIdx.x == 0) a.sx_out[tok] = s;
            }
        }
    }
    __syncthreads();

    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;

    for (int s = s0; s < s1; s += kPrefetch) {
        uint4 cur[kPrefetch];
        uint32_t csc[kPrefetch], czp[kPrefetch];
#pragma unroll
        for (int u = 0; u < kPrefetch; u++) {
            cur[u] = buf[u];
            csc[u] = bsc[u];
            czp[u] = bzp[u];
        }
#pragma unroll
        for (int u = 0; u < kPrefetch; u++) fetch(s + kPrefetch + u, buf[u], bsc[u], bzp[u]);
#pragma unroll
        for (int u = 0; u < kPrefetch; u++) {
            const int ss = s + u, c = 4 * ss + j;
            if (!(tile_ok && ss < s1 && c < CK)) continue;
            const float scale = PERCH ? psc : __half2float(__ushort_as_half((unsigned short)csc[u]));
            const int zp = PERCH ? pzp : (int)czp[u];
            const uint4 d = cur[u];
            uint32_t su;
            if (BITS == 4) {
                su = __builtin_amdgcn_udot8(d.x, 0x11111111u, 0u, false);
                su = __builtin_amdgcn_udot8(d.y, 0x11111111u, su, false);
                su = __builtin_amdgcn_udot8(d.z, 0x11111111u, su, false);
                su = __builtin_amdgcn_udot8(d.w, 0x11111111u, su, false);
            } else {
                su = __builtin_amdgcn_udot4(d.x, 0x01010101u, 0u, false);
                su = __builtin_amdgcn_udot4(d.y, 0x01010101u, su, false);
                su = __builtin_amdgcn_udot4(d.z, 0x01010101u, su, false);
                su = __builtin_amdgcn_udot4(d.w, 0x01010101u, su, false);
            }
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const uint4 *P = reinterpret_cast<const uint4 *>(xpl + (t * CK + c) * PD);
                uint32_t xu;
                if (BITS == 4) {
                    uint32_t S[4];
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        const uint4 q = P[p];
                        uint32_t v = __builtin_amdgcn_udot8(q.x, d.x, 0u, false);
                        v = __builtin_amdgcn_udot8(q.y, d.y, v, false);
                        v = __builtin_amdgcn_udot8(q.z, d.z, v, false);
                        S[p] = __builtin_amdgcn_udot8(q.w, d.w, v, false);
                    }
                    xu = S[0] + (S[1] << 4) + (S[2] << 8) + (S[3] << 12);
                } else {
                    uint32_t S[2];
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        const uint4 q = P[p];
                        uint32_t v = __builtin_amdgcn_udot4(q.x, d.x, 0u, false);
                        v = __builtin_amdgcn_udot4(q.y, d.y, v, false);
                        v = __builtin_amdgcn_udot4(q.z, d.z, v, false);
                        S[p] = __builtin_amdgcn_udot4(q.w, d.w, v, false);
                    }
                    xu = S[0] + (S[1] << 8);
                }
                const int G = (int)(xu - 32768u * su) - zp * xsum[t * CK + c];
                if (DBG) {
                    const int o = tile * 16 + r;
                    if (o < a.n) a.dbg[(size_t)o * CK + c] = G;
                }
                acc[t] = fmaf((float)G, scale, acc[t]);
            }
        }
    }

    // Rows: sum the four lanes of a row, then the ks waves of a tile.
#pragma unroll
    for (int t = 0; t < MT; t++) {
        acc[t] += __shfl_xor(acc[t], 16);
        acc[t] += __shfl_xor(acc[t], 32);
    }
    if (a.ks > 1) {
        if (j == 0)
            for (int t = 0; t < MT; t++) part[(wid * MT + t) * 16 + r] = acc[t];
        __syncthreads();
        if (kpart == 0)
            for (int t = 0; t < MT; t++) {
                float v = 0.0f;
                for (int q = 0; q < a.ks; q++) v += part[((wid + q) * MT + t) * 16 + r];
                acc[t] = v;
            }
    }

    const int o = tile * 16 + r;
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    if (kpart == 0 && tile_ok && o < a.n) {
        for (int t = 0; t < MT; t++) {
            const int tok = tb * MT + t;
            if (tok >= a.T) break;
            float v = acc[t] * s_sx[t];
            if (a.flags & LLMQ_BIAS) v += a.bias[o];
            if (a.flags & LLMQ_GELU) v = gelu_f(v);
            float *dst = a.out + (size_t)tok * a.ldo + o;
            if (a.flags & LLMQ_RESID) v += *dst;
            if (j == 0) *dst = v;
            if (MT == 1) {
                best_v = v;
                best_i = o;
            }
        }
    }
    if (MT == 1 && a.amax) {
        // Largest logit of the workgroup; equal values keep the smaller index
        // (argmax's first maximum, gpt2t.mojo:792-797).
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            float ov = __shfl_xor(best_v, off);
            int oi = __shfl_xor(best_i, off);
            if (ov > best_v || (ov == best_v && oi < best_i)) {
                best_v = ov;
                best_i = oi;
            }
        }
        if (lane == 0 && kpart == 0) s_best[wid / a.ks] = ArgmaxPart{best_v, best_i};
        __syncthreads();
        if (tid == 0) {
            ArgmaxPart b = s_best[0];
            for (int q = 1; q < tpw; q++) {
                ArgmaxPart c = s_best[q];
                if (c.v > b.v || (c.v == b.v && c.idx < b.idx)) b = c;
            }
            a.amax[blockIdx.x] = b;
        }
    }
}

int pick_ks(const llmq_mat *w, int64_t T) {
    if (const char *e = getenv("LLMQ_GEMV_KS")) {
        int v = atoi(e);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    if (T > 1) return 1;
    if (w->ntiles >= 2048) return 1;
    if (w->ntiles >= 1024) return 2;
    return 4;
}

template <int BITS, int MT, bool LN, bool PERCH, bool DBG>
void launch_t(llmq_ctx *ctx, const GemvArgs &a, dim3 grid, size_t lds) {
    hipLaunchKernelGGL((gemv_a16_kernel<BITS, MT, LN, PERCH, DBG>), grid, dim3(kThreads), lds, ctx->stream, a);
}

template <int BITS, int MT, bool LN>
void dispatch_perch(llmq_ctx *ctx, const GemvArgs &a, dim3 grid, size_t lds, bool perch, bool dbg) {
    if (dbg && MT == 1 && !LN) {
        if (perch)
            launch_t<BITS, MT, LN, true, true>(ctx, a, grid, lds);
        else
            launch_t<BITS, MT, LN, false, true>(ctx, a, grid, lds);
    } else if (perch) {
        launch_t<BITS, MT, LN, true, false>(ctx, a, grid, lds);
    } else {
        launch_t<BITS, MT, LN, false, false>(ctx, a, grid, lds);
    }
}

template <int BITS, int MT>
void dispatch_ln(llmq_ctx *ctx, const GemvArgs &a, dim3 grid, size_t lds, bool ln, bool perch, bool dbg) {
    if (ln)
        dispatch_perch<BITS, MT, true>(ctx, a, grid, lds, perch, dbg);
    else
        dispatch_perch<BITS, MT, false>(ctx, a, grid, lds, perch, dbg);
}

template <int BITS>
void dispatch_mt(llmq_ctx *ctx, const GemvArgs &a, int mt, dim3 grid, size_t lds, bool ln, bool perch, bool dbg) {
    if (mt == 8)
        dispatch_ln<BITS, 8>(ctx, a, grid, lds, ln, perch, dbg);
    else if (mt == 4)
        dispatch_ln<BITS, 4>(ctx, a, grid, lds, ln, perch, dbg);
    else
        dispatch_ln<BITS, 1>(ctx, a, grid, lds, ln, perch, dbg);
}

size_t lds_bytes(const llmq_mat *w, int mt) {
    const int PD = w->bits == 4 ? 16 : 8;
    return (size_t)mt * w->CK * PD * 4 + (size_t)mt * w->CK * 4;
}

}  // namespace

int gemv_a16_num_parts(const llmq_mat *w) {
    const int ks = pick_ks(w, 1);
    const int tpw = 4 / ks;
    return (int)((w->ntiles + tpw - 1) / tpw);
}

int launch_gemv_a16(llmq_ctx *ctx, const GemvRequest &rq) {
    const llmq_mat *w = rq.w;
    LLMQ_REQUIRE(w && w->kind == MAT_QUANT, "linear: not a QuantMatrix");
    LLMQ_REQUIRE(w->bits == 4 || w->bits == 8, "linear: bits must be 4 or 8");
    LLMQ_REQUIRE(rq.T >= 1, "linear: T must be >= 1");
    LLMQ_REQUIRE(w->k % 32 == 0, "linear: the reduction axis must be a multiple of 32");
    LLMQ_REQUIRE(rq.x && rq.out, "linear: null activation pointer");
    LLMQ_REQUIRE(!(rq.flags & LLMQ_BIAS) || rq.bias, "linear: LLMQ_BIAS without a bias");
    LLMQ_REQUIRE(!rq.amax || rq.T == 1, "linear: argmax partials need T == 1");
    LLMQ_REQUIRE(!rq.dbg || (rq.T == 1 && !rq.ln_w), "linear: chunk sums need T == 1 without LayerNorm");
    const size_t max_lds = 64 * 1024;
    int mt = 1;
    if (rq.T > 1) {
        if (lds_bytes(w, 8) <= max_lds)
            mt = 8;
        else if (lds_bytes(w, 4) <= max_lds)
            mt = 4;
    }
    const size_t lds = lds_bytes(w, mt);
    if (lds > max_lds)
        return llmq_set_error(LLMQ_EUNSUPPORTED, "linear: reduction axis %lld too long for the LDS prologue",
                              (long long)w->k);
    const int ks = pick_ks(w, rq.T);
    const int tpw = 4 / ks;
    GemvArgs a;
    a.codes = reinterpret_cast<const uint4 *>(w->codes);
    a.scales = w->scales;
    a.zps = w->zps;
    a.n = (int)w->n;
    a.K = (int)w->k;
    a.ntiles = (int)w->ntiles;
    a.CK = (int)w->CK;
    a.NG = (int)w->NG;
    a.CPG = (int)(w->group / (w->bits == 4 ? 32 : 16));
    a.T = (int)rq.T;
    a.ks = ks;
    a.flags = rq.flags;
    a.ldx = rq.ldx ? rq.ldx : w->k;
    a.ldo = rq.ldo ? rq.ldo : w->n;
    a.x = rq.x;
    a.ln_w = rq.ln_w;
    a.ln_b = rq.ln_b;
    a.bias = rq.bias;
    a.out = rq.out;
    a.amax = rq.amax;
    a.dbg = rq.dbg;
    a.xq_out = rq.xq_out;
    a.sx_out = rq.sx_out;
    dim3 grid((unsigned)((w->ntiles + tpw - 1) / tpw), (unsigned)((rq.T + mt - 1) / mt));
    LLMQ_REQUIRE(!rq.amax || (int64_t)grid.x <= rq.amax_cap, "linear: %u argmax partials exceed capacity %d", grid.x,
                 rq.amax_cap);
    const bool ln = rq.ln_w != nullptr, perch = w->NG == 1, dbg = rq.dbg != nullptr;
    if (w->bits == 4)
        dispatch_mt<4>(ctx, a, mt, grid, lds, ln, perch, dbg);
    else
        dispatch_mt<8>(ctx, a, mt, grid, lds, ln, perch, dbg);
    LLMQ_HIP(hipGetLastError());
    if (rq.amax_count) *rq.amax_count = (int)grid.x;
    return LLMQ_OK;
}
