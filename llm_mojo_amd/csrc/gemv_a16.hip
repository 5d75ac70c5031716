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
constexpr int kSteps = 8;  // code steps per wave whose loads are all issued before the first use

struct GemvArgs {
    const uint4 *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    int n, K, ntiles, CK, NG, cpg_shift, T, ks, flags;  // group of chunk c: c >> cpg_shift
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
// Workgroup barrier that orders LDS only: global loads issued before it stay
// in flight (the weight stream overlaps the prologue).  Nothing in these
// kernels communicates through global memory inside a launch.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Sum / max over the 256 threads; every thread gets the same bits.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    lds_barrier();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    return ((red[0] + red[1]) + red[2]) + red[3];
}
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max(v);
    lds_barrier();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Activations of one token row in registers: unit u = tid + 256 * i holds
// VPT consecutive values (one plane dword of the int4 / int8 layout).
template <int VPT, int UPT>
__device__ __forceinline__ void load_units(const float *__restrict__ xr, int nunits, float (&v)[UPT][VPT]) {
    const float4 *x4 = reinterpret_cast<const float4 *>(xr);
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = threadIdx.x + kThreads * i;
        const bool ok = u < nunits;
        const int uc = ok ? u : 0;  // always a valid address: no branch around the load
#pragma unroll
        for (int h = 0; h < VPT / 4; h++) {
            const float4 f = x4[uc * (VPT / 4) + h];
            v[i][4 * h] = ok ? f.x : 0.0f;
            v[i][4 * h + 1] = ok ? f.y : 0.0f;
            v[i][4 * h + 2] = ok ? f.z : 0.0f;
            v[i][4 * h + 3] = ok ? f.w : 0.0f;
        }
    }
}

// One token row, from registers: optional LayerNorm (kernels.mojo:179-197),
// quantize_rows (kernels.mojo:400-416), then the activation planes and
// per-chunk sums into LDS.  Returns the row's scale sx.
template <int BITS, int UPT, bool LN>
__device__ float prep_token(const GemvArgs &a, float (&v)[UPT][BITS == 4 ? 8 : 4],
                            const float (&lw)[UPT][BITS == 4 ? 8 : 4], const float (&lb)[UPT][BITS == 4 ? 8 : 4],
                            uint32_t *xpl, int *xsum, float *red, int16_t *xq_dbg) {
    constexpr int VPT = BITS == 4 ? 8 : 4;  // activations per unit (one plane dword)
    constexpr int PD = BITS == 4 ? 16 : 8;  // plane dwords per chunk
    const int K = a.K, nunits = K / VPT, tid = threadIdx.x;
    if (LN) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < UPT; i++)
#pragma unroll
            for (int e = 0; e < VPT; e++) sum += v[i][e];  // padding units hold zeros
        const float mean = block_sum(sum, red) / (float)K;
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            if (tid + kThreads * i >= nunits) continue;
#pragma unroll
            for (int e = 0; e < VPT; e++) {
                float d = v[i][e] - mean;
                sq += d * d;
            }
        }
        const float var = block_sum(sq, red) / (float)K;
        const float rstd = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
        for (int i = 0; i < UPT; i++)
#pragma unroll
            for (int e = 0; e < VPT; e++) {
                float nn = (v[i][e] - mean) * rstd;
                v[i][e] = nn * lw[i][e] + lb[i][e];
            }
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        if (tid + kThreads * i >= nunits) continue;
#pragma unroll
        for (int e = 0; e < VPT; e++) m = fmaxf(m, fabsf(v[i][e]));
    }
    m = block_max(m, red);
    float s = m / 32767.0f;
    if (s == 0.0f) s = 1.0f;
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + kThreads * i;
        if (u >= nunits) continue;  // whole groups of four units drop out together
        uint32_t p[4] = {0, 0, 0, 0};
        int qs = 0;
#pragma unroll
        for (int e = 0; e < VPT; e++) {
            const int q = llmq_to_int(roundf(v[i][e] * inv));
            if (xq_dbg) xq_dbg[u * VPT + e] = (int16_t)q;
            qs += q;
            const uint32_t X = (uint32_t)(q + 32768);
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
        const int c = u >> 2, ii = u & 3;  // four units fill one chunk
#pragma unroll
        for (int pl = 0; pl < PD / 4; pl++) xpl[c * PD + pl * 4 + ii] = p[pl];
        qs += __shfl_xor(qs, 1);
        qs += __shfl_xor(qs, 2);
        if (ii == 0) xsum[c] = qs;
    }
    return s;
}

template <int BITS, int MT, bool LN, bool DBG, int UPT, bool LOOP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void gemv_a16_kernel(GemvArgs a) {
    constexpr int VPT = BITS == 4 ? 8 : 4;
    constexpr int PD = BITS == 4 ? 16 : 8;
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ float part[4 * MT * 16];
    __shared__ float pre_red[4];
    __shared__ float s_sx[MT];
    __shared__ ArgmaxPart s_best[4];

    const int CK = a.CK;
    uint32_t *xpl = smem;                                      // [MT][CK][PD]
    int *xsum = reinterpret_cast<int *>(smem + MT * CK * PD);  // [MT][CK]
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int tpw = 4 / a.ks;
    const int tile = blockIdx.x * tpw + wid / a.ks;
    const int kpart = wid % a.ks;
    const int S = (CK + 3) >> 2;
    const int s0 = (S * kpart) / a.ks, s1 = (S * (kpart + 1)) / a.ks;
    const int r = lane & 15, j = lane >> 4;
    const bool tile_ok = tile < a.ntiles;
    const int o = tile * 16 + r;
    const bool row_ok = tile_ok && o < a.n;
    const int tb = blockIdx.y, tok0 = tb * MT;
    const int nunits = a.K / VPT;

    // 1. Everything the epilogue reads, and the first token's activations,
    //    are requested first: nothing later waits behind the weight stream.
    const int oc = row_ok ? o : 0;  // clamped row: loads need no branch
    float e_bias = 0.0f, e_res = 0.0f;
    if (MT == 1) {
        e_bias = a.bias[oc];  // a.bias is valid memory even without LLMQ_BIAS
        e_res = a.out[(size_t)tok0 * a.ldo + oc];
    }
    float xv[UPT][VPT], lw[UPT][VPT], lb[UPT][VPT];
    load_units<VPT, UPT>(a.x + (size_t)tok0 * a.ldx, nunits, xv);
    if (LN) {
        load_units<VPT, UPT>(a.ln_w, nunits, lw);
        load_units<VPT, UPT>(a.ln_b, nunits, lb);
    }

    // 2. The wave's code chunks (up to kSteps steps), scales and zero points.
    //    Loads are never behind a branch and use 32-bit offsets from the
    //    matrix base, so the compiler counts them precisely and waits for
    //    each only where it is used.  Steps past the wave's range read the
    //    padding that follows every matrix (pad_chunks) and get scale 0.
    const int tile_c = tile_ok ? tile : 0;
    const uint32_t code_lane = ((uint32_t)tile_c * CK * 16u + (uint32_t)j * 16u + (uint32_t)r);  // in uint4
    const uint32_t grp_lane = (uint32_t)tile_c * a.NG * 16u + (uint32_t)r;
    uint4 wc[kSteps];
    uint32_t wsc[kSteps], wzp[kSteps];
    auto fetch = [&](int sb) {
#pragma unroll
        for (int u = 0; u < kSteps; u++) {
            const uint32_t s = (uint32_t)(sb + u);
            wc[u] = a.codes[code_lane + s * 64u];
            const uint32_t gi = grp_lane + ((4u * s + (uint32_t)j) >> a.cpg_shift) * 16u;
            wsc[u] = a.scales[gi];
            wzp[u] = a.zps[gi];
        }
    };
    // Issue order matters: the prologue needs x before any weight has
    // arrived, and vmcnt counts completions in issue order.
    __builtin_amdgcn_sched_barrier(0);
    fetch(s0);
    __builtin_amdgcn_sched_barrier(0);

    // 3. Prologue, overlapping the code loads: the token block's activations,
    //    quantized, into LDS.  Token 0 is straight-line code so its x loads
    //    stay ahead of the weight loads.
    {
        int16_t *dbgq = (a.xq_out && blockIdx.x == 0) ? a.xq_out + (size_t)tok0 * a.K : nullptr;
        const float s = prep_token<BITS, UPT, LN>(a, xv, lw, lb, xpl, xsum, pre_red, dbgq);
        if (tid == 0) {
            s_sx[0] = s;
            if (a.sx_out && blockIdx.x == 0) a.sx_out[tok0] = s;
        }
    }
    for (int t = 1; t < MT; t++) {
        const int tok = tok0 + t;
        if (tok >= a.T) break;
        load_units<VPT, UPT>(a.x + (size_t)tok * a.ldx, nunits, xv);
        int16_t *dbgq = (a.xq_out && blockIdx.x == 0) ? a.xq_out + (size_t)tok * a.K : nullptr;
        const float s = prep_token<BITS, UPT, LN>(a, xv, lw, lb, xpl + t * CK * PD, xsum + t * CK, pre_red, dbgq);
        if (tid == 0) {
            s_sx[t] = s;
            if (a.sx_out && blockIdx.x == 0) a.sx_out[tok] = s;
        }
    }
    lds_barrier();

    // 4. Integer sums per chunk, float accumulation per row.  Single-batch
    //    kernels (every wave has at most kSteps steps) are straight-line code;
    //    LOOP kernels walk longer reduction axes one batch at a time.
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) acc[t] = 0.0f;
    for (int sb = s0; sb < s1; sb += kSteps) {
        if (LOOP && sb != s0) {
            __builtin_amdgcn_sched_barrier(0);
            fetch(sb);
        }
#pragma unroll
        for (int u = 0; u < kSteps; u++) {
            const int ss = sb + u;
            const bool ok = tile_ok && ss < s1 && 4 * ss + j < CK;
            const int c = ok ? 4 * ss + j : 0;  // LDS reads stay in range; scale is 0
            const float scale = ok ? __half2float(__ushort_as_half((unsigned short)wsc[u])) : 0.0f;
            const int zp = (int)wzp[u];
            const uint4 d = wc[u];
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
                    uint32_t Sp[4];
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        const uint4 q = P[p];
                        uint32_t v = __builtin_amdgcn_udot8(q.x, d.x, 0u, false);
                        v = __builtin_amdgcn_udot8(q.y, d.y, v, false);
                        v = __builtin_amdgcn_udot8(q.z, d.z, v, false);
                        Sp[p] = __builtin_amdgcn_udot8(q.w, d.w, v, false);
                    }
                    xu = Sp[0] + (Sp[1] << 4) + (Sp[2] << 8) + (Sp[3] << 12);
                } else {
                    uint32_t Sp[2];
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        const uint4 q = P[p];
                        uint32_t v = __builtin_amdgcn_udot4(q.x, d.x, 0u, false);
                        v = __builtin_amdgcn_udot4(q.y, d.y, v, false);
                        v = __builtin_amdgcn_udot4(q.z, d.z, v, false);
                        Sp[p] = __builtin_amdgcn_udot4(q.w, d.w, v, false);
                    }
                    xu = Sp[0] + (Sp[1] << 8);
                }
                const int G = (int)(xu - 32768u * su) - zp * xsum[t * CK + c];
                if (DBG && row_ok && ok) a.dbg[(size_t)o * CK + c] = G;
                acc[t] = fmaf((float)G, scale, acc[t]);
                // Keep each (step, token)'s LDS reads next to their use: without
                // this the scheduler hoists them all and runs out of registers.
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (!LOOP) break;
    }

    // 5. Rows: sum the four lanes of a row, then the ks waves of a tile.
#pragma unroll
    for (int t = 0; t < MT; t++) {
        acc[t] += __shfl_xor(acc[t], 16);
        acc[t] += __shfl_xor(acc[t], 32);
    }
    if (a.ks > 1) {
        if (j == 0)
            for (int t = 0; t < MT; t++) part[(wid * MT + t) * 16 + r] = acc[t];
        lds_barrier();
        if (kpart == 0)
            for (int t = 0; t < MT; t++) {
                float v = 0.0f;
                for (int q = 0; q < a.ks; q++) v += part[((wid + q) * MT + t) * 16 + r];
                acc[t] = v;
            }
    }

    // 6. Epilogue: scale, bias, GELU, residual, store.
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    if (kpart == 0 && row_ok) {
        for (int t = 0; t < MT; t++) {
            const int tok = tok0 + t;
            if (tok >= a.T) break;
            float v = acc[t] * s_sx[t];
            if (a.flags & LLMQ_BIAS) v += MT == 1 ? e_bias : a.bias[o];
            if (a.flags & LLMQ_GELU) v = gelu_ref(v);
            float *dst = a.out + (size_t)tok * a.ldo + o;
            if (a.flags & LLMQ_RESID) v += MT == 1 ? e_res : *dst;
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
        lds_barrier();
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
    if (w->ntiles <= 1024) return 4;  // latency-bound sizes: the most waves
    const int64_t S = (w->CK + 3) / 4;
    for (int ks = 1; ks < 4; ks *= 2)
        if ((S + ks - 1) / ks <= kSteps) return ks;
    return 4;
}

template <int BITS, int MT, bool LN, bool DBG, int UPT>
void launch_t(llmq_ctx *ctx, const GemvArgs &a, dim3 grid, size_t lds, bool loop) {
    if (loop)
        hipLaunchKernelGGL((gemv_a16_kernel<BITS, MT, LN, DBG, UPT, true>), grid, dim3(kThreads), lds, ctx->stream, a);
    else
        hipLaunchKernelGGL((gemv_a16_kernel<BITS, MT, LN, DBG, UPT, false>), grid, dim3(kThreads), lds, ctx->stream,
                           a);
}

template <int BITS, int MT, int UPT>
void dispatch_flags(llmq_ctx *ctx, const GemvArgs &a, dim3 grid, size_t lds, bool ln, bool dbg, bool loop) {
    if (MT == 1 && dbg)
        launch_t<BITS, 1, false, true, UPT>(ctx, a, grid, lds, loop);
    else if (ln) {
        if constexpr (UPT <= 2) launch_t<BITS, MT, true, false, UPT>(ctx, a, grid, lds, loop);
    } else {
        launch_t<BITS, MT, false, false, UPT>(ctx, a, grid, lds, loop);
    }
}

template <int BITS, int MT>
void dispatch_upt(llmq_ctx *ctx, const GemvArgs &a, int upt, dim3 grid, size_t lds, bool ln, bool dbg, bool loop) {
    if (upt <= 1)
        dispatch_flags<BITS, MT, 1>(ctx, a, grid, lds, ln, dbg, loop);
    else if (upt <= 2)
        dispatch_flags<BITS, MT, 2>(ctx, a, grid, lds, ln, dbg, loop);
    else if (upt <= 4)
        dispatch_flags<BITS, MT, 4>(ctx, a, grid, lds, ln, dbg, loop);
    else
        dispatch_flags<BITS, MT, 8>(ctx, a, grid, lds, ln, dbg, loop);
}

template <int BITS>
void dispatch_mt(llmq_ctx *ctx, const GemvArgs &a, int mt, int upt, dim3 grid, size_t lds, bool ln, bool dbg,
                 bool loop) {
    if (mt == 8)
        dispatch_upt<BITS, 8>(ctx, a, upt, grid, lds, ln, dbg, loop);
    else if (mt == 4)
        dispatch_upt<BITS, 4>(ctx, a, upt, grid, lds, ln, dbg, loop);
    else
        dispatch_upt<BITS, 1>(ctx, a, upt, grid, lds, ln, dbg, loop);
}

size_t lds_bytes(const llmq_mat *w, int mt) {
    const int PD = w->bits == 4 ? 16 : 8;
    return (size_t)mt * w->CK * PD * 4 + (size_t)mt * w->CK * 4;
}

}  // namespace

int gemv_a16_num_parts(const llmq_mat *w, bool ln) {
    if (exact_order() && gemv_exact_supports(w)) return gemv_exact_num_parts(w);
    if (gemv1_supports(w, ln)) return gemv1_num_parts(w, ln);
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
    // (the int8 head kernel keeps no per-chunk sums: chunk-sum requests for
    // it take gemv1)
    LLMQ_REQUIRE(!rq.kv || rq.T > 1, "linear: the key / value store is for prompts");
    const bool exact = rq.T == 1 && exact_order() && gemv_exact_supports(w) && !(rq.dbg && w->bits == 8);
    LLMQ_REQUIRE(exact || !(rq.emb || rq.state_copy), "linear: the embed step and the state copy need the exact kernel");
    if (exact) return launch_gemv_exact(ctx, rq);
    if (rq.T == 1 && gemv1_supports(w, rq.ln_w != nullptr)) return launch_gemv1(ctx, rq);
    {
        // Prompts: the int8-MFMA GEMM (LN + quantize_rows into workspace
        // first), whose float steps are tile_i16's, from two tokens on
        int min_t = exact_order() ? 2 : 8;
        if (const char *e = getenv("LLMQ_MFMA_MIN_T")) min_t = atoi(e);
        if (rq.T >= min_t && min_t > 0 && gemm_mfma_supports(w, rq.T)) {
            // workspace: int16 codes, token scales, then (int4-g32) the fp16
            // planes; a caller-given workspace too small for the planes runs
            // the int8-MFMA form, whose results are the same bits
            const size_t xb = ((size_t)rq.T * w->k * 2 + 255) & ~(size_t)255;
            const size_t sb = ((size_t)rq.T * 4 + 255) & ~(size_t)255;
            const size_t need = xb + sb;
            const size_t need16 = gemm_f16_supports(w, rq.T) ? need + gemm_f16_planes_bytes(w, rq.T) : 0;
            void *ws = rq.ws;
            bool f16 = need16 > 0;
            if (ws) {
                LLMQ_REQUIRE(need <= rq.ws_cap, "linear: %lld tokens x %lld inputs need %zu bytes of workspace, %zu given",
                             (long long)rq.T, (long long)w->k, need, rq.ws_cap);
                f16 = f16 && need16 <= rq.ws_cap;
            } else {
                RC(ctx_workspace(ctx, f16 ? need16 : need, &ws));
            }
            uint8_t *base = reinterpret_cast<uint8_t *>(ws);
            return launch_gemm_mfma(ctx, rq, reinterpret_cast<int16_t *>(base), reinterpret_cast<float *>(base + xb),
                                    f16 ? base + need : nullptr);
        }
    }
    LLMQ_REQUIRE(!rq.kv, "linear: the key / value store needs the prompt GEMM");
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
    const int64_t cpg = w->group / (w->bits == 4 ? 32 : 16);  // chunks per group
    if (w->NG == 1) {
        a.cpg_shift = 31;  // per-channel: every chunk is group 0
    } else {
        LLMQ_REQUIRE((cpg & (cpg - 1)) == 0, "linear: group %lld is not a power of two times 32",
                     (long long)w->group);
        a.cpg_shift = __builtin_ctzll((unsigned long long)cpg);
    }
    a.T = (int)rq.T;
    a.ks = ks;
    a.flags = rq.flags;
    a.ldx = rq.ldx ? rq.ldx : w->k;
    a.ldo = rq.ldo ? rq.ldo : w->n;
    a.x = rq.x;
    a.ln_w = rq.ln_w;
    a.ln_b = rq.ln_b;
    a.bias = rq.bias ? rq.bias : rq.out;  // read (and ignored) without LLMQ_BIAS
    a.out = rq.out;
    a.amax = rq.amax;
    a.dbg = rq.dbg;
    a.xq_out = rq.xq_out;
    a.sx_out = rq.sx_out;
    dim3 grid((unsigned)((w->ntiles + tpw - 1) / tpw), (unsigned)((rq.T + mt - 1) / mt));
    LLMQ_REQUIRE(!rq.amax || (int64_t)grid.x <= rq.amax_cap, "linear: %u argmax partials exceed capacity %d", grid.x,
                 rq.amax_cap);
    const bool ln = rq.ln_w != nullptr, dbg = rq.dbg != nullptr;
    if (ln && (w->k / (w->bits == 4 ? 8 : 4) + kThreads - 1) / kThreads > 2)
        return llmq_set_error(LLMQ_EUNSUPPORTED, "ln_linear: LayerNorm prologue supports IN <= %d",
                              w->bits == 4 ? 4096 : 2048);
    const int vpt = w->bits == 4 ? 8 : 4;
    const int64_t units = w->k / vpt;
    const int upt = (int)((units + kThreads - 1) / kThreads);
    if (upt > 8)
        return llmq_set_error(LLMQ_EUNSUPPORTED, "linear: reduction axis %lld too long", (long long)w->k);
    const int64_t S = (w->CK + 3) / 4;
    const bool loop = (S + ks - 1) / ks > kSteps;  // some wave has more than one batch
    if (w->bits == 4)
        dispatch_mt<4>(ctx, a, mt, upt, grid, lds, ln, dbg, loop);
    else
        dispatch_mt<8>(ctx, a, mt, upt, grid, lds, ln, dbg, loop);
    LLMQ_HIP(hipGetLastError());
    if (rq.amax_count) *rq.amax_count = (int)grid.x;
    return LLMQ_OK;
}
