// One-token W4A16 / W8A16 GEMV (decode): QuantMatrix.dot_row_i16 over every
// row (tensor.mojo:518-577) as driven by matmul_rows_a16 / linear_team with
// T == 1 (kernels.mojo:419-470, 774-866), with quantize_rows
// (kernels.mojo:400-416) and optionally layernorm (kernels.mojo:179-197)
// fused in front and the store_out / finish epilogue (kernels.mojo:38-48,
// 274-282) behind.
//
// Arithmetic is that of the multi-token kernel (gemv_a16.hip): per 16-byte
// code chunk c of row o the exact integer
//     G[o, c] = sum_{k in c} xq_k * (u_{o,k} - zp_{o,g(c)})
// from unsigned dot products on planes of X = xq + 32768, then
// acc += G * scale and y = act(acc * sx + b) (+ residual).
//
// Work mapping.  A workgroup has NW waves (4 or 16) and owns a contiguous
// run of nt whole row tiles of 16 rows (nt differs by at most one between
// workgroups).  Step s of a tile is chunks 4s..4s+3 of its 16 rows: lane
// (r, j) = (lane % 16, lane / 16) reads chunk 4s + j of row r, so one
// 128-bit load per lane covers 1 KiB of contiguous codes.  The run's nt * S
// steps are split evenly over the waves (a wave may cross one tile
// boundary).  All code loads of a wave (STEPS >= its steps) are issued at
// kernel start, before anything waits; steps past the wave's range repeat
// its last valid address (an L1 hit, no HBM traffic) and get scale 0.
//
// Scales and zero points: the groups a wave touches are contiguous in the
// [tile][group][16] layout, so the wave loads them with one or two 16-byte
// loads per lane and redistributes them through a wave-private LDS slot
// (instead of two narrow loads per step).
//
// The activation prologue (LayerNorm, max |x|, int16 codes, planes) is done
// by every workgroup over the whole row: 16-wave workgroups make this cheap
// for long rows.  Reductions use DPP inside a wave and LDS across waves, in
// a fixed order, so results are identical run to run.
#include "common.h"

namespace {

constexpr int kMaxSteps = 8;
constexpr int kMaxTiles = 8;  // row tiles per workgroup

struct Gemv1Args {
    const uint4 *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    uint32_t codes_bytes, scales_bytes, zps_bytes;  // buffer extents (loads past them read zeros)
    int n, K, ntiles, CK, NG, cpg_shift, tmax, flags;
    const float *x, *ln_w, *ln_b, *bias;
    float *out;
    ArgmaxPart *amax;
    int32_t *dbg;
    int16_t *xq_out;
    float *sx_out;
};

// Buffer loads: an offset at or past the buffer's extent returns zeros
// without touching memory, which is how steps, lanes and units that carry no
// data are disabled without branches or wasted traffic.
constexpr uint32_t kOOB = 0x80000000u;  // every buffer here is below 2 GiB
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float bload4f(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// DPP lane permutations within rows of 16 lanes (every lane active).
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kHalfMirror = 0x141, kRowMirror = 0x140;

// Sum / max over each row of 16 lanes; every lane of the row gets the same
// bits (each step combines two values commutatively).
__device__ __forceinline__ float row_sum(float v) {
    v += dppf<kQuadXor1>(v);
    v += dppf<kQuadXor2>(v);
    v += dppf<kHalfMirror>(v);
    v += dppf<kRowMirror>(v);
    return v;
}
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dppf<kQuadXor1>(v));
    v = fmaxf(v, dppf<kQuadXor2>(v));
    v = fmaxf(v, dppf<kHalfMirror>(v));
    v = fmaxf(v, dppf<kRowMirror>(v));
    return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Wave-uniform sum / max.
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
// Over the workgroup; red must hold NW floats and not be reused by another
// reduction of the same prologue.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NW; i++) s += red[i];
    return s;
}
template <int NW>
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    lds_barrier();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NW; i++) s = fmaxf(s, red[i]);
    return s;
}

// Unit u = threadIdx.x + NT * i holds four consecutive activations
// x[4u..4u+3]; units past the row hold zeros.
template <int NT, int UPT>
__device__ __forceinline__ void load_units(const float *__restrict__ xr, int nunits, float4 (&v)[UPT]) {
    const auto rx = make_rsrc(xr, (uint32_t)nunits * 16u);
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const uint32_t u = threadIdx.x + NT * i;
        const uint4 f = bload16(rx, u < (uint32_t)nunits ? u * 16u : kOOB);
        v[i] = make_float4(__uint_as_float(f.x), __uint_as_float(f.y), __uint_as_float(f.z), __uint_as_float(f.w));
    }
}

// Int(round(v)) of quantize_rows without branches: round half away from
// zero, NaN -> 0, saturated at +-1e9 (the values here stay within +-32767).
__device__ __forceinline__ int round_to_int(float v) {
    float r = roundf(v);
    r = r != r ? 0.0f : r;
    r = fminf(fmaxf(r, -1.0e9f), 1.0e9f);
    return (int)r;
}

// Activation planes of four int16 codes X_e = xq_e + 32768 (e = 0..3),
// packed A = X0 | X1 << 16, B = X2 | X3 << 16.  int4: a 4 x 4 transpose of
// nibbles (two delta swaps, then a byte shuffle) leaves plane p's nibbles of
// X0..X3 in bits 16p..16p+15 of (A | B << 32).  int8: byte plane 0 (low
// bytes) and 1 (high bytes).
__device__ __forceinline__ void nibble_transpose(uint32_t &A, uint32_t &B) {
    uint32_t t = (A ^ (A >> 12)) & 0x0000F0F0u;
    A ^= t ^ (t << 12);
    t = (B ^ (B >> 12)) & 0x0000F0F0u;
    B ^= t ^ (t << 12);
    const uint32_t a2 = __builtin_amdgcn_perm(B, A, 0x06020400u);
    const uint32_t b2 = __builtin_amdgcn_perm(B, A, 0x07030501u);
    A = a2;
    B = b2;
}

template <int BITS, int NW, bool LN, int UPT, int STEPS, int WIN, bool DBG>
__global__ __launch_bounds__(NW * 64) void gemv1_kernel(Gemv1Args a) {
    constexpr int NT = NW * 64;
    constexpr int PD = BITS == 4 ? 16 : 8;  // plane dwords per chunk
    constexpr int SC_LD = (STEPS * 4 * 32 + 1023) / 1024;  // 16-byte scale loads per lane (groups of 16 rows x 2 B)
    constexpr int ZP_LD = (STEPS * 4 * 16 + 1023) / 1024;
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ __align__(16) uint16_t s_sc[NW][SC_LD * 512];
    __shared__ __align__(16) uint8_t s_zp[NW][ZP_LD * 1024];
    __shared__ float red[3][NW];
    __shared__ ArgmaxPart s_best[NW];

    const int CK = a.CK;
    uint32_t *xpl = smem;                                       // [CK][PD] activation planes
    int *xsum = reinterpret_cast<int *>(smem + CK * PD);        // [CK] sum of xq per chunk
    float *part = reinterpret_cast<float *>(smem + CK * (PD + 1));  // [tmax][NW][16 rows][4] partial sums
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: the index math below is scalar
    const int r = lane & 15, j = lane >> 4;
    const int S = (CK + 3) >> 2;
    // Tiles [t0, t0 + nt) of this workgroup; their nt * S steps split evenly
    // over the waves: wave wid takes steps [g0, g0 + ns), i.e. from step sA of
    // local tile tA on, crossing at most one tile boundary (ns <= S + 1).
    const int t0 = (int)((blockIdx.x * (uint32_t)a.ntiles) / gridDim.x);
    const int nt = (int)(((blockIdx.x + 1) * (uint32_t)a.ntiles) / gridDim.x) - t0;
    const int W = nt * S;
    const int g0 = (wid * W) / NW;
    const int ns = ((wid + 1) * W) / NW - g0;
    const int tA = ns > 0 ? (int)((uint32_t)g0 / (uint32_t)S) : 0;
    const int sA = ns > 0 ? g0 - tA * S : 0;
    const int nunits = a.K / 4;

    // 1. The activations first, then the weights, then the epilogue operands
    //    (wave t of the workgroup finishes local tile t).  Every load goes
    //    out before anything waits; code loads use 32-bit byte offsets from
    //    the matrix base.
    float4 xv[UPT], lw[UPT], lb[UPT];
    load_units<NT, UPT>(a.x, nunits, xv);
    if (LN) {
        load_units<NT, UPT>(a.ln_w, nunits, lw);
        load_units<NT, UPT>(a.ln_b, nunits, lb);
    }

    // Groups this wave touches: global group indices tile * NG + (chunk >>
    // cpg_shift), contiguous in the [tile][group][16] layout: [glo, glo + ng).
    const int gE = g0 + max(ns, 1) - 1;  // last step
    const int tE = (int)((uint32_t)gE / (uint32_t)S), sE = gE - tE * S;
    const int glo = (t0 + tA) * a.NG + ((4 * sA) >> a.cpg_shift);
    const int ghi = (t0 + tE) * a.NG + (min(4 * sE + 3, CK - 1) >> a.cpg_shift);
    const int ng = ns > 0 ? ghi - glo + 1 : 1;
    uint4 wsc[SC_LD], wzp[ZP_LD];
    uint4 wc[STEPS];
    // Step u < ns of the wave is step sA + u of local tile tA (or, past the
    // boundary, step sA + u - S of tile tA + 1).  Byte offset of lane (r, j)'s
    // 16 codes: ((tile * CK + 4 * step + j) * 16 + r) * 16.
    const int last = max(ns, 1) - 1;
    const uint32_t offA = ((uint32_t)(t0 + tA) * (uint32_t)CK + 4u * (uint32_t)sA) * 256u;
    const uint32_t wrap_adj = (uint32_t)(CK - 4 * S) * 256u;  // 0 when CK is a multiple of 4
    const uint32_t lane_off = (uint32_t)j * 256u + (uint32_t)r * 16u;
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rs = make_rsrc(a.scales, a.scales_bytes);
    const auto rz = make_rsrc(a.zps, a.zps_bytes);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < SC_LD; i++) {
        const uint32_t off = (uint32_t)(i * 1024 + lane * 16);  // bytes into the wave's scale block
        wsc[i] = bload16(rs, off < (uint32_t)ng * 32u ? (uint32_t)glo * 32u + off : kOOB);
    }
#pragma unroll
    for (int i = 0; i < ZP_LD; i++) {
        const uint32_t off = (uint32_t)(i * 1024 + lane * 16);
        wzp[i] = bload16(rz, off < (uint32_t)ng * 16u ? (uint32_t)glo * 16u + off : kOOB);
    }
    // The first WIN code steps go out now, step u + WIN once step u is
    // consumed (WIN < STEPS for matrices streamed from HBM: fewer bytes in
    // flight ahead of the activation row's own fetch, which gates the
    // prologue, and the sums then overlap the stream).
    auto code_off = [&](int u) -> uint32_t {
        const uint32_t off = offA + (uint32_t)u * 1024u + (sA + u >= S ? wrap_adj : 0u) + lane_off;
        return u < ns ? off : kOOB;
    };
#pragma unroll
    for (int u = 0; u < WIN; u++) wc[u] = bload16(rc, code_off(u));
    const int o = (t0 + wid) * 16 + r;  // the row this lane finishes (wave wid < nt)
    const bool row_ok = wid < nt && o < a.n;
    const auto rb = make_rsrc(a.bias, (uint32_t)a.n * 4u);  // a.bias is valid memory even without LLMQ_BIAS
    const auto ro = make_rsrc(a.out, (uint32_t)a.n * 4u);
    const float e_bias = bload4f(rb, row_ok ? (uint32_t)o * 4u : kOOB);
    const float e_res = bload4f(ro, row_ok ? (uint32_t)o * 4u : kOOB);
    __builtin_amdgcn_sched_barrier(0);

    // 2. Prologue: LayerNorm, quantize_rows, activation planes into LDS.
    //    LDS planes are [chunk][dword i of the chunk's codes][plane]: int4
    //    dword i pairs with the 8 activations of units 2i, 2i+1 (four planes
    //    of nibbles), int8 dword i with unit i (two planes of bytes).
    if (LN) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < UPT; i++) sum += (xv[i].x + xv[i].y) + (xv[i].z + xv[i].w);  // padding units hold zeros
        const float mean = block_sum<NW>(sum, red[0]) / (float)a.K;
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            if (tid + NT * i >= nunits) continue;
            const float d0 = xv[i].x - mean, d1 = xv[i].y - mean, d2 = xv[i].z - mean, d3 = xv[i].w - mean;
            sq += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
        const float var = block_sum<NW>(sq, red[1]) / (float)a.K;
        const float rstd = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            xv[i].x = ((xv[i].x - mean) * rstd) * lw[i].x + lb[i].x;
            xv[i].y = ((xv[i].y - mean) * rstd) * lw[i].y + lb[i].y;
            xv[i].z = ((xv[i].z - mean) * rstd) * lw[i].z + lb[i].z;
            xv[i].w = ((xv[i].w - mean) * rstd) * lw[i].w + lb[i].w;
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < UPT; i++)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[i].x), fabsf(xv[i].y)), fmaxf(fabsf(xv[i].z), fabsf(xv[i].w))));
    m = block_max<NW>(m, red[2]);
    float sx = m / 32767.0f;
    if (sx == 0.0f) sx = 1.0f;
    const float inv = 1.0f / sx;
    const bool xq_dbg = a.xq_out != nullptr && blockIdx.x == 0;
    if (xq_dbg && tid == 0 && a.sx_out) a.sx_out[0] = sx;
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + NT * i;
        const int q0 = round_to_int(xv[i].x * inv), q1 = round_to_int(xv[i].y * inv);
        const int q2 = round_to_int(xv[i].z * inv), q3 = round_to_int(xv[i].w * inv);
        if (xq_dbg && u < nunits) {
            const uint32_t lo = ((uint32_t)q0 & 0xFFFFu) | ((uint32_t)q1 << 16);
            const uint32_t hi = ((uint32_t)q2 & 0xFFFFu) | ((uint32_t)q3 << 16);
            reinterpret_cast<uint2 *>(a.xq_out)[u] = make_uint2(lo, hi);
        }
        int qs = (q0 + q1) + (q2 + q3);
        uint32_t A = (uint32_t)(q0 + 32768) | ((uint32_t)(q1 + 32768) << 16);
        uint32_t B = (uint32_t)(q2 + 32768) | ((uint32_t)(q3 + 32768) << 16);
        // Sum of xq over the chunk (8 units for int4, 4 for int8): the chunk's
        // units are consecutive lanes of one wave, aligned.
        qs += dppi<kQuadXor1>(qs);
        qs += dppi<kQuadXor2>(qs);
        if (BITS == 4) qs += dppi<kHalfMirror>(qs);
        if (BITS == 4) {
            nibble_transpose(A, B);
            // Unit pairs (2i, 2i+1) make the 8-activation plane dwords: the even
            // unit keeps planes 0, 1 and the odd one planes 2, 3.
            const bool odd = u & 1;
            const uint32_t other = (uint32_t)dppi<kQuadXor1>((int)(odd ? A : B));
            const uint32_t mine = odd ? B : A;
            const uint32_t lo_src = odd ? other : mine, hi_src = odd ? mine : other;
            const uint32_t pa = __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);
            const uint32_t pb = __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);
            if (u < nunits) {
                reinterpret_cast<uint2 *>(xpl)[u] = make_uint2(pa, pb);  // dword 4(u / 2) + 2(u & 1)
                if ((u & 7) == 0) xsum[u >> 3] = qs;
            }
        } else {
            const uint32_t p0 = __builtin_amdgcn_perm(B, A, 0x06040200u);
            const uint32_t p1 = __builtin_amdgcn_perm(B, A, 0x07050301u);
            if (u < nunits) {
                reinterpret_cast<uint2 *>(xpl)[u] = make_uint2(p0, p1);
                if ((u & 3) == 0) xsum[u >> 2] = qs;
            }
        }
    }
    // Scales and zero points of the wave into its LDS slot (wave-private; the
    // barrier below orders these writes before the reads).
#pragma unroll
    for (int i = 0; i < SC_LD; i++) reinterpret_cast<uint4 *>(s_sc[wid])[i * 64 + lane] = wsc[i];
#pragma unroll
    for (int i = 0; i < ZP_LD; i++) reinterpret_cast<uint4 *>(s_zp[wid])[i * 64 + lane] = wzp[i];
    lds_barrier();

    // 3. Integer sums per chunk, float accumulation per lane and tile (the
    //    wave's first tile tA, then tA + 1).  The wave's scales and zero
    //    points come out of LDS first, unconditionally (clamped index).
    float scl[STEPS];
    int zpl[STEPS], cl[STEPS];
#pragma unroll
    for (int u = 0; u < STEPS; u++) {
        const int uc = min(u, last);
        const bool second = sA + uc >= S;
        const int ss = sA + uc - (second ? S : 0);
        const int c_raw = 4 * ss + j;
        const bool ok = u < ns && c_raw < CK;
        const int c = ok ? c_raw : 0;
        const int gl = ok ? (t0 + tA + (second ? 1 : 0)) * a.NG + (c >> a.cpg_shift) - glo : 0;
        const float sc = __half2float(__ushort_as_half(s_sc[wid][gl * 16 + r]));
        scl[u] = ok ? sc : 0.0f;
        zpl[u] = (int)s_zp[wid][gl * 16 + r];
        cl[u] = c;
    }
    float accA = 0.0f, accB = 0.0f;
#pragma unroll
    for (int u = 0; u < STEPS; u++) {
        if (u >= ns) break;  // wave-uniform: steps past the wave's range carry no codes
        const bool second = sA + u >= S;
        const int tl = tA + (second ? 1 : 0);
        const int c = cl[u];
        const float scale = scl[u];
        const int zp = zpl[u];
        const uint4 d = wc[u];
        if (u + WIN < STEPS) {
            __builtin_amdgcn_sched_barrier(0);
            wc[u + WIN] = bload16(rc, code_off(u + WIN));
            __builtin_amdgcn_sched_barrier(0);
        }
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
        const uint4 *P = reinterpret_cast<const uint4 *>(xpl + c * PD);
        uint32_t xu;
        if (BITS == 4) {
            // P[i] = planes 0..3 of the activations paired with code dword i.
            const uint4 q0 = P[0], q1 = P[1], q2 = P[2], q3 = P[3];
            uint32_t S0 = __builtin_amdgcn_udot8(q0.x, d.x, 0u, false);
            S0 = __builtin_amdgcn_udot8(q1.x, d.y, S0, false);
            S0 = __builtin_amdgcn_udot8(q2.x, d.z, S0, false);
            S0 = __builtin_amdgcn_udot8(q3.x, d.w, S0, false);
            uint32_t S1 = __builtin_amdgcn_udot8(q0.y, d.x, 0u, false);
            S1 = __builtin_amdgcn_udot8(q1.y, d.y, S1, false);
            S1 = __builtin_amdgcn_udot8(q2.y, d.z, S1, false);
            S1 = __builtin_amdgcn_udot8(q3.y, d.w, S1, false);
            uint32_t S2 = __builtin_amdgcn_udot8(q0.z, d.x, 0u, false);
            S2 = __builtin_amdgcn_udot8(q1.z, d.y, S2, false);
            S2 = __builtin_amdgcn_udot8(q2.z, d.z, S2, false);
            S2 = __builtin_amdgcn_udot8(q3.z, d.w, S2, false);
            uint32_t S3 = __builtin_amdgcn_udot8(q0.w, d.x, 0u, false);
            S3 = __builtin_amdgcn_udot8(q1.w, d.y, S3, false);
            S3 = __builtin_amdgcn_udot8(q2.w, d.z, S3, false);
            S3 = __builtin_amdgcn_udot8(q3.w, d.w, S3, false);
            xu = S0 + (S1 << 4) + (S2 << 8) + (S3 << 12);
        } else {
            // P[0] = (plane 0, 1) of dwords 0, 1; P[1] the same of dwords 2, 3.
            const uint4 q01 = P[0], q23 = P[1];
            uint32_t S0 = __builtin_amdgcn_udot4(q01.x, d.x, 0u, false);
            S0 = __builtin_amdgcn_udot4(q01.z, d.y, S0, false);
            S0 = __builtin_amdgcn_udot4(q23.x, d.z, S0, false);
            S0 = __builtin_amdgcn_udot4(q23.z, d.w, S0, false);
            uint32_t S1 = __builtin_amdgcn_udot4(q01.y, d.x, 0u, false);
            S1 = __builtin_amdgcn_udot4(q01.w, d.y, S1, false);
            S1 = __builtin_amdgcn_udot4(q23.y, d.z, S1, false);
            S1 = __builtin_amdgcn_udot4(q23.w, d.w, S1, false);
            xu = S0 + (S1 << 8);
        }
        const int G = (int)(xu - 32768u * su) - zp * xsum[c];
        if (DBG) {
            const int row = (t0 + tl) * 16 + r;
            if (row < a.n && 4 * (sA + u - (second ? S : 0)) + j < CK) a.dbg[(size_t)row * CK + c] = G;
        }
        accA = fmaf((float)G, second ? 0.0f : scale, accA);
        accB = fmaf((float)G, second ? scale : 0.0f, accB);
    }

    // 4. Per row: the 4 lanes of each wave and the waves that touched the
    //    tile, in a fixed order, by wave t for local tile t.
    for (int t = 0; t < a.tmax; t++) {
        const float v = t == tA ? accA : (t == tA + 1 ? accB : 0.0f);
        part[((t * NW + wid) * 16 + r) * 4 + j] = v;
    }
    lds_barrier();
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    if (wid < nt && j == 0) {
        const float4 *p4 = reinterpret_cast<const float4 *>(part) + wid * NW * 16 + r;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < NW; q++) {
            const float4 t = p4[q * 16];
            v += (t.x + t.y) + (t.z + t.w);
        }
        if (row_ok) {
            v = v * sx;
            if (a.flags & LLMQ_BIAS) v += e_bias;
            if (a.flags & LLMQ_GELU) v = gelu_ref(v);
            if (a.flags & LLMQ_RESID) v += e_res;
            a.out[o] = v;
            best_v = v;
            best_i = o;
        }
    }
    if (a.amax) {
        // Largest logit of the workgroup; equal values keep the smaller index
        // (argmax's first maximum, gpt2t.mojo:792-797).
        if (wid < nt) {
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) {
                const float ov = __shfl_xor(best_v, off);
                const int oi = __shfl_xor(best_i, off);
                if (ov > best_v || (ov == best_v && oi < best_i)) {
                    best_v = ov;
                    best_i = oi;
                }
            }
            if (lane == 0) s_best[wid] = ArgmaxPart{best_v, best_i};
        }
        lds_barrier();
        if (tid == 0) {
            ArgmaxPart b = s_best[0];
            for (int q = 1; q < nt; q++) {
                const ArgmaxPart c = s_best[q];
                if (c.v > b.v || (c.v == b.v && c.idx < b.idx)) b = c;
            }
            a.amax[blockIdx.x] = b;
        }
    }
}

struct Plan {
    int nw, tmax, spw, steps, upt, grid, win;
};

// Matrices at least this large are taken as streamed from HBM (the
// last-level cache is 256 MB, but a decode step over a large model streams
// every matrix once): they keep kStreamWin code steps in flight per wave.
constexpr int64_t kStreamBytes = 20ll << 20;
constexpr int kStreamWin = 2;

int steps_for(int spw) { return spw <= 2 ? 2 : spw <= 4 ? 4 : 8; }

// Workgroup shape for a matrix.  Matrices below kStreamBytes of codes, or
// with short rows (at most 4 steps a wave in one tile): 4-wave workgroups,
// one row tile each (up to 8 steps a wave and 4 activation units a thread;
// longer rows fall back to 16 waves).  Large long-row (HBM-streamed)
// matrices: 16-wave workgroups, one per CU, each with a
// contiguous run of whole tiles (so CUs differ by at most one tile of work)
// and the per-workgroup prologue spread over 1024 threads.  Each wave holds
// at most kMaxSteps steps and crosses at most one tile boundary; past that,
// more workgroups.
Plan make_plan(const llmq_mat *w) {
    Plan p{};
    const int S = (int)((w->CK + 3) / 4);
    const int units = (int)(w->k / 4);           // four activations per thread
    // 16-wave workgroups for long-row matrices streamed from HBM (with the
    // code-step window below); 4-wave workgroups of one row tile otherwise,
    // which launch faster (measured against 16 waves: 3072x768 5.08 ->
    // 4.84 us, 4096x4096 5.70 -> 5.33 us, the 50257x768 int8 head 14.1 ->
    // 10.8 us from HBM).
    int nw = (w->ntiles * w->CK * 256 >= kStreamBytes && (S + 3) / 4 > 4) ? 16 : 4;
    if (const char *e = getenv("LLMQ_GEMV1_NW")) {
        const int v = atoi(e);
        if (v == 4 || v == 16) nw = v;
    }
    if (nw == 4 && (units > 1024 || (S + 3) / 4 > kMaxSteps)) nw = 16;  // 4-wave kernels: <= 8 steps, <= 4 units
    int64_t grid = w->ntiles;
    if (nw == 16) {
        int cus = 256;
        if (const char *e = getenv("LLMQ_GEMV1_GRID")) cus = std::max(1, atoi(e));
        grid = std::min<int64_t>(w->ntiles, cus);
        const int cap = std::min(kMaxSteps, S + 1);
        int tmax = (int)((w->ntiles + grid - 1) / grid);
        if (tmax > kMaxTiles || (tmax * S + 15) / 16 > cap) {
            tmax = std::max(1, std::min(kMaxTiles, cap * 16 / S));
            grid = (w->ntiles + tmax - 1) / tmax;
        }
    }
    p.nw = nw;
    p.grid = (int)grid;
    p.tmax = (int)((w->ntiles + grid - 1) / grid);
    p.spw = (p.tmax * S + nw - 1) / nw;
    p.steps = steps_for(p.spw);
    p.upt = (units + nw * 64 - 1) / (nw * 64);
    const int64_t code_bytes = w->ntiles * w->CK * 256;
    p.win = (nw == 16 && code_bytes >= kStreamBytes) ? kStreamWin : p.steps;
    if (const char *e = getenv("LLMQ_GEMV1_WIN")) p.win = atoi(e) == kStreamWin ? kStreamWin : p.steps;
    return p;
}

// Dynamic LDS: activation planes, chunk sums, per-tile partial sums.
size_t lds_bytes(const llmq_mat *w, const Plan &p) {
    const int PD = w->bits == 4 ? 16 : 8;
    return (size_t)w->CK * (PD + 1) * 4 + (size_t)p.tmax * p.nw * 64 * 4;
}


template <int BITS, int NW, bool LN, int UPT, int STEPS>
void launch_t(llmq_ctx *ctx, const Gemv1Args &a, int grid, size_t lds, int win) {
    if constexpr (!LN) {
        if (a.dbg) {
            hipLaunchKernelGGL((gemv1_kernel<BITS, NW, LN, UPT, STEPS, STEPS, true>), dim3((unsigned)grid),
                               dim3(NW * 64), lds, ctx->stream, a);
            return;
        }
    }
    if constexpr (NW == 16 && STEPS > kStreamWin) {
        if (win == kStreamWin) {
            hipLaunchKernelGGL((gemv1_kernel<BITS, NW, LN, UPT, STEPS, kStreamWin, false>), dim3((unsigned)grid),
                               dim3(NW * 64), lds, ctx->stream, a);
            return;
        }
    }
    hipLaunchKernelGGL((gemv1_kernel<BITS, NW, LN, UPT, STEPS, STEPS, false>), dim3((unsigned)grid), dim3(NW * 64),
                       lds, ctx->stream, a);
}

template <int BITS, int NW, bool LN, int UPT>
int launch_steps(llmq_ctx *ctx, const Gemv1Args &a, const Plan &p, size_t lds) {
    switch (p.steps) {
        case 2: launch_t<BITS, NW, LN, UPT, 2>(ctx, a, p.grid, lds, p.win); return LLMQ_OK;
        case 4: launch_t<BITS, NW, LN, UPT, 4>(ctx, a, p.grid, lds, p.win); return LLMQ_OK;
        case 8: launch_t<BITS, NW, LN, UPT, 8>(ctx, a, p.grid, lds, p.win); return LLMQ_OK;
    }
    return llmq_set_error(LLMQ_EUNSUPPORTED, "linear: no kernel for %d waves x %d steps", NW, p.steps);
}

template <int BITS>
int launch_bits(llmq_ctx *ctx, const Gemv1Args &a, const Plan &p, size_t lds, bool ln) {
    if (p.nw == 4) {
        if (p.upt == 1) return ln ? launch_steps<BITS, 4, true, 1>(ctx, a, p, lds) : launch_steps<BITS, 4, false, 1>(ctx, a, p, lds);
        if (!ln && p.upt == 2) return launch_steps<BITS, 4, false, 2>(ctx, a, p, lds);
        if (!ln && p.upt <= 4) return launch_steps<BITS, 4, false, 4>(ctx, a, p, lds);
    } else if (ln) {
        if (p.upt == 1) return launch_steps<BITS, 16, true, 1>(ctx, a, p, lds);
    } else {
        if (p.upt == 1) return launch_steps<BITS, 16, false, 1>(ctx, a, p, lds);
        if (p.upt == 2) return launch_steps<BITS, 16, false, 2>(ctx, a, p, lds);
        if (p.upt <= 4) return launch_steps<BITS, 16, false, 4>(ctx, a, p, lds);
    }
    return llmq_set_error(LLMQ_EUNSUPPORTED, "linear: reduction axis %d too long%s", a.K,
                          ln ? " for the LayerNorm prologue" : "");
}

}  // namespace

// Whether the one-token kernel takes w (else the multi-token kernel loops
// over the reduction axis).
bool gemv1_supports(const llmq_mat *w, bool ln) {
    const Plan p = make_plan(w);
    (void)ln;
    const int64_t code_bytes = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256;
    return p.spw <= kMaxSteps && p.spw <= (w->CK + 3) / 4 + 1 && p.upt <= 4 && lds_bytes(w, p) <= 64 * 1024 &&
           code_bytes < (int64_t)kOOB;
}

int gemv1_num_parts(const llmq_mat *w, bool ln) { return (void)ln, make_plan(w).grid; }

int launch_gemv1(llmq_ctx *ctx, const GemvRequest &rq) {
    const llmq_mat *w = rq.w;
    const bool ln = rq.ln_w != nullptr;
    const Plan p = make_plan(w);
    LLMQ_REQUIRE(gemv1_supports(w, ln), "linear: no one-token kernel for reduction axis %lld", (long long)w->k);
    LLMQ_REQUIRE(!rq.amax || p.grid <= rq.amax_cap, "linear: %d argmax partials exceed capacity %d", p.grid,
                 rq.amax_cap);
    const size_t lds = lds_bytes(w, p);
    Gemv1Args a;
    a.codes = reinterpret_cast<const uint4 *>(w->codes);
    a.scales = w->scales;
    a.zps = w->zps;
    a.codes_bytes = (uint32_t)((w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256);
    a.scales_bytes = (uint32_t)((w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS * 2);
    a.zps_bytes = (uint32_t)((w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS);
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
    a.tmax = p.tmax;
    a.flags = rq.flags;
    a.x = rq.x;
    a.ln_w = rq.ln_w;
    a.ln_b = rq.ln_b;
    a.bias = rq.bias ? rq.bias : rq.out;  // read (and ignored) without LLMQ_BIAS
    a.out = rq.out;
    a.amax = rq.amax;
    a.dbg = rq.dbg;
    a.xq_out = rq.xq_out;
    a.sx_out = rq.sx_out;
    int rc = w->bits == 4 ? launch_bits<4>(ctx, a, p, lds, ln) : launch_bits<8>(ctx, a, p, lds, ln);
    if (rc != LLMQ_OK) return rc;
    LLMQ_HIP(hipGetLastError());
    if (rq.amax_count) *rq.amax_count = p.grid;
    return LLMQ_OK;
}
