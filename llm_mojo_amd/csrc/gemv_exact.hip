// One-token GEMVs in the reference's own float order, for the two formats
// of config 0's decode: BLOCKED int4-g32-a16 layers and the int8
// per-channel A16 head (QuantMatrix.dot_row_i16, tensor.mojo:518-566, as
// driven by matmul_rows_a16 / linear_team with T == 1, kernels.mojo:419-470,
// 774-866), with quantize_rows (kernels.mojo:400-416) and optionally
// layernorm (kernels.mojo:179-197) in front and store_out / finish
// (kernels.mojo:38-48, 274-282) behind.  Outputs are bit-identical to the
// reference's arithmetic: every integer sum is exact, and every float
// operation is the reference's, in its order.
//
// BLOCKED (tensor.mojo:522-540).  The reference keeps 16 float lanes per
// row; lane L (L = g + 8h) owns half h (weights 16h .. 16h + 15) of group g
// of every 256-weight block, and per block does
//     accf[L] = fma(f32(sum x u) - zp * sum x, scale, accf[L])
// then reduce_add over the 16 lanes (a halving tree) and * sx.  Here one GPU
// lane owns group g of 8 rows' chunks: lane = 8 g + r (r = row within the
// wave's 8), so per block a wave reads, for each of the 8 groups, 8 rows x
// 16 B = one contiguous 128-byte line of the row-tile layout.  The lane
// keeps the two chains (h = 0, 1) of its group in block order; the tree's
// first level (L, L + 8) is in-lane and the others pair lanes 32, 16 and 8
// apart.  The integer half sums come from unsigned nibble dot products
// against planes of X = xq + 32768: sum x u = sum_p 16^p dot8(plane_p, u) -
// 32768 sum u, exact in int32, and f32(that) - zp * sum x is the exact
// half-group sum G, below 2^24, so f32(G) is the reference's operand.
//
// int8 per channel (tensor.mojo:541-566).  Reference lane L accumulates, in
// int32, the pairs (2L, 2L + 1) of every 32-weight piece of the row, then
// f32(acc).fma(s, 0) and reduce_add.  Integer sums do not depend on order,
// so any GPU lane may add any of a row's pairs: lane (r, j) of a wave reads
// chunk 4s + j (16 codes) of row r per step, i.e. the 8 pairs of reference
// lanes 8 (j & 1) .. + 7, and keeps 8 int32 accumulators (v_dot2 of the
// int16 activation pair with the zero-extended code pair); lanes j, j + 2
// and the waves of the tile are then added, the zero point applied as
// acc - zp * sum x (exact), and the float steps run in the reference's order.
#include "common.h"

namespace {

constexpr int kPlaneStride = 20;  // dwords per 32-activation chunk in LDS (16 used; no bank conflicts)

// ------------------------------------------------------------- activations

// Int(round(v)) of quantize_rows: half away from zero; the values stay
// within +-32767.
__device__ __forceinline__ int q_round(float v) { return (int)roundf(v); }

// Loads the token row as units of four floats: unit u = threadIdx.x + NT i.
template <int NT, int UPT>
__device__ __forceinline__ void load_row(const float *p, int nunits, float4 (&v)[UPT]) {
    const auto r = llmq_rsrc(p, (uint32_t)nunits * 16u);
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const uint32_t u = threadIdx.x + NT * i;
        const uint4 f = llmq_bload16(r, u < (uint32_t)nunits ? u * 16u : kLlmqOOB);
        v[i] = make_float4(__uint_as_float(f.x), __uint_as_float(f.y), __uint_as_float(f.z), __uint_as_float(f.w));
    }
}

// LayerNorm (optional), then quantize_rows' scale: the row in xv is
// replaced by the normalized one; returns sx.  xs: K floats of LDS, bc: 2,
// red: NT / 64.  Ends with a barrier.
template <int NT, int UPT, bool LN>
__device__ __forceinline__ float act_prologue(float4 (&xv)[UPT], const float4 (&lw)[UPT], const float4 (&lb)[UPT],
                                              int K, float *xs, float *bc, float *red) {
    const int nunits = K / 4;
    if (LN) {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = threadIdx.x + NT * i;
            if (u < nunits) reinterpret_cast<float4 *>(xs)[u] = xv[i];
        }
        llmq_lds_barrier();
        float mean, rstd;
        llmq_ln_stats(xs, K, bc, mean, rstd);
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            xv[i].x = ((xv[i].x - mean) * rstd) * lw[i].x + lb[i].x;
            xv[i].y = ((xv[i].y - mean) * rstd) * lw[i].y + lb[i].y;
            xv[i].z = ((xv[i].z - mean) * rstd) * lw[i].z + lb[i].z;
            xv[i].w = ((xv[i].w - mean) * rstd) * lw[i].w + lb[i].w;
        }
    }
    // max |x| (exact in any order), over the workgroup
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < UPT; i++)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[i].x), fabsf(xv[i].y)), fmaxf(fabsf(xv[i].z), fabsf(xv[i].w))));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    llmq_lds_barrier();
    m = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) m = fmaxf(m, red[w]);
    float s = m / 32767.0f;
    if (s == 0.0f) s = 1.0f;
    return s;
}

// Nibble planes of four int16 codes X_e = xq_e + 32768 packed as A = X0 |
// X1 << 16, B = X2 | X3 << 16: a 4 x 4 nibble transpose leaves plane p's
// nibbles of X0..X3 in bits 16p .. 16p + 15 of (A | B << 32).
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
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E;

// ---------------------------------------------------------------- BLOCKED

struct BlkArgs {
    const uint4 *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    uint32_t codes_bytes, scales_bytes, zps_bytes;
    int n, K, CK, nwaves, flags;
    const float *x, *ln_w, *ln_b, *bias;
    float *out;
    int32_t *dbg;
    int16_t *xq_out;
    float *sx_out;
};

template <int NW, bool LN, int UPT, int WIN, bool DBG>
__global__ __launch_bounds__(NW * 64) void gemv_blk_kernel(BlkArgs a) {
    constexpr int NT = NW * 64;
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t *planes = smem;                                             // [CK][kPlaneStride]
    int *hsum = reinterpret_cast<int *>(smem + a.CK * kPlaneStride);     // [CK][2] sum of xq per half
    float *xs = reinterpret_cast<float *>(hsum + 2 * a.CK);              // [K] (LayerNorm)
    __shared__ float bc[2], red[NW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gw = blockIdx.x * NW + wid;  // global wave: rows 8 gw .. 8 gw + 7
    const bool live = gw < a.nwaves;
    const int tile = gw >> 1, rr = 8 * (gw & 1) + (lane & 7), g = lane >> 3;
    const int o = tile * 16 + rr;
    const int nb = a.K >> 8;
    const int nunits = a.K >> 2;

    // Activations first, then the first WIN blocks of codes, scales and zero
    // points, then the epilogue operands: all in flight before any wait.
    float4 xv[UPT], lw[UPT], lb[UPT];
    load_row<NT, UPT>(a.x, nunits, xv);
    if (LN) {
        load_row<NT, UPT>(a.ln_w, nunits, lw);
        load_row<NT, UPT>(a.ln_b, nunits, lb);
    }
    const auto rc = llmq_rsrc(a.codes, a.codes_bytes);
    const auto rs = llmq_rsrc(a.scales, a.scales_bytes);
    const auto rz = llmq_rsrc(a.zps, a.zps_bytes);
    // block b of this lane: chunk c = 8 b + g of row o
    auto code_off = [&](int b) -> uint32_t {
        const uint32_t c = (uint32_t)(8 * b + g);
        return live && b < nb ? (((uint32_t)tile * (uint32_t)a.CK + c) * 16u + (uint32_t)rr) * 16u : kLlmqOOB;
    };
    auto meta_off = [&](int b) -> uint32_t {  // [tile][group][16 rows]
        const uint32_t c = (uint32_t)(8 * b + g);
        return live && b < nb ? ((uint32_t)tile * (uint32_t)a.CK + c) * 16u + (uint32_t)rr : kLlmqOOB;
    };
    uint4 wc[WIN];
    uint32_t wsc[WIN], wzp[WIN];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < WIN; u++) {
        wc[u] = llmq_bload16(rc, code_off(u));
        const uint32_t mo = meta_off(u);
        wsc[u] = llmq_bload2(rs, mo == kLlmqOOB ? kLlmqOOB : mo * 2u);
        wzp[u] = llmq_bload1(rz, mo);
    }
    const bool row_ok = live && g == 0 && o < a.n;
    const auto rb = llmq_rsrc(a.bias, (uint32_t)a.n * 4u);
    const auto ro = llmq_rsrc(a.out, (uint32_t)a.n * 4u);
    const float e_bias = __uint_as_float(llmq_bload4(rb, row_ok ? (uint32_t)o * 4u : kLlmqOOB));
    const float e_res = __uint_as_float(llmq_bload4(ro, row_ok ? (uint32_t)o * 4u : kLlmqOOB));
    __builtin_amdgcn_sched_barrier(0);

    // Prologue: LayerNorm, quantize_rows, nibble planes and half sums.
    const float sx = act_prologue<NT, UPT, LN>(xv, lw, lb, a.K, xs, bc, red);
    const float inv = 1.0f / sx;
    const bool xq_dbg = a.xq_out != nullptr && blockIdx.x == 0;
    if (xq_dbg && tid == 0 && a.sx_out) a.sx_out[0] = sx;
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + NT * i;
        const int q0 = q_round(xv[i].x * inv), q1 = q_round(xv[i].y * inv);
        const int q2 = q_round(xv[i].z * inv), q3 = q_round(xv[i].w * inv);
        if (xq_dbg && u < nunits) {
            const uint32_t lo = ((uint32_t)q0 & 0xFFFFu) | ((uint32_t)q1 << 16);
            const uint32_t hi = ((uint32_t)q2 & 0xFFFFu) | ((uint32_t)q3 << 16);
            reinterpret_cast<uint2 *>(a.xq_out)[u] = make_uint2(lo, hi);
        }
        // sum over the half (4 consecutive units = 4 consecutive lanes)
        int qs = (q0 + q1) + (q2 + q3);
        qs += dppi<kQuadXor1>(qs);
        qs += dppi<kQuadXor2>(qs);
        uint32_t A = (uint32_t)(q0 + 32768) | ((uint32_t)(q1 + 32768) << 16);
        uint32_t B = (uint32_t)(q2 + 32768) | ((uint32_t)(q3 + 32768) << 16);
        nibble_transpose(A, B);
        // units 2i, 2i + 1 of a chunk make the plane dwords of code dword i:
        // the even unit stores planes 0, 1 and the odd one planes 2, 3
        const bool odd = u & 1;
        const uint32_t other = (uint32_t)dppi<kQuadXor1>((int)(odd ? A : B));
        const uint32_t mine = odd ? B : A;
        const uint32_t lo_src = odd ? other : mine, hi_src = odd ? mine : other;
        const uint32_t pa = __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);
        const uint32_t pb = __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);
        if (u < nunits) {
            const int c = u >> 3, e = u & 7;
            reinterpret_cast<uint2 *>(planes + c * kPlaneStride + 4 * (e >> 1) + 2 * (e & 1))[0] = make_uint2(pa, pb);
            if ((u & 3) == 0) hsum[2 * c + (e >> 2)] = qs;
        }
    }
    llmq_lds_barrier();

    // Blocks in order: the integer half sums, then the two fma chains.
    float acc0 = 0.0f, acc1 = 0.0f;
    const uint32_t K1 = 0x11111111u;
    for (int b0 = 0; b0 < nb; b0 += WIN) {
#pragma unroll
        for (int u = 0; u < WIN; u++) {
            const int b = b0 + u;
            if (b < nb) {  // wave-uniform
            const uint4 d = wc[u];
            const float sc = __half2float(__ushort_as_half((unsigned short)wsc[u]));
            const int zp = (int)wzp[u];
            __builtin_amdgcn_sched_barrier(0);
            wc[u] = llmq_bload16(rc, code_off(b + WIN));
            const uint32_t mo = meta_off(b + WIN);
            wsc[u] = llmq_bload2(rs, mo == kLlmqOOB ? kLlmqOOB : mo * 2u);
            wzp[u] = llmq_bload1(rz, mo);
            __builtin_amdgcn_sched_barrier(0);
            const int c = 8 * b + g;
            const uint4 *P = reinterpret_cast<const uint4 *>(planes + c * kPlaneStride);
            const uint4 p0 = P[0], p1 = P[1], p2 = P[2], p3 = P[3];
            const int2 hs = reinterpret_cast<const int2 *>(hsum)[c];
            // half 0: code dwords 0, 1; half 1: dwords 2, 3
            uint32_t a0 = __builtin_amdgcn_udot8(p0.x, d.x, 0u, false);
            a0 = __builtin_amdgcn_udot8(p1.x, d.y, a0, false);
            uint32_t a1 = __builtin_amdgcn_udot8(p0.y, d.x, 0u, false);
            a1 = __builtin_amdgcn_udot8(p1.y, d.y, a1, false);
            uint32_t a2 = __builtin_amdgcn_udot8(p0.z, d.x, 0u, false);
            a2 = __builtin_amdgcn_udot8(p1.z, d.y, a2, false);
            uint32_t a3 = __builtin_amdgcn_udot8(p0.w, d.x, 0u, false);
            a3 = __builtin_amdgcn_udot8(p1.w, d.y, a3, false);
            uint32_t b0s = __builtin_amdgcn_udot8(p2.x, d.z, 0u, false);
            b0s = __builtin_amdgcn_udot8(p3.x, d.w, b0s, false);
            uint32_t b1s = __builtin_amdgcn_udot8(p2.y, d.z, 0u, false);
            b1s = __builtin_amdgcn_udot8(p3.y, d.w, b1s, false);
            uint32_t b2s = __builtin_amdgcn_udot8(p2.z, d.z, 0u, false);
            b2s = __builtin_amdgcn_udot8(p3.z, d.w, b2s, false);
            uint32_t b3s = __builtin_amdgcn_udot8(p2.w, d.z, 0u, false);
            b3s = __builtin_amdgcn_udot8(p3.w, d.w, b3s, false);
            uint32_t su0 = __builtin_amdgcn_udot8(d.x, K1, 0u, false);
            su0 = __builtin_amdgcn_udot8(d.y, K1, su0, false);
            uint32_t su1 = __builtin_amdgcn_udot8(d.z, K1, 0u, false);
            su1 = __builtin_amdgcn_udot8(d.w, K1, su1, false);
            const uint32_t xu0 = a0 + (a1 << 4) + (a2 << 8) + (a3 << 12);
            const uint32_t xu1 = b0s + (b1s << 4) + (b2s << 8) + (b3s << 12);
            const int G0 = (int)(xu0 - 32768u * su0) - zp * hs.x;
            const int G1 = (int)(xu1 - 32768u * su1) - zp * hs.y;
            if (DBG && live && o < a.n) a.dbg[(size_t)o * a.CK + c] = G0 + G1;
            acc0 = fmaf((float)G0, sc, acc0);
            acc1 = fmaf((float)G1, sc, acc1);
            }
        }
    }
    // reduce_add: (L, L + 8) in-lane, then groups g, g + 4 / + 2 / + 1.
    float v = acc0 + acc1;
    v = v + __shfl_down(v, 32);
    v = v + __shfl_down(v, 16);
    v = v + __shfl_down(v, 8);
    if (row_ok) {
        float r = v * sx;
        if (a.flags & LLMQ_BIAS) r += e_bias;
        if (a.flags & LLMQ_GELU) r = gelu_ref(r);
        if (a.flags & LLMQ_RESID) r += e_res;
        a.out[o] = r;
    }
}

// ------------------------------------------------------ int8 per channel

struct Ch8Args {
    const uint4 *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    uint32_t codes_bytes;
    int n, K, CK, ntiles, flags;
    const float *x, *ln_w, *ln_b, *bias;
    float *out;
    ArgmaxPart *amax;
    int16_t *xq_out;
    float *sx_out;
};

// Workgroup: NW waves over TPW row tiles (NW / TPW waves share a tile's
// steps, contiguously).  Step s of a tile is chunks 4s .. 4s + 3 of its 16
// rows; lane (r, j) = (lane & 15, lane >> 4) reads chunk 4s + j.
template <int NW, int TPW, bool LN, int UPT, int SPW>
__global__ __launch_bounds__(NW * 64) void head8_kernel(Ch8Args a) {
    constexpr int NT = NW * 64, WPT = NW / TPW;  // waves per tile
    extern __shared__ __align__(16) uint32_t smem[];
    int16_t *xq = reinterpret_cast<int16_t *>(smem);                        // [K] natural order
    int *part = reinterpret_cast<int *>(smem + a.K / 2);                     // [TPW][WPT][2][16 rows][8]
    float *xs = reinterpret_cast<float *>(part + TPW * WPT * 2 * 16 * 8);    // [K] (LayerNorm)
    __shared__ int xsl[16];        // sum of xq over reference lane L's pairs
    __shared__ float bc[2], red[NW];
    __shared__ ArgmaxPart s_best[NW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, j = lane >> 4;
    const int tl = wid / WPT, wt = wid % WPT;  // tile of the workgroup, wave within the tile
    const int tile = blockIdx.x * TPW + tl;
    const bool live = tile < a.ntiles;
    const int S = a.CK >> 2;  // steps per tile (CK a multiple of 4)
    const int s0 = (wt * S) / WPT, ns = ((wt + 1) * S) / WPT - s0;
    const int nunits = a.K >> 2;

    float4 xv[UPT], lw[UPT], lb[UPT];
    load_row<NT, UPT>(a.x, nunits, xv);
    if (LN) {
        load_row<NT, UPT>(a.ln_w, nunits, lw);
        load_row<NT, UPT>(a.ln_b, nunits, lb);
    }
    const auto rc = llmq_rsrc(a.codes, a.codes_bytes);
    uint4 wc[SPW];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        const uint32_t c = (uint32_t)(4 * (s0 + u) + j);
        wc[u] = llmq_bload16(rc, live && u < ns ? (((uint32_t)tile * (uint32_t)a.CK + c) * 16u + (uint32_t)r) * 16u
                                                : kLlmqOOB);
    }
    const int o = tile * 16 + r;
    const bool row_ok = live && o < a.n;
    const float scale = row_ok ? __half2float(__ushort_as_half(a.scales[tile * 16 + r])) : 0.0f;
    const int zp = row_ok ? (int)a.zps[tile * 16 + r] : 0;
    __builtin_amdgcn_sched_barrier(0);

    const float sx = act_prologue<NT, UPT, LN>(xv, lw, lb, a.K, xs, bc, red);
    const float inv = 1.0f / sx;
    const bool xq_dbg = a.xq_out != nullptr && blockIdx.x == 0;
    if (xq_dbg && tid == 0 && a.sx_out) a.sx_out[0] = sx;
    if (tid < 16) xsl[tid] = 0;
    llmq_lds_barrier();
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + NT * i;
        const int q0 = q_round(xv[i].x * inv), q1 = q_round(xv[i].y * inv);
        const int q2 = q_round(xv[i].z * inv), q3 = q_round(xv[i].w * inv);
        if (u < nunits) {
            const uint32_t lo = ((uint32_t)q0 & 0xFFFFu) | ((uint32_t)q1 << 16);
            const uint32_t hi = ((uint32_t)q2 & 0xFFFFu) | ((uint32_t)q3 << 16);
            reinterpret_cast<uint2 *>(xq)[u] = make_uint2(lo, hi);
            if (xq_dbg) reinterpret_cast<uint2 *>(a.xq_out)[u] = make_uint2(lo, hi);
            // unit u holds pairs 2 (u & 7) and 2 (u & 7) + 1 of its 32-piece
            atomicAdd(&xsl[2 * (u & 7)], q0 + q1);
            atomicAdd(&xsl[2 * (u & 7) + 1], q2 + q3);
        }
    }
    llmq_lds_barrier();

    // 8 int32 lanes of sum x u: lane (r, j) holds reference lanes
    // 8 (j & 1) + i, i = 0..7 (chunk 4s + j has parity j & 1).
    int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    typedef short s2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int u = 0; u < SPW; u++) {
        if (u < ns) {  // wave-uniform
        const int c = 4 * (s0 + u) + j;
        const uint4 d = wc[u];
        const uint4 x0 = reinterpret_cast<const uint4 *>(xq)[2 * c];      // pairs 0..3 of the chunk
        const uint4 x1 = reinterpret_cast<const uint4 *>(xq)[2 * c + 1];  // pairs 4..7
        const uint32_t xp[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t up = __builtin_amdgcn_perm(0u, dw[i >> 1], (i & 1) ? 0x0c030c02u : 0x0c010c00u);
            acc[i] = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, xp[i]), __builtin_bit_cast(s2, up), acc[i], false);
        }
        }
    }
    // lanes j and j + 2 hold the same reference lanes
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] += __shfl_down(acc[i], 32);
    // waves of the tile, through LDS (lanes j = 0, 1)
    if (j < 2) {
#pragma unroll
        for (int i = 0; i < 8; i++) part[(((tl * WPT + wt) * 2 + j) * 16 + r) * 8 + i] = acc[i];
    }
    llmq_lds_barrier();
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    if (wt == 0) {
        // lane (r, j < 2): reference lanes 8 j + i of row r, as floats
        float vl[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (j < 2) {
#pragma unroll
            for (int i = 0; i < 8; i++) {
                int t = 0;
#pragma unroll
                for (int w = 0; w < WPT; w++) t += part[(((tl * WPT + w) * 2 + j) * 16 + r) * 8 + i];
                const int G = t - zp * xsl[8 * j + i];
                vl[i] = fmaf((float)G, scale, 0.0f);
            }
        }
        // reduce_add: (L, L + 8) pairs lanes j = 0, 1 (16 apart), the rest in-lane
#pragma unroll
        for (int i = 0; i < 8; i++) vl[i] = vl[i] + __shfl_down(vl[i], 16);
        const float b0 = vl[0] + vl[4], b1 = vl[1] + vl[5], b2 = vl[2] + vl[6], b3 = vl[3] + vl[7];
        const float c0 = b0 + b2, c1 = b1 + b3;
        const float v = c0 + c1;
        if (j == 0 && row_ok) {
            float y = v * sx;
            if (a.flags & LLMQ_BIAS) y += a.bias[o];
            if (a.flags & LLMQ_GELU) y = gelu_ref(y);
            if (a.flags & LLMQ_RESID) y += a.out[o];
            a.out[o] = y;
            best_v = y;
            best_i = o;
        }
    }
    if (a.amax) {
        // largest output of the workgroup; equal values keep the smaller
        // index (argmax's first maximum, gpt2t.mojo:792-797)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best_v, off);
            const int oi = __shfl_xor(best_i, off);
            if (ov > best_v || (ov == best_v && oi < best_i)) {
                best_v = ov;
                best_i = oi;
            }
        }
        if (lane == 0) s_best[wid] = ArgmaxPart{best_v, best_i};
        llmq_lds_barrier();
        if (tid == 0) {
            ArgmaxPart b = s_best[0];
            for (int q = 1; q < NW; q++) {
                const ArgmaxPart c = s_best[q];
                if (c.v > b.v || (c.v == b.v && c.idx < b.idx)) b = c;
            }
            a.amax[blockIdx.x] = b;
        }
    }
}

// ------------------------------------------------------------ launchers

int upt_for(int K, int nt) { return (K / 4 + nt - 1) / nt; }

template <int NW, bool LN, int UPT>
void blk_launch_win(llmq_ctx *ctx, const BlkArgs &a, int grid, size_t lds, int win) {
#define BLK(W, D) hipLaunchKernelGGL((gemv_blk_kernel<NW, LN, UPT, W, D>), dim3((unsigned)grid), dim3(NW * 64), lds, \
                                     ctx->stream, a)
    if (a.dbg) {
        if constexpr (!LN) {
            BLK(4, true);
            return;
        }
    }
    if (win <= 4) BLK(4, false); else if (win <= 8) BLK(8, false); else BLK(16, false);
#undef BLK
}

template <int NW, bool LN>
int blk_launch_upt(llmq_ctx *ctx, const BlkArgs &a, int grid, size_t lds, int win) {
    switch (upt_for(a.K, NW * 64)) {
        case 1: blk_launch_win<NW, LN, 1>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 2: blk_launch_win<NW, LN, 2>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 3: blk_launch_win<NW, LN, 3>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 4: blk_launch_win<NW, LN, 4>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 5: case 6: blk_launch_win<NW, LN, 6>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 7: case 8: blk_launch_win<NW, LN, 8>(ctx, a, grid, lds, win); return LLMQ_OK;
    }
    return llmq_set_error(LLMQ_EUNSUPPORTED, "linear: reduction axis %d too long for %d waves", a.K, NW);
}

}  // namespace

// Which matrices the exact one-token kernels take.
bool gemv_exact_supports(const llmq_mat *w) {
    if (w->kind != MAT_QUANT || !w->a16) return false;
    const int64_t code_bytes = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256;
    if (code_bytes >= (int64_t)kLlmqOOB || (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 32 >= (int64_t)kLlmqOOB) return false;
    if (w->bits == 4 && w->group == 32) return w->k % 256 == 0 && w->k / 4 <= 8 * 256;  // BLOCKED
    if (w->bits == 8 && w->NG == 1) return w->k % 64 == 0 && w->k <= 4096;  // int8 per channel: 4 units a thread
    return false;
}

// Workgroups (= argmax partials) of the head kernel for w.
static void head8_shape(const llmq_mat *w, int *nw, int *tpw, int *grid) {
    // one tile per 4-wave workgroup: 12 steps of a 768-input row make 3 a wave
    *nw = 4;
    *tpw = 1;
    *grid = (int)w->ntiles;
}

int gemv_exact_num_parts(const llmq_mat *w) {
    int nw, tpw, grid;
    head8_shape(w, &nw, &tpw, &grid);
    return w->bits == 8 ? grid : 0;
}

int launch_gemv_exact(llmq_ctx *ctx, const GemvRequest &rq) {
    const llmq_mat *w = rq.w;
    LLMQ_REQUIRE(rq.T == 1 && gemv_exact_supports(w), "linear: no exact one-token kernel for this matrix");
    const bool ln = rq.ln_w != nullptr;
    const int K = (int)w->k;
    if (w->bits == 4) {
        LLMQ_REQUIRE(!rq.amax, "linear: argmax partials need the int8 head kernel");
        BlkArgs a;
        a.codes = reinterpret_cast<const uint4 *>(w->codes);
        a.scales = w->scales;
        a.zps = w->zps;
        a.codes_bytes = (uint32_t)((w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256);
        a.scales_bytes = (uint32_t)((w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS * 2);
        a.zps_bytes = (uint32_t)((w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS);
        a.n = (int)w->n;
        a.K = K;
        a.CK = (int)w->CK;
        a.nwaves = (int)(2 * w->ntiles);
        a.flags = rq.flags;
        a.x = rq.x;
        a.ln_w = rq.ln_w;
        a.ln_b = rq.ln_b;
        a.bias = rq.bias ? rq.bias : rq.out;
        a.out = rq.out;
        a.dbg = rq.dbg;
        a.xq_out = rq.xq_out;
        a.sx_out = rq.sx_out;
        int nw = 4;
        if (const char *e = getenv("LLMQ_BLK_NW")) nw = atoi(e) == 1 ? 1 : atoi(e) == 2 ? 2 : atoi(e) == 8 ? 8 : 4;
        int win = K / 256 <= 4 ? 4 : K / 256 <= 8 ? 8 : 16;
        const int64_t bytes = w->ntiles * w->CK * 256;
        if (bytes >= (20ll << 20)) win = 4;  // streamed from HBM: a few blocks in flight per wave
        if (const char *e = getenv("LLMQ_BLK_WIN")) win = atoi(e);
        const int grid = (int)((a.nwaves + nw - 1) / nw);
        const size_t lds = (size_t)w->CK * (kPlaneStride + 2) * 4 + (ln ? (size_t)K * 4 : 0);
        LLMQ_REQUIRE(lds <= 64 * 1024, "linear: %zu bytes of LDS", lds);
        int rc;
        switch (nw) {
            case 1: rc = ln ? blk_launch_upt<1, true>(ctx, a, grid, lds, win) : blk_launch_upt<1, false>(ctx, a, grid, lds, win); break;
            case 2: rc = ln ? blk_launch_upt<2, true>(ctx, a, grid, lds, win) : blk_launch_upt<2, false>(ctx, a, grid, lds, win); break;
            case 8: rc = ln ? blk_launch_upt<8, true>(ctx, a, grid, lds, win) : blk_launch_upt<8, false>(ctx, a, grid, lds, win); break;
            default: rc = ln ? blk_launch_upt<4, true>(ctx, a, grid, lds, win) : blk_launch_upt<4, false>(ctx, a, grid, lds, win); break;
        }
        if (rc != LLMQ_OK) return rc;
        LLMQ_HIP(hipGetLastError());
        return LLMQ_OK;
    }
    // int8 per channel
    LLMQ_REQUIRE(!rq.dbg, "linear: chunk sums are not kept by the int8 head kernel");
    int nw, tpw, grid;
    head8_shape(w, &nw, &tpw, &grid);
    LLMQ_REQUIRE(!rq.amax || grid <= rq.amax_cap, "linear: %d argmax partials exceed capacity %d", grid, rq.amax_cap);
    Ch8Args a;
    a.codes = reinterpret_cast<const uint4 *>(w->codes);
    a.scales = w->scales;
    a.zps = w->zps;
    a.codes_bytes = (uint32_t)((w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256);
    a.n = (int)w->n;
    a.K = K;
    a.CK = (int)w->CK;
    a.ntiles = (int)w->ntiles;
    a.flags = rq.flags;
    a.x = rq.x;
    a.ln_w = rq.ln_w;
    a.ln_b = rq.ln_b;
    a.bias = rq.bias ? rq.bias : rq.out;
    a.out = rq.out;
    a.amax = rq.amax;
    a.xq_out = rq.xq_out;
    a.sx_out = rq.sx_out;
    const int S = (int)(w->CK / 4), spw = (S + (nw / tpw) - 1) / (nw / tpw);
    const size_t lds = (size_t)K * 2 + (size_t)tpw * (nw / tpw) * 2 * 16 * 8 * 4 + (ln ? (size_t)K * 4 : 0);
    LLMQ_REQUIRE(lds <= 64 * 1024, "head: %zu bytes of LDS", lds);
    const int upt = upt_for(K, nw * 64);
#define H8(U, SP)                                                                                       \
    do {                                                                                                \
        if (ln)                                                                                         \
            hipLaunchKernelGGL((head8_kernel<4, 1, true, U, SP>), dim3((unsigned)grid), dim3(256), lds,  \
                               ctx->stream, a);                                                         \
        else                                                                                            \
            hipLaunchKernelGGL((head8_kernel<4, 1, false, U, SP>), dim3((unsigned)grid), dim3(256), lds, \
                               ctx->stream, a);                                                         \
    } while (0)
    if (upt == 1 && spw <= 4) H8(1, 4);
    else if (upt <= 4 && spw <= 4) H8(4, 4);
    else if (upt <= 4 && spw <= 16) H8(4, 16);
    else return llmq_set_error(LLMQ_EUNSUPPORTED, "head: reduction axis %d too long", K);
#undef H8
    LLMQ_HIP(hipGetLastError());
    if (rq.amax_count) *rq.amax_count = grid;
    return LLMQ_OK;
}
