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
//
// Activations come either as float rows (each workgroup then runs
// LayerNorm / quantize_rows / the plane transform in its prologue), or as a
// prepared record (REC: linear_team's xq / xp / xs / sx, built once by
// act_prep_kernel), which the GEMV streams against with no prologue.
#include "common.h"

namespace {

constexpr int kPlaneStride = 20;  // dwords per 32-activation chunk in LDS (16 used; no bank conflicts)

// A 128-bit buffer load of streamed weight codes, marked non-temporal (no
// reuse expected: the caches keep the activations instead).
__device__ __forceinline__ uint4 bload16_stream(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

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

// Wave 0's copy of the row for LayerNorm's 16 lane chains (NV > 0): lane
// l holds v[i] = x[16 i + l], loaded straight from memory.
template <int NV>
__device__ __forceinline__ void load_lnv(const float *x, float (&v)[NV > 0 ? NV : 1]) {
    if constexpr (NV > 0) {
        if (threadIdx.x < 64) {
            const auto r = llmq_rsrc(x, (uint32_t)NV * 64u);
            const uint32_t l = threadIdx.x & 15;
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = __uint_as_float(llmq_bload4(r, (16u * i + l) * 4u));
        }
    }
}

// LayerNorm (optional), then quantize_rows' scale: the row in xv is
// replaced by the normalized one; returns sx.  LayerNorm's statistics come
// from wave 0's registers (NV > 0, see load_lnv) or from the row staged in
// xs (K floats of LDS).  bc: 2 floats, red: NT / 64.  Ends with a barrier.
template <int NT, int UPT, bool LN, int NV>
__device__ __forceinline__ float act_prologue(float4 (&xv)[UPT], const float4 (&lw)[UPT], const float4 (&lb)[UPT],
                                              const float (&lnv)[NV > 0 ? NV : 1], int K, float *xs, float *bc,
                                              float *red) {
    const int nunits = K / 4;
    if (LN) {
        float mean, rstd;
        if constexpr (NV > 0) {
            if (threadIdx.x < 64) {
                const float2 st = llmq_ln_stats_regs<NV>(lnv);
                if (threadIdx.x == 0) {
                    bc[0] = st.x;
                    bc[1] = st.y;
                }
            }
            llmq_lds_barrier();
            mean = bc[0];
            rstd = bc[1];
        } else {
#pragma unroll
            for (int i = 0; i < UPT; i++) {
                const int u = threadIdx.x + NT * i;
                if (u < nunits) reinterpret_cast<float4 *>(xs)[u] = xv[i];
            }
            llmq_lds_barrier();
            llmq_ln_stats(xs, K, bc, mean, rstd);
        }
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
    m = llmq_wave_max(m);
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

// quantize_rows' codes of the normalized row xv (scale sx) in the forms the
// GEMVs read: with `planes` (PS dwords a 32-activation chunk), the four
// nibble planes of X = xq + 32768 per code dword and the per-half-group
// sums of xq; with `xq`, the codes themselves; with `xsl` (16 ints of LDS,
// zeroed), reference lane L's sum of its activation pairs (2L, 2L + 1) of
// every 32-activation piece (int8 per channel).  Every thread must take part
// (DPP exchanges); the pointers may be LDS or global memory.
template <int NT, int UPT, int PS>
__device__ __forceinline__ void build_act(const float4 (&xv)[UPT], float sx, int K, uint32_t *planes, int *hsum,
                                          int16_t *xq, int *xsl) {
    const float inv = 1.0f / sx;
    const int nunits = K >> 2;
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = threadIdx.x + NT * i;
        const int q0 = q_round(xv[i].x * inv), q1 = q_round(xv[i].y * inv);
        const int q2 = q_round(xv[i].z * inv), q3 = q_round(xv[i].w * inv);
        if (xq && u < nunits) {
            const uint32_t lo = ((uint32_t)q0 & 0xFFFFu) | ((uint32_t)q1 << 16);
            const uint32_t hi = ((uint32_t)q2 & 0xFFFFu) | ((uint32_t)q3 << 16);
            reinterpret_cast<uint2 *>(xq)[u] = make_uint2(lo, hi);
        }
        if (xsl && u < nunits) {  // unit u holds pairs 2 (u & 7), 2 (u & 7) + 1 of its 32-piece
            atomicAdd(&xsl[2 * (u & 7)], q0 + q1);
            atomicAdd(&xsl[2 * (u & 7) + 1], q2 + q3);
        }
        if (planes) {
            // sum over the half (4 consecutive units = 4 consecutive lanes)
            int qs = (q0 + q1) + (q2 + q3);
            qs += dppi<kQuadXor1>(qs);
            qs += dppi<kQuadXor2>(qs);
            uint32_t A = (uint32_t)(q0 + 32768) | ((uint32_t)(q1 + 32768) << 16);
            uint32_t B = (uint32_t)(q2 + 32768) | ((uint32_t)(q3 + 32768) << 16);
            nibble_transpose(A, B);
            // units 2i, 2i + 1 of a chunk make the plane dwords of code
            // dword i: the even unit stores planes 0, 1, the odd one 2, 3
            const bool odd = u & 1;
            const uint32_t other = (uint32_t)dppi<kQuadXor1>((int)(odd ? A : B));
            const uint32_t mine = odd ? B : A;
            const uint32_t lo_src = odd ? other : mine, hi_src = odd ? mine : other;
            const uint32_t pa = __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);
            const uint32_t pb = __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);
            if (u < nunits) {
                const int c = u >> 3, e = u & 7;
                reinterpret_cast<uint2 *>(planes + c * PS + 4 * (e >> 1) + 2 * (e & 1))[0] = make_uint2(pa, pb);
                if ((u & 3) == 0) hsum[2 * c + (e >> 2)] = qs;
            }
        }
    }
}

// The prepared record of one token's activations (linear_team's xq, xp,
// xs, sx; llmq_act_prepare): one workgroup.
template <int NT, int UPT, bool LN>
__global__ __launch_bounds__(NT) void act_prep_kernel(const float *__restrict__ x, const float *__restrict__ ln_w,
                                                      const float *__restrict__ ln_b, int K, uint8_t *__restrict__ rec) {
    extern __shared__ __align__(16) float xs[];  // [K] (LayerNorm)
    __shared__ float bc[2], red[NT / 64];
    __shared__ int xsl[16];
    const ActLayout L = llmq_act_layout(K);
    const int nunits = K >> 2;
    float4 xv[UPT], lw[UPT], lb[UPT];
    load_row<NT, UPT>(x, nunits, xv);
    if (LN) {
        load_row<NT, UPT>(ln_w, nunits, lw);
        load_row<NT, UPT>(ln_b, nunits, lb);
    }
    if (threadIdx.x < 16) xsl[threadIdx.x] = 0;
    const float none[1] = {0.0f};
    const float sx = act_prologue<NT, UPT, LN, 0>(xv, lw, lb, none, K, xs, bc, red);
    build_act<NT, UPT, 16>(xv, sx, K, reinterpret_cast<uint32_t *>(rec + L.planes), reinterpret_cast<int *>(rec + L.hsum),
                           reinterpret_cast<int16_t *>(rec + L.xq), xsl);
    llmq_lds_barrier();
    if (threadIdx.x < 16) reinterpret_cast<int *>(rec + L.xsl)[threadIdx.x] = xsl[threadIdx.x];
    if (threadIdx.x == 0) reinterpret_cast<float *>(rec + L.sx)[0] = sx;
}

// ---------------------------------------------------------------- BLOCKED

// The embed step taken into the prologue (EMB): the embedding's codes (int8,
// or int4 nibbles, in tiles of 16 rows as embed_kernel reads them), scales
// and zero points, the position rows, the previous head's argmax partials
// and the decode state.
struct EmbArgs {
    const uint8_t *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    const float *wpe;
    const ArgmaxPart *parts;
    int64_t *gen;
    int *state;
    float *x;
    uint32_t codes_bytes, meta_rows, wpe_bytes;  // meta_rows: scale / zero-point entries
    int bits, CK, NG, cpg, n_rows, nparts;
};

struct BlkArgs {
    const uint4 *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    uint32_t codes_bytes, scales_bytes, zps_bytes;
    int n, K, CK, nwaves, flags;
    const float *x, *ln_w, *ln_b, *bias;
    const uint8_t *rec;
    float *out;
    int32_t *dbg;
    int16_t *xq_out;
    float *sx_out;
    ArgmaxPart *amax;  // per-workgroup argmax partials (a head), or null
    int *state_copy;   // state[0..1] = state[2..3] by one thread, or null
    EmbArgs e;
};

// EMB, the loads issued first: the decode state and the first 4 NT argmax
// partials (indices past the end re-read the last partial, which cannot
// change the pick).
template <int NT>
__device__ __forceinline__ void emb_issue(const EmbArgs &e, int &st0, int &st1, ArgmaxPart (&ep)[4]) {
    st0 = e.state[0];
    st1 = e.state[1];
#pragma unroll
    for (int k = 0; k < 4; k++) ep[k] = e.parts[min((int)threadIdx.x + NT * k, e.nparts - 1)];
}

// EMB, the rest of embed_kernel's work for this workgroup: the pick (the
// larger value wins, equal values keep the smaller index: a total order, so
// any reduction order gives embed_kernel's token), then this thread's units
// of the row, x = ((u - zp) * s) + wpe[pos] (row_op, tensor.mojo:463-473),
// staged in xs; wave 0's LayerNorm copy (lnv: lane l holds x[16 i + l]) is
// read back from there.  Workgroup 0 stores the row, gen[step] and the new
// position and step (state[2], state[3]).  Ends with a barrier.
template <int NT, int UPT, int NV>
__device__ __forceinline__ void emb_row(const EmbArgs &e, int st0, int st1, const ArgmaxPart (&ep)[4],
                                        float4 (&xv)[UPT], float (&lnv)[NV > 0 ? NV : 1], float *xs, int nunits) {
    constexpr int NW = NT / 64;
    __shared__ float s_v[NW];
    __shared__ int s_i[NW];
    const int tid = threadIdx.x;
    const int pos = st0 + 1, step = st1 + 1;
    // the position row first: it needs only the state
    const auto rp = llmq_rsrc(e.wpe, e.wpe_bytes);
    float4 wp[UPT];
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const uint32_t u = (uint32_t)(tid + NT * i);
        const uint4 f = llmq_bload16(rp, u < (uint32_t)nunits ? ((uint32_t)pos * (uint32_t)nunits + u) * 16u : kLlmqOOB);
        wp[i] = make_float4(__uint_as_float(f.x), __uint_as_float(f.y), __uint_as_float(f.z), __uint_as_float(f.w));
    }
    float v = -INFINITY;
    int idx = 0x7fffffff;
    auto take = [&](float cv, int ci) {
        if (cv > v || (cv == v && ci < idx)) {
            v = cv;
            idx = ci;
        }
    };
#pragma unroll
    for (int k = 0; k < 4; k++) take(ep[k].v, ep[k].idx);
    for (int p = tid + 4 * NT; p < e.nparts; p += NT) take(e.parts[p].v, e.parts[p].idx);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const int oi = __shfl_xor(idx, off);
        take(ov, oi);
    }
    if ((tid & 63) == 0) {
        s_v[tid >> 6] = v;
        s_i[tid >> 6] = idx;
    }
    llmq_lds_barrier();
    v = s_v[0];
    idx = s_i[0];
#pragma unroll
    for (int w = 1; w < NW; w++) take(s_v[w], s_i[w]);
    // an argmax over logits that are all NaN has no index: token 0's row
    const int row = (idx >= 0 && idx < e.n_rows) ? idx : 0;
    const uint32_t tile = (uint32_t)row >> 4, r = (uint32_t)row & 15u;
    const auto rc = llmq_rsrc(e.codes, e.codes_bytes);
    const auto rs = llmq_rsrc(e.scales, e.meta_rows * 2u);
    const auto rz = llmq_rsrc(e.zps, e.meta_rows);
    uint32_t cw[UPT], sb[UPT], zb[UPT];
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const uint32_t u = (uint32_t)(tid + NT * i), k0 = 4u * u;
        const bool ok = u < (uint32_t)nunits;
        // the unit's four codes: bytes k0 % 16 .. + 3 of a 16-code chunk, or
        // nibbles k0 % 32 .. + 3 (two bytes) of a 32-code one
        const uint32_t c = e.bits == 4 ? k0 >> 5 : k0 >> 4;
        const uint32_t off = ((tile * (uint32_t)e.CK + c) * 16u + r) * 16u + (e.bits == 4 ? (k0 & 31u) >> 1 : k0 & 15u);
        cw[i] = llmq_bload4(rc, ok ? off & ~3u : kLlmqOOB) >> (8u * (off & 3u));
        const uint32_t gi = (tile * (uint32_t)e.NG + c / (uint32_t)e.cpg) * 16u + r;
        sb[i] = llmq_bload2(rs, ok ? gi * 2u : kLlmqOOB);
        zb[i] = llmq_bload1(rz, ok ? gi : kLlmqOOB);
    }
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const float s = __half2float(__ushort_as_half((unsigned short)sb[i]));
        const float zp = (float)zb[i];
        float q[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t u = e.bits == 4 ? (cw[i] >> (4 * j)) & 15u : (cw[i] >> (8 * j)) & 255u;
            q[j] = ((float)u - zp) * s;
        }
        xv[i] = make_float4(q[0] + wp[i].x, q[1] + wp[i].y, q[2] + wp[i].z, q[3] + wp[i].w);
        const int u = tid + NT * i;
        if (u < nunits) {
            reinterpret_cast<float4 *>(xs)[u] = xv[i];
            if (blockIdx.x == 0) reinterpret_cast<float4 *>(e.x)[u] = xv[i];
        }
    }
    if (blockIdx.x == 0 && tid == 0) {
        e.gen[step] = idx;
        e.state[2] = pos;
        e.state[3] = step;
    }
    llmq_lds_barrier();
    if constexpr (NV > 0) {
        if (tid < 64) {
#pragma unroll
            for (int i = 0; i < NV; i++) lnv[i] = xs[16 * i + (tid & 15)];
        }
    }
}

// Workgroup: NW waves over NW / KS row octets; the KS waves of an octet
// split its blocks into contiguous runs and leave each block's exact
// half-group sums and scale in LDS, from which the octet's first wave runs
// the two fma chains over all blocks in order.  REC: the activations'
// planes and half sums are read from the prepared record, a block's worth
// with its codes.
template <int NW, int KS, bool LN, int UPT, int WIN, bool DBG, bool REC, int NV, bool EMB>
__global__ __launch_bounds__(NW * 64) void gemv_blk_kernel(BlkArgs a) {
    constexpr int NT = NW * 64, OPW = NW / KS;
    extern __shared__ __align__(16) uint32_t smem[];
    uint32_t *planes = smem;                                             // [CK][kPlaneStride]
    int *hsum = reinterpret_cast<int *>(smem + a.CK * kPlaneStride);     // [CK][2] sum of xq per half
    float *xs = reinterpret_cast<float *>(hsum + 2 * a.CK);              // [K] (LayerNorm)
    // each octet's per-block exact half sums and scales, [OPW][nb][3][64]
    float *hand = xs + (LN ? a.K : 0);
    __shared__ float bc[2], red[NW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ol = wid / KS, ks = wid % KS;
    const int gw = blockIdx.x * OPW + ol;  // global octet: rows 8 gw .. 8 gw + 7
    const bool live = gw < a.nwaves;
    const int tile = gw >> 1, rr = 8 * (gw & 1) + (lane & 7), g = lane >> 3;
    const int o = tile * 16 + rr;
    const int nb = a.K >> 8;
    const int b_lo = (ks * nb) / KS, b_hi = ((ks + 1) * nb) / KS;
    const int nunits = a.K >> 2;
    const ActLayout AL = llmq_act_layout(a.K);

    // Activations first, then the first WIN blocks of codes, scales and zero
    // points (and record planes), then the epilogue operands: all in flight
    // before any wait.
    float4 xv[UPT], lw[UPT], lb[UPT];
    float lnv[NV > 0 ? NV : 1];
    int e_st0 = 0, e_st1 = 0;  // EMB: the decode state and the first argmax partials instead of a row
    ArgmaxPart ep[4];
    if (!REC) {
        if constexpr (EMB) {
            emb_issue<NT>(a.e, e_st0, e_st1, ep);
        } else {
            if (LN) load_lnv<NV>(a.x, lnv);
            load_row<NT, UPT>(a.x, nunits, xv);
        }
        if (LN) {
            load_row<NT, UPT>(a.ln_w, nunits, lw);
            load_row<NT, UPT>(a.ln_b, nunits, lb);
        }
    }
    if (a.state_copy && blockIdx.x == 0 && tid == 0) {
        a.state_copy[0] = a.state_copy[2];
        a.state_copy[1] = a.state_copy[3];
    }
    const auto rc = llmq_rsrc(a.codes, a.codes_bytes);
    const auto rs = llmq_rsrc(a.scales, a.scales_bytes);
    const auto rz = llmq_rsrc(a.zps, a.zps_bytes);
    const auto rr_ = llmq_rsrc(a.rec, REC ? (uint32_t)AL.bytes : 0u);
    // block b of this lane: chunk c = 8 b + g of row o (g32: chunk = group)
    auto code_off = [&](int b) -> uint32_t {
        const uint32_t c = (uint32_t)(8 * b + g);
        return live && b < b_hi ? (((uint32_t)tile * (uint32_t)a.CK + c) * 16u + (uint32_t)rr) * 16u : kLlmqOOB;
    };
    auto meta_off = [&](int b) -> uint32_t {  // [tile][group][16 rows]
        const uint32_t c = (uint32_t)(8 * b + g);
        return live && b < b_hi ? ((uint32_t)tile * (uint32_t)a.CK + c) * 16u + (uint32_t)rr : kLlmqOOB;
    };
    // REC: the record's planes and half sums (72 bytes a chunk), 16 bytes
    // a thread per round, requested before the weights
    constexpr int RPT = REC ? 6 : 1;  // rounds: up to 6 * 16 * NT bytes (K = 8192 at NT = 256)
    uint4 wr[RPT];
    if constexpr (REC) {
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const uint32_t off = (uint32_t)(tid + NT * i) * 16u;
            wr[i] = llmq_bload16(rr_, off < (uint32_t)AL.xq ? off : kLlmqOOB);
        }
    }
    // Codes, and the dwords holding the row's scale (16 bits at 16 (rr & 1)) and
    // zero point (8 bits at 8 (rr & 3)): whole-dword values in flight need no
    // masking until they are used.
    uint4 wc[WIN];
    uint32_t wsc[WIN], wzp[WIN];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < WIN; u++) {
        wc[u] = bload16_stream(rc, code_off(b_lo + u));
        const uint32_t mo = meta_off(b_lo + u);
        wsc[u] = llmq_bload4(rs, mo == kLlmqOOB ? kLlmqOOB : (mo * 2u) & ~3u);
        wzp[u] = llmq_bload4(rz, mo & ~3u);
    }
    const bool row_ok = live && ks == 0 && g == 0 && o < a.n;
    const auto rb = llmq_rsrc(a.bias, (uint32_t)a.n * 4u);
    const auto ro = llmq_rsrc(a.out, (uint32_t)a.n * 4u);
    const float e_bias = __uint_as_float(llmq_bload4(rb, row_ok ? (uint32_t)o * 4u : kLlmqOOB));
    const float e_res = __uint_as_float(llmq_bload4(ro, row_ok ? (uint32_t)o * 4u : kLlmqOOB));
    float sx;
    if constexpr (REC) sx = __uint_as_float(llmq_bload4(rr_, (uint32_t)AL.sx));
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (!REC) {
        if constexpr (EMB) emb_row<NT, UPT, NV>(a.e, e_st0, e_st1, ep, xv, lnv, xs, nunits);
        // Prologue: LayerNorm, quantize_rows, nibble planes and half sums.
        sx = act_prologue<NT, UPT, LN, NV>(xv, lw, lb, lnv, a.K, xs, bc, red);
        const bool xq_dbg = a.xq_out != nullptr && blockIdx.x == 0;
        if (xq_dbg && tid == 0 && a.sx_out) a.sx_out[0] = sx;
        build_act<NT, UPT, kPlaneStride>(xv, sx, a.K, planes, hsum, xq_dbg ? a.xq_out : nullptr, nullptr);
    } else {
        // the staged record into LDS: plane chunks re-strided, half sums as they are
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const uint32_t q = (uint32_t)(tid + NT * i);  // 16-byte piece of the record
            if (q * 16u < (uint32_t)AL.hsum)
                reinterpret_cast<uint4 *>(planes + (q >> 2) * kPlaneStride)[q & 3] = wr[i];
            else if (q * 16u < (uint32_t)AL.xq)
                reinterpret_cast<uint4 *>(hsum)[q - (uint32_t)AL.hsum / 16u] = wr[i];
        }
    }
    llmq_lds_barrier();

    // The wave's blocks in order: the integer half sums, then (KS == 1) the
    // two fma chains, or (KS > 1) the operands handed to wave 0 of the octet.
    float acc0 = 0.0f, acc1 = 0.0f;
    float *hd = hand + (size_t)ol * nb * 192;
    const uint32_t K1 = 0x11111111u;
    // Block b's codes, scale and zero point (zeros past the wave's blocks).
    auto fetch = [&](int b, uint4 &w, uint32_t &sv, uint32_t &zv) {
        w = bload16_stream(rc, code_off(b));
        const uint32_t mo = meta_off(b);
        sv = llmq_bload4(rs, mo == kLlmqOOB ? kLlmqOOB : (mo * 2u) & ~3u);
        zv = llmq_bload4(rz, mo & ~3u);
    };
    // Block b's half sums and scale into the hand-off slots.
    auto block = [&](int b, const uint4 d, uint32_t wscv, uint32_t wzpv) {
        const int c = 8 * b + g;
        const float sc = __half2float(__ushort_as_half((unsigned short)(wscv >> (16 * (rr & 1)))));
        const int zp = (int)((wzpv >> (8 * (rr & 3))) & 255u);
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
        // to LDS: the chains run once every block is in (keeping them
        // out of the loop leaves its iterations independent)
        hd[(b * 3 + 0) * 64 + lane] = (float)G0;
        hd[(b * 3 + 1) * 64 + lane] = (float)G1;
        hd[(b * 3 + 2) * 64 + lane] = sc;
    };
    // Two register sets take turns (blocks b0 .. in wc, b0 + WIN .. in wn), so
    // a block's loads land in the registers the loop reads them from and the
    // WIN blocks in flight stay in flight across iterations (one set, re-filled
    // while its old values were still live, cost a copy, and a wait for the
    // loads just issued, at every iteration's end).
    uint4 wn[WIN];
    uint32_t wsn[WIN], wzn[WIN];
    for (int b0 = b_lo; b0 < b_hi; b0 += 2 * WIN) {
#pragma unroll
        for (int u = 0; u < WIN; u++) {
            const int b = b0 + u;
            const uint4 d = wc[u];
            const uint32_t sv = wsc[u], zv = wzp[u];
            __builtin_amdgcn_sched_barrier(0);
            fetch(b + WIN, wn[u], wsn[u], wzn[u]);
            __builtin_amdgcn_sched_barrier(0);
            if (b < b_hi) block(b, d, sv, zv);  // wave-uniform
        }
#pragma unroll
        for (int u = 0; u < WIN; u++) {
            const int b = b0 + WIN + u;
            const uint4 d = wn[u];
            const uint32_t sv = wsn[u], zv = wzn[u];
            __builtin_amdgcn_sched_barrier(0);
            fetch(b + WIN, wc[u], wsc[u], wzp[u]);
            __builtin_amdgcn_sched_barrier(0);
            if (b < b_hi) block(b, d, sv, zv);
        }
    }
    if constexpr (KS > 1) llmq_lds_barrier();  // (KS == 1: the wave reads its own writes)
    {
        if (ks == 0) {  // the octet's two chains over all blocks, in order
            int b = 0;
            for (; b + 4 <= nb; b += 4) {  // four blocks' operands, then their chains
                float t0[4], t1[4], sc[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    t0[k] = hd[((b + k) * 3 + 0) * 64 + lane];
                    t1[k] = hd[((b + k) * 3 + 1) * 64 + lane];
                    sc[k] = hd[((b + k) * 3 + 2) * 64 + lane];
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    acc0 = fmaf(t0[k], sc[k], acc0);
                    acc1 = fmaf(t1[k], sc[k], acc1);
                }
            }
            for (; b < nb; b++) {
                acc0 = fmaf(hd[(b * 3 + 0) * 64 + lane], hd[(b * 3 + 2) * 64 + lane], acc0);
                acc1 = fmaf(hd[(b * 3 + 1) * 64 + lane], hd[(b * 3 + 2) * 64 + lane], acc1);
            }
        }
    }
    // reduce_add: (L, L + 8) in-lane, then groups g, g + 4 / + 2 / + 1.
    float v = acc0 + acc1;
    v = v + llmq_from_lane_plus32(v);
    v = v + llmq_from_lane_plus16(v);
    v = v + llmq_dppf<0x108>(v);  // row_shl:8
    float r = -INFINITY;
    if (row_ok) {
        r = v * sx;
        if (a.flags & LLMQ_BIAS) r += e_bias;
        if (a.flags & LLMQ_GELU) r = gelu_ref(r);
        if (a.flags & LLMQ_RESID) r += e_res;
        a.out[o] = r;
    }
    if (a.amax) {  // (uniform over the grid: every wave reaches the barrier)
        // largest output of the workgroup; equal values keep the smaller
        // index (argmax's first maximum, gpt2t.mojo:792-797)
        __shared__ ArgmaxPart s_best[NW];
        float best_v = r;
        int best_i = row_ok ? o : 0x7fffffff;
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

// ------------------------------------------------------ int8 per channel

struct Ch8Args {
    const uint4 *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    uint32_t codes_bytes;
    int n, K, CK, ntiles, flags;
    const float *x, *ln_w, *ln_b, *bias;
    const uint8_t *rec;
    float *out;
    ArgmaxPart *amax;
    int16_t *xq_out;
    float *sx_out;
    int iters;         // tile groups a workgroup takes
    int *state_copy;   // state[0..1] = state[2..3] by one thread, or null
};

// Workgroup: NW waves over TPW row tiles at a time (NW / TPW waves share a
// tile's steps, contiguously), for a.iters such groups of tiles, group
// blockIdx.x + i * gridDim.x, the next group's codes requested while the
// current one computes: the activation prologue runs once per workgroup.
// Step s of a tile is chunks 4s .. 4s + 3 of its 16 rows; lane (r, j) =
// (lane & 15, lane >> 4) reads chunk 4s + j.  REC: the int16 codes and lane
// sums come from the prepared record.
template <int NW, int TPW, bool LN, int UPT, int SPW, bool REC, int NV>
__global__ __launch_bounds__(NW * 64) void head8_kernel(Ch8Args a) {
    constexpr int NT = NW * 64, WPT = NW / TPW;  // waves per tile
    extern __shared__ __align__(16) uint32_t smem[];
    int16_t *xq = reinterpret_cast<int16_t *>(smem);                                    // [K] natural order
    int *part = reinterpret_cast<int *>(smem + (REC ? 0 : a.K / 2));                     // [TPW][WPT][2][16][8]
    float *xs = reinterpret_cast<float *>(part + TPW * WPT * 2 * 16 * 8);                // [K] (LayerNorm)
    __shared__ int xsl[16];  // sum of xq over reference lane L's pairs
    __shared__ float bc[2], red[NW];
    __shared__ ArgmaxPart s_best[NW];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, j = lane >> 4;
    const int tl = wid / WPT, wt = wid % WPT;  // tile of the group, wave within the tile
    const int S = a.CK >> 2;  // steps per tile (CK a multiple of 4)
    const int s0 = (wt * S) / WPT, ns = ((wt + 1) * S) / WPT - s0;
    const int nunits = a.K >> 2;
    const ActLayout AL = llmq_act_layout(a.K);
    const auto rr_ = llmq_rsrc(a.rec, REC ? (uint32_t)AL.bytes : 0u);
    auto tile_of = [&](int it) { return (int)((blockIdx.x + (uint32_t)it * gridDim.x) * TPW) + tl; };

    float4 xv[UPT], lw[UPT], lb[UPT];
    float lnv[NV > 0 ? NV : 1];
    if (!REC) {
        if (LN) load_lnv<NV>(a.x, lnv);
        load_row<NT, UPT>(a.x, nunits, xv);
        if (LN) {
            load_row<NT, UPT>(a.ln_w, nunits, lw);
            load_row<NT, UPT>(a.ln_b, nunits, lb);
        }
    }
    if (a.state_copy && blockIdx.x == 0 && tid == 0) {
        a.state_copy[0] = a.state_copy[2];
        a.state_copy[1] = a.state_copy[3];
    }
    const auto rc = llmq_rsrc(a.codes, a.codes_bytes);
    const auto rs = llmq_rsrc(a.scales, (uint32_t)a.ntiles * 32u);
    const auto rz = llmq_rsrc(a.zps, (uint32_t)a.ntiles * 16u);
    uint4 wc[SPW], wn[SPW], wx[REC ? SPW : 1][2];
    uint32_t sc_c, zp_c, sc_n = 0, zp_n = 0;  // this lane's row scale bits and zero point
    // one tile's codes (the steps of this wave) and its row's scale / zero point
    auto load_tile = [&](int tile, uint4 *w, uint32_t &scb, uint32_t &zpb) {
        const bool ok_t = tile < a.ntiles;
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t c = (uint32_t)(4 * (s0 + u) + j);
            const bool ok = ok_t && u < ns;
            w[u] = bload16_stream(rc, ok ? (((uint32_t)tile * (uint32_t)a.CK + c) * 16u + (uint32_t)r) * 16u : kLlmqOOB);
        }
        scb = llmq_bload2(rs, ok_t ? ((uint32_t)tile * 16u + (uint32_t)r) * 2u : kLlmqOOB);
        zpb = llmq_bload1(rz, ok_t ? (uint32_t)tile * 16u + (uint32_t)r : kLlmqOOB);
    };
    __builtin_amdgcn_sched_barrier(0);
    load_tile(tile_of(0), wc, sc_c, zp_c);
    if constexpr (REC) {  // the chunks' int16 codes: the same for every tile
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            const uint32_t c = (uint32_t)(4 * (s0 + u) + j);
            const bool ok = u < ns;
            wx[u][0] = llmq_bload16(rr_, ok ? (uint32_t)AL.xq + c * 32u : kLlmqOOB);
            wx[u][1] = llmq_bload16(rr_, ok ? (uint32_t)AL.xq + c * 32u + 16u : kLlmqOOB);
        }
    }
    float sx;
    if constexpr (REC) {
        sx = __uint_as_float(llmq_bload4(rr_, (uint32_t)AL.sx));
        if (tid < 16) xsl[tid] = (int)llmq_bload4(rr_, (uint32_t)AL.xsl + 4u * tid);
    }
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (!REC) {
        if (tid < 16) xsl[tid] = 0;
        sx = act_prologue<NT, UPT, LN, NV>(xv, lw, lb, lnv, a.K, xs, bc, red);
        const bool xq_dbg = a.xq_out != nullptr && blockIdx.x == 0;
        if (xq_dbg && tid == 0 && a.sx_out) a.sx_out[0] = sx;
        build_act<NT, UPT, 16>(xv, sx, a.K, nullptr, nullptr, xq, xsl);
        if (xq_dbg) {
#pragma unroll
            for (int i = 0; i < UPT; i++) {
                const int u = tid + NT * i;
                if (u < nunits) reinterpret_cast<uint2 *>(a.xq_out)[u] = reinterpret_cast<const uint2 *>(xq)[u];
            }
        }
    }
    llmq_lds_barrier();

    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    typedef short s2 __attribute__((ext_vector_type(2)));
    for (int it = 0; it < a.iters; it++) {
        const int tile = tile_of(it);
        if (it + 1 < a.iters) load_tile(tile_of(it + 1), wn, sc_n, zp_n);
        // 8 int32 lanes of sum x u: lane (r, j) holds reference lanes
        // 8 (j & 1) + i, i = 0..7 (chunk 4s + j has parity j & 1).
        int acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < SPW; u++) {
            if (u < ns) {  // wave-uniform
            const int c = 4 * (s0 + u) + j;
            const uint4 d = wc[u];
            uint4 x0, x1;
            if constexpr (REC) {
                x0 = wx[u][0];
                x1 = wx[u][1];
            } else {
                x0 = reinterpret_cast<const uint4 *>(xq)[2 * c];      // pairs 0..3 of the chunk
                x1 = reinterpret_cast<const uint4 *>(xq)[2 * c + 1];  // pairs 4..7
            }
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
        for (int i = 0; i < 8; i++) acc[i] += llmq_from_lane_plus32(acc[i]);
        if constexpr (WPT > 1) {  // waves of the tile, through LDS (lanes j = 0, 1)
            if (j < 2) {
#pragma unroll
                for (int i = 0; i < 8; i++) part[(((tl * WPT + wt) * 2 + j) * 16 + r) * 8 + i] = acc[i];
            }
            llmq_lds_barrier();
            if (wt == 0) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    int t = 0;
#pragma unroll
                    for (int w = 0; w < WPT; w++) t += part[(((tl * WPT + w) * 2 + j) * 16 + r) * 8 + i];
                    acc[i] = t;
                }
            }
        }
        if (wt == 0) {
            const int o = tile * 16 + r;
            const bool row_ok = tile < a.ntiles && o < a.n;
            const float scale = row_ok ? __half2float(__ushort_as_half((unsigned short)sc_c)) : 0.0f;
            const int zp = row_ok ? (int)zp_c : 0;
            // lane (r, j < 2): reference lanes 8 j + i of row r, as floats
            float vl[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            if (j < 2) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int G = acc[i] - zp * xsl[8 * j + i];
                    vl[i] = fmaf((float)G, scale, 0.0f);
                }
            }
            // reduce_add: (L, L + 8) pairs lanes j = 0, 1 (16 apart), the rest in-lane
#pragma unroll
            for (int i = 0; i < 8; i++) vl[i] = vl[i] + llmq_from_lane_plus16(vl[i]);
            const float b0 = vl[0] + vl[4], b1 = vl[1] + vl[5], b2 = vl[2] + vl[6], b3 = vl[3] + vl[7];
            const float c0 = b0 + b2, c1 = b1 + b3;
            const float v = c0 + c1;
            if (j == 0 && row_ok) {
                float y = v * sx;
                if (a.flags & LLMQ_BIAS) y += a.bias[o];
                if (a.flags & LLMQ_GELU) y = gelu_ref(y);
                if (a.flags & LLMQ_RESID) y += a.out[o];
                a.out[o] = y;
                if (y > best_v || (y == best_v && o < best_i)) {
                    best_v = y;
                    best_i = o;
                }
            }
        }
        if constexpr (WPT > 1) llmq_lds_barrier();  // part is rewritten by the next group
#pragma unroll
        for (int u = 0; u < SPW; u++) wc[u] = wn[u];
        sc_c = sc_n;
        zp_c = zp_n;
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

// LayerNorm's chains from registers for rows up to 768 / 1024 inputs
// (48 / 64 values a lane), from LDS beyond.
inline int ln_nv(int K) { return K == 768 ? 48 : K == 1024 ? 64 : 0; }

template <int NW, int KS, bool LN, int UPT, bool REC, int NV>
void blk_launch_nv(llmq_ctx *ctx, const BlkArgs &a, int grid, size_t lds, int win) {
#define BLK(W, D, E) hipLaunchKernelGGL((gemv_blk_kernel<NW, KS, LN, UPT, W, D, REC, NV, E>), dim3((unsigned)grid), \
                                        dim3(NW * 64), lds, ctx->stream, a)
    if (a.dbg) {
        if constexpr (!LN && !REC) {
            BLK(4, true, false);
            return;
        }
    }
    if constexpr (LN && !REC && NV > 0) {
        if (a.e.parts) {  // (launch_exact admits the embed step only here)
            if (win <= 2) BLK(2, false, true); else BLK(4, false, true);
            return;
        }
    }
    if (win <= 2) BLK(2, false, false); else if (win <= 4) BLK(4, false, false);
    else if (win <= 8) BLK(8, false, false); else BLK(16, false, false);
#undef BLK
}

template <int NW, int KS, bool LN, int UPT, bool REC>
void blk_launch_win(llmq_ctx *ctx, const BlkArgs &a, int grid, size_t lds, int win) {
    if constexpr (LN && UPT == 1) {
        if (ln_nv(a.K) == 48) return blk_launch_nv<NW, KS, LN, UPT, REC, 48>(ctx, a, grid, lds, win);
        if (ln_nv(a.K) == 64) return blk_launch_nv<NW, KS, LN, UPT, REC, 64>(ctx, a, grid, lds, win);
    }
    blk_launch_nv<NW, KS, LN, UPT, REC, 0>(ctx, a, grid, lds, win);
}

template <int NW, int KS, bool LN>
int blk_launch_upt(llmq_ctx *ctx, const BlkArgs &a, int grid, size_t lds, int win) {
    if (a.rec) {
        if constexpr (!LN) {
            blk_launch_win<NW, KS, false, 1, true>(ctx, a, grid, lds, win);
            return LLMQ_OK;
        }
    }
    switch (upt_for(a.K, NW * 64)) {
        case 1: blk_launch_win<NW, KS, LN, 1, false>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 2: blk_launch_win<NW, KS, LN, 2, false>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 3: blk_launch_win<NW, KS, LN, 3, false>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 4: blk_launch_win<NW, KS, LN, 4, false>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 5: case 6: blk_launch_win<NW, KS, LN, 6, false>(ctx, a, grid, lds, win); return LLMQ_OK;
        case 7: case 8: blk_launch_win<NW, KS, LN, 8, false>(ctx, a, grid, lds, win); return LLMQ_OK;
    }
    return llmq_set_error(LLMQ_EUNSUPPORTED, "linear: reduction axis %d too long for %d waves", a.K, NW);
}

template <int KS>
int blk_launch_ks(llmq_ctx *ctx, const BlkArgs &a, bool ln, int grid, size_t lds, int win) {
    return ln ? blk_launch_upt<4, KS, true>(ctx, a, grid, lds, win) : blk_launch_upt<4, KS, false>(ctx, a, grid, lds, win);
}

bool exact_supports(const llmq_mat *w) {
    if (w->kind != MAT_QUANT || !w->a16) return false;
    const int64_t code_bytes = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256;
    if (code_bytes >= (int64_t)kLlmqOOB || (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 32 >= (int64_t)kLlmqOOB) return false;
    if (w->bits == 4 && w->group == 32) return w->k % 256 == 0 && w->k / 4 <= 8 * 256;  // BLOCKED
    if (w->bits == 8 && w->NG == 1) return w->k % 64 == 0 && w->k <= 4096;  // int8 per channel: 4 units a thread
    return false;
}

// Shape of the head kernel for w: nw waves, tpw tiles at a time, grid
// workgroups (= argmax partials), iters tile groups each.  A wave per tile
// and about two workgroups a CU (measured on the 50257 x 768 head: 13.3 us
// with a workgroup per tile, 9.4 us so; LLMQ_HEAD_TPW / LLMQ_HEAD_GRID
// override, for measurement).
void head8_shape(const llmq_mat *w, int *nw, int *tpw, int *grid, int *iters) {
    *nw = 4;
    // a tile's steps in at most 12 registers a wave (S = CK / 4 steps a tile)
    const int64_t S = w->CK / 4;
    int t = S <= 12 ? 4 : S <= 24 ? 2 : 1, g = 512;
    if (const char *e = getenv("LLMQ_HEAD_TPW")) t = atoi(e);
    if (t != 2 && t != 4) t = 1;
    while (t > 1 && (S + 4 / t - 1) / (4 / t) > 16) t /= 2;
    if (const char *e = getenv("LLMQ_HEAD_GRID")) g = atoi(e);  // 0: a workgroup per tile group
    const int groups = (int)((w->ntiles + t - 1) / t);
    if (g <= 0 || g > groups) g = groups;
    *tpw = t;
    *iters = (groups + g - 1) / g;
    *grid = (groups + *iters - 1) / *iters;
}

// Shape of the BLOCKED kernel for w: ks waves a row octet, win blocks in
// flight a wave, grid workgroups (= argmax partials).  4-wave workgroups; KS
// waves per row octet split its blocks so that long rows still spread over
// enough waves (and CUs); two blocks in flight per wave (measured best from
// 768 to 4096 inputs).  LLMQ_BLK_KS / LLMQ_BLK_WIN override, for measurement.
void blk_shape(const llmq_mat *w, bool dbg, int *ks_out, int *win_out, int *grid) {
    const int nb = (int)(w->k / 256);
    int ks = nb >= 8 ? 4 : nb >= 4 ? 2 : 1;
    const int64_t bytes = w->ntiles * w->CK * 256;
    if (bytes >= (20ll << 20)) ks = nb >= 4 ? 2 : 1;
    if (const char *e = getenv("LLMQ_BLK_KS")) ks = atoi(e) == 1 ? 1 : atoi(e) == 2 ? 2 : 4;
    if (dbg) ks = 1;
    int win = 2;
    if (const char *e = getenv("LLMQ_BLK_WIN")) win = atoi(e);
    if (dbg) win = 4;
    const int opw = 4 / ks;
    *ks_out = ks;
    *win_out = win;
    *grid = (int)((2 * w->ntiles + opw - 1) / opw);
}

// Shared by both activation forms: rq.x (floats) or rec (a prepared record).
int launch_exact(llmq_ctx *ctx, const GemvRequest &rq, const uint8_t *rec) {
    const llmq_mat *w = rq.w;
    LLMQ_REQUIRE(rq.T == 1 && exact_supports(w), "linear: no exact one-token kernel for this matrix");
    const bool ln = rq.ln_w != nullptr;
    LLMQ_REQUIRE(!(rec && (ln || rq.dbg || rq.xq_out)), "linear: a prepared record takes no LayerNorm or debug output");
    const int K = (int)w->k;
    if (w->bits == 4) {
        int ks, win, grid;
        blk_shape(w, rq.dbg != nullptr, &ks, &win, &grid);
        LLMQ_REQUIRE(!rq.amax || grid <= rq.amax_cap, "linear: %d argmax partials exceed capacity %d", grid,
                     rq.amax_cap);
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
        a.rec = rec;
        a.bias = rq.bias ? rq.bias : rq.out;
        a.out = rq.out;
        a.dbg = rq.dbg;
        a.xq_out = rq.xq_out;
        a.sx_out = rq.sx_out;
        a.amax = rq.amax;
        a.state_copy = rq.state_copy;
        a.e = EmbArgs{};
        if (const EmbedFold *f = rq.emb) {
            const llmq_mat *E = f->E;
            LLMQ_REQUIRE(!rec && gemv_exact_embed_ok(w, E) && ln && !rq.dbg && f->wpe && f->parts && f->nparts > 0 &&
                             f->gen && f->state && f->x && f->wpe_rows > 0 && f->wpe_rows * K * 4 < (int64_t)kLlmqOOB,
                         "linear: no embed step in this kernel's prologue");
            a.e.codes = E->codes;
            a.e.scales = E->scales;
            a.e.zps = E->zps;
            a.e.wpe = f->wpe;
            a.e.parts = f->parts;
            a.e.gen = f->gen;
            a.e.state = f->state;
            a.e.x = f->x;
            a.e.codes_bytes = (uint32_t)((E->ntiles * E->CK + LLMQ_PAD_CHUNKS) * 256);
            a.e.meta_rows = (uint32_t)((E->ntiles * E->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS);
            a.e.wpe_bytes = (uint32_t)(f->wpe_rows * K * 4);
            a.e.bits = E->bits;
            a.e.CK = (int)E->CK;
            a.e.NG = (int)E->NG;
            a.e.cpg = (int)(E->group / (E->bits == 4 ? 32 : 16));
            a.e.n_rows = (int)E->n;
            a.e.nparts = f->nparts;
        }
        const int nb = K / 256, opw = 4 / ks;
        LLMQ_REQUIRE(!rec || llmq_act_layout(K).xq <= 6 * 16 * 256, "linear_act: reduction axis %d too long", K);
        const size_t lds = (size_t)w->CK * (kPlaneStride + 2) * 4 + (ln ? (size_t)K * 4 : 0) +
                           (size_t)opw * nb * 3 * 64 * 4;
        LLMQ_REQUIRE(lds <= 64 * 1024, "linear: %zu bytes of LDS", lds);
        int rc;
        switch (ks) {
            case 1: rc = blk_launch_ks<1>(ctx, a, ln, grid, lds, win); break;
            case 2: rc = blk_launch_ks<2>(ctx, a, ln, grid, lds, win); break;
            default: rc = blk_launch_ks<4>(ctx, a, ln, grid, lds, win); break;
        }
        if (rc != LLMQ_OK) return rc;
        LLMQ_HIP(hipGetLastError());
        if (rq.amax_count) *rq.amax_count = grid;
        return LLMQ_OK;
    }
    // int8 per channel
    LLMQ_REQUIRE(!rq.dbg, "linear: chunk sums are not kept by the int8 head kernel");
    LLMQ_REQUIRE(!rq.emb, "linear: no embed step in the int8 head kernel's prologue");
    int nw, tpw, grid, iters;
    head8_shape(w, &nw, &tpw, &grid, &iters);
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
    a.rec = rec;
    a.bias = rq.bias ? rq.bias : rq.out;
    a.out = rq.out;
    a.amax = rq.amax;
    a.xq_out = rq.xq_out;
    a.sx_out = rq.sx_out;
    a.iters = iters;
    a.state_copy = rq.state_copy;
    const int S = (int)(w->CK / 4), spw = (S + (nw / tpw) - 1) / (nw / tpw);
    const size_t lds = (rec ? 0 : (size_t)K * 2) + (size_t)tpw * (nw / tpw) * 2 * 16 * 8 * 4 + (ln ? (size_t)K * 4 : 0);
    LLMQ_REQUIRE(lds <= 64 * 1024, "head: %zu bytes of LDS", lds);
    const int upt = upt_for(K, nw * 64);
#define H8T(T, LNV, U, SP, R, NV) \
    hipLaunchKernelGGL((head8_kernel<4, T, LNV, U, SP, R, NV>), dim3((unsigned)grid), dim3(256), lds, ctx->stream, a)
#define H8(LNV, U, SP, R, NV)                      \
    do {                                           \
        if (tpw == 4) H8T(4, LNV, U, SP, R, NV);   \
        else if (tpw == 2) H8T(2, LNV, U, SP, R, NV); \
        else H8T(1, LNV, U, SP, R, NV);            \
    } while (0)
    if (rec) {
        if (spw <= 4) H8(false, 1, 4, true, 0);
        else if (spw <= 8) H8(false, 1, 8, true, 0);
        else if (spw <= 12) H8(false, 1, 12, true, 0);
        else if (spw <= 16) H8(false, 1, 16, true, 0);
        else return llmq_set_error(LLMQ_EUNSUPPORTED, "head: reduction axis %d too long", K);
    } else if (upt == 1 && spw <= 12) {
        const int sp = spw <= 4 ? 4 : spw <= 8 ? 8 : 12;
#define H8S(LNV, NV)                                  \
    do {                                              \
        if (sp == 4) H8(LNV, 1, 4, false, NV);        \
        else if (sp == 8) H8(LNV, 1, 8, false, NV);   \
        else H8(LNV, 1, 12, false, NV);               \
    } while (0)
        if (ln && ln_nv(K) == 48) H8S(true, 48);
        else if (ln && ln_nv(K) == 64) H8S(true, 64);
        else if (ln) H8S(true, 0);
        else H8S(false, 0);
#undef H8S
    } else if (upt <= 4 && spw <= 4) {
        if (ln) H8(true, 4, 4, false, 0); else H8(false, 4, 4, false, 0);
    } else if (upt <= 4 && spw <= 16) {
        if (ln) H8(true, 4, 16, false, 0); else H8(false, 4, 16, false, 0);
    } else {
        return llmq_set_error(LLMQ_EUNSUPPORTED, "head: reduction axis %d too long", K);
    }
#undef H8T
#undef H8
    LLMQ_HIP(hipGetLastError());
    if (rq.amax_count) *rq.amax_count = grid;
    return LLMQ_OK;
}

}  // namespace

bool gemv_exact_supports(const llmq_mat *w) { return exact_supports(w); }

bool gemv_exact_embed_ok(const llmq_mat *w, const llmq_mat *E) {
    if (!w || !exact_supports(w) || w->bits != 4 || ln_nv((int)w->k) == 0 || upt_for((int)w->k, 256) != 1) return false;
    if (!E || E->kind != MAT_QUANT || (E->bits != 4 && E->bits != 8) || E->k != w->k || E->n > INT32_MAX) return false;
    const int64_t cpc = E->bits == 4 ? 32 : 16;  // codes a chunk
    if (E->group % cpc != 0 || E->group / cpc < 1) return false;
    return (E->ntiles * E->CK + LLMQ_PAD_CHUNKS) * 256 < (int64_t)kLlmqOOB &&
           (E->ntiles * E->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS * 2 < (int64_t)kLlmqOOB;
}

int gemv_exact_num_parts(const llmq_mat *w) {
    int grid;
    if (w->bits == 4) {
        int ks, win;
        blk_shape(w, false, &ks, &win, &grid);
    } else {
        int nw, tpw, iters;
        head8_shape(w, &nw, &tpw, &grid, &iters);
    }
    return grid;
}

int launch_gemv_exact(llmq_ctx *ctx, const GemvRequest &rq) { return launch_exact(ctx, rq, nullptr); }

int launch_act_prepare(llmq_ctx *ctx, const float *x, int64_t K, const float *ln_w, const float *ln_b, void *rec) {
    LLMQ_REQUIRE(x && rec && K >= 32 && K % 32 == 0 && K <= 16384, "act_prepare: K must be a multiple of 32, at most 16384");
    LLMQ_REQUIRE(!ln_w == !ln_b, "act_prepare: LayerNorm needs both weight and bias");
    const bool ln = ln_w != nullptr;
    const size_t lds = ln ? (size_t)K * 4 : 0;
    uint8_t *r = static_cast<uint8_t *>(rec);
#define AP(NT, U)                                                                                                  \
    do {                                                                                                           \
        if (ln)                                                                                                    \
            hipLaunchKernelGGL((act_prep_kernel<NT, U, true>), dim3(1), dim3(NT), lds, ctx->stream, x, ln_w, ln_b, \
                               (int)K, r);                                                                         \
        else                                                                                                       \
            hipLaunchKernelGGL((act_prep_kernel<NT, U, false>), dim3(1), dim3(NT), lds, ctx->stream, x, ln_w,      \
                               ln_b, (int)K, r);                                                                   \
    } while (0)
    if (K <= 1024) AP(256, 1);
    else if (K <= 4096) AP(1024, 1);
    else AP(1024, 4);
#undef AP
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_linear_act(llmq_ctx *ctx, float *out, const void *rec, const llmq_mat *w, const float *bias, int flags) {
    LLMQ_REQUIRE(out && rec && w, "linear_act: bad arguments");
    LLMQ_REQUIRE(exact_supports(w), "linear_act: takes int4-g32-a16 (BLOCKED) and int8 per-channel A16 matrices");
    LLMQ_REQUIRE(!(flags & LLMQ_BIAS) || bias, "linear_act: LLMQ_BIAS without a bias");
    GemvRequest rq;
    rq.w = w;
    rq.out = out;
    rq.bias = bias;
    rq.T = 1;
    rq.flags = flags;
    return launch_exact(ctx, rq, static_cast<const uint8_t *>(rec));
}

// ------------------------------------------------- dot_row_i16 per row

namespace {

// QuantMatrix.dot_row_i16 (tensor.mojo:518-577): four rows a wave, lane
// L = tid & 15 of a row's 16 standing for the reference's SIMD lane L, with
// its int32 sums (wrapping, as VPDPWSSD does), its float chain and the
// 16-lane halving sum, so each result is the reference's bit for bit.
// xq holds the int16 codes in natural column order; the BLOCKED branch
// gathers, for lane L, the activations permute_x_i16 would give it
// (tensor.mojo:498-516: group L % 8, weights 16 (L / 8) .. + 15 of every
// 256-block) and their float sum.  The int8 per-channel branch
// (f32(acc).fma(s, 0)) is the general loop's single group.
__global__ __launch_bounds__(64) void dot_row_i16_kernel(const uint8_t *__restrict__ codes,
                                                         const uint16_t *__restrict__ scales,
                                                         const uint8_t *__restrict__ zps, int bits, int blocked,
                                                         int64_t K, int64_t G, int64_t CK, int64_t NG, int64_t row0,
                                                         int64_t nrows, const int16_t *__restrict__ xq,
                                                         float *__restrict__ out) {
    const int L = threadIdx.x & 15;
    const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 4);
    const bool live = i < nrows;
    const int64_t row = row0 + (live ? i : 0);
    float accf = 0.0f;
    if (blocked) {
        const int64_t tile = row >> 4, r = row & 15;
        const int g = L & 7, h = L >> 3;
        for (int64_t blk = 0; blk < K / 256; blk++) {
            uint32_t acc = 0;
            float xs = 0.0f;
            for (int e = 16 * h; e < 16 * h + 16; e++) {
                const int64_t col = blk * 256 + 32 * g + e;
                const int x = xq[col];
                acc += (uint32_t)(x * llmq_tile_code(codes, 4, CK, row, col));
                xs += (float)x;  // exact: at most 16 * 32767
            }
            const int64_t gi = (tile * NG + blk * 8 + g) * 16 + r;
            const float sc = __half2float(__ushort_as_half(scales[gi]));
            accf = fmaf((float)(int)acc - (float)zps[gi] * xs, sc, accf);
        }
    } else {
        accf = llmq_dot1_lane(codes, scales, zps, bits, K, G, CK, NG, row, xq, L);
    }
    accf = llmq_reduce16(accf);
    if (live && L == 0) out[i] = accf;
}

}  // namespace

int launch_dot_row_i16(llmq_ctx *ctx, const llmq_mat *w, int64_t row0, int64_t nrows, const int16_t *xq, float *out) {
    LLMQ_REQUIRE(w && w->kind == MAT_QUANT, "dot_row_i16: not a QuantMatrix");
    LLMQ_REQUIRE(w->a16, "dot_row_i16: %s has no int16 path (an a16 format is needed)", "the matrix");
    LLMQ_REQUIRE(xq && out, "dot_row_i16: null pointer");
    LLMQ_REQUIRE(row0 >= 0 && nrows >= 1 && row0 + nrows <= w->n, "dot_row_i16: rows %lld..%lld beyond %lld",
                 (long long)row0, (long long)(row0 + nrows), (long long)w->n);
    const int blocked = w->bits == 4 && w->group_param == 32;  // tensor.mojo:296 (K in whole 256-blocks)
    const int64_t grid = (nrows + 3) / 4;
    LLMQ_REQUIRE(grid < (1ll << 31), "dot_row_i16: too many rows");
    hipLaunchKernelGGL(dot_row_i16_kernel, dim3((unsigned)grid), dim3(64), 0, ctx->stream, w->codes, w->scales, w->zps,
                       w->bits, blocked, w->k, w->group, w->CK, w->NG, row0, nrows, xq, out);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
