// Prompt-side W4A16 / W8A16 GEMM on int8 MFMA: matmul_rows_a16 for T > 1
// (kernels.mojo:419-509) with tile_i16's arithmetic (kernels.mojo:512-573).
//
// Per token t, output row o and segment of min(G, 256) inputs of group g
// (G inputs per group; a segment is the group for G <= 256), the exact
// integer
//     G[t, o, seg] = sum_{k in seg} xq[t, k] * (u[o, k] - zp[o, g])
// is computed on the matrix cores, then the float accumulation follows the
// reference operation by operation:
//     acc = fma(float(G), scale[o, g], acc)   (segments in order)
//     y   = acc * sx[t] + b[o]  -> GELU / residual (store_out)
//
// int16 activations go to the int8 MFMA as two planes,
//     x = 256 * hi + (lo - 128) + 128,   hi = x >> 8,  lo = x & 255,
// so sum x*w = 256 * sum hi*w + sum (lo-128)*w + 128 * sum w.  int4 weights
// enter as w = u - zp (|w| <= 15, an int8); int8 weights, whose u - zp needs
// 9 bits, as w = 16 * wh + wl with wl = w & 15 and wh = w >> 4, i.e. four
// MFMA products per 32 inputs.  Every partial is exact in int32 (a segment
// stays within 256 * 32767 * 255 < 2^31, the reference's own flush bound;
// intermediate wraparound cancels).
//
// Mapping: a workgroup of 4 waves owns 64 tokens x 64 output rows (4 row
// tiles); wave (wm, wn) computes the 32 x 32 block (tokens 32 wm.., rows
// 32 wn..) with v_mfma_i32_32x32x32_i8, one call per 32 inputs and plane.
// The reduction axis is walked in staged blocks of 256 inputs (128 or 64
// when those do not divide it), each loaded as 64-input sub-blocks: the next
// block's activations, codes, zero points and scales are loaded into
// registers while the current block, staged in LDS (activation planes,
// weights as int8 rows, per-row weight sums, scales), feeds the matrix cores;
// two LDS buffers alternate, one barrier per block.  Large blocks matter:
// a block costs one memory round trip, and the few workgroups of a prompt
// GEMM cannot hide it behind each other.
//
// Activations come from act_q16_kernel: LayerNorm (kernels.mojo:179-197) when
// asked, then quantize_rows (kernels.mojo:400-416), one workgroup per token.
#include "common.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int TM = 64;           // tokens per workgroup
constexpr int TN = 64;           // output rows per workgroup
constexpr int KB0 = 64;          // inputs per prefetched sub-block
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

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

// ------------------------------------------------------------ activations

__device__ __forceinline__ float block_reduce(float v, float *red, bool is_max) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o);
        v = is_max ? fmaxf(v, w) : v + w;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : ((red[0] + red[1]) + red[2]) + red[3];
}

// One workgroup (256 threads) per token row: optional LayerNorm, then
// quantize_rows.  Values are held in registers, 4 per unit of a float4.
template <bool LN, int UPT>
__global__ __launch_bounds__(256) void act_q16_kernel(const float *__restrict__ x, int64_t ldx,
                                                      const float *__restrict__ lw, const float *__restrict__ lb,
                                                      int K, int16_t *__restrict__ xq, float *__restrict__ sx) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x, nunits = K / 4;
    const float4 *xr = reinterpret_cast<const float4 *>(x + (int64_t)t * ldx);
    float4 v[UPT];
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + 256 * i;
        v[i] = u < nunits ? xr[u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (LN) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < UPT; i++) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        const float mean = block_reduce(s, red, false) / (float)K;
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            if (tid + 256 * i >= nunits) continue;
            const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
            q += (a * a + b * b) + (c * c + d * d);
        }
        const float var = block_reduce(q, red, false) / (float)K;
        const float rstd = 1.0f / sqrtf(var + 1e-5f);
        const float4 *w4 = reinterpret_cast<const float4 *>(lw), *b4 = reinterpret_cast<const float4 *>(lb);
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + 256 * i;
            if (u >= nunits) continue;
            const float4 w = w4[u], b = b4[u];
            v[i].x = ((v[i].x - mean) * rstd) * w.x + b.x;
            v[i].y = ((v[i].y - mean) * rstd) * w.y + b.y;
            v[i].z = ((v[i].z - mean) * rstd) * w.z + b.z;
            v[i].w = ((v[i].w - mean) * rstd) * w.w + b.w;
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < UPT; i++) m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    m = block_reduce(m, red, true);
    float s = m / 32767.0f;
    if (s == 0.0f) s = 1.0f;
    const float inv = 1.0f / s;
    if (tid == 0) sx[t] = s;
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + 256 * i;
        if (u >= nunits) continue;
        const int q0 = llmq_to_int(roundf(v[i].x * inv)), q1 = llmq_to_int(roundf(v[i].y * inv));
        const int q2 = llmq_to_int(roundf(v[i].z * inv)), q3 = llmq_to_int(roundf(v[i].w * inv));
        const uint32_t lo = ((uint32_t)q0 & 0xFFFFu) | ((uint32_t)q1 << 16);
        const uint32_t hi = ((uint32_t)q2 & 0xFFFFu) | ((uint32_t)q3 << 16);
        reinterpret_cast<uint2 *>(xq + (int64_t)t * K)[u] = make_uint2(lo, hi);
    }
}

// ------------------------------------------------------------------- GEMM

struct MfArgs {
    const int16_t *xq;
    const float *sx;
    const uint8_t *codes;
    const uint16_t *scales;
    const uint8_t *zps;
    const float *bias;
    float *out;
    int64_t ldo;
    uint32_t xq_bytes, codes_bytes, scales_bytes, zps_bytes;
    int T, K, n, ntiles, CK, NG, G, seg, flags;
};

// Registers of one 64-input sub-block of a staged block, loaded ahead of
// its use.
template <int BITS>
struct Pref {
    uint4 a0, a1;                        // 16 activations (int16) of one token
    uint4 code;                          // int4: 16 codes in .x, .y; int8: 16 codes
    // zero point byte and float16 scale bits of one (row, sub-step) scale
    // (threads < 128), as the aligned dwords holding them and their bit
    // offsets: extracted where they are used, so no wait follows the loads
    uint32_t zpw, zsh, scw, ssh;
};

// One staged block of NS sub-blocks (KB = 64 NS inputs), double-buffered.
template <int BITS, int NS>
struct Lds {
    static constexpr int KB = KB0 * NS;
    static constexpr int RS = KB + 16;   // row stride in bytes (conflict-free 16-byte reads)
    uint8_t a_hi[2][TM * RS];
    uint8_t a_lo[2][TM * RS];
    uint8_t w0[2][TN * RS];              // int4: u - zp; int8: wl = w & 15
    uint8_t w1[2][BITS == 8 ? TN * RS : 16];  // int8: wh = w >> 4
    int wsum[2][2 * NS][TN];             // sum of w per (32-input sub-step, row)
    float scale[2][2 * NS][TN];          // scale of the group of each (sub-step, row)
    float sx[TM];
};

// Loads of sub-block sb (inputs 64 sb ..) into p.
template <int BITS>
__device__ __forceinline__ void prefetch(const MfArgs &a, int sb, int tok0, int tile0, Pref<BITS> &p,
                                         __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rc,
                                         __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rz) {
    const int t = threadIdx.x, k0 = sb * KB0;
    {   // activations: token m = t / 4, inputs k0 + 16 q ..
        const int m = t >> 2, q = t & 3;
        const int tok = tok0 + m;
        const uint32_t off = tok < a.T ? (uint32_t)(((int64_t)tok * a.K + k0 + 16 * q) * 2) : kOOB;
        p.a0 = bload16(rx, off);
        p.a1 = bload16(rx, off == kOOB ? kOOB : off + 16u);
    }
    int tile, r, g;
    uint32_t coff;
    if (BITS == 4) {  // (tile, chunk c of 32 inputs, row r, half h of 16 inputs)
        const int tt = t >> 6, c = (t >> 5) & 1, h = t & 1;
        r = (t >> 1) & 15;
        tile = tile0 + tt;
        g = (k0 + 32 * c) / a.G;
        coff = (uint32_t)((((int64_t)tile * a.CK + 2 * sb + c) * 16 + r) * 16 + 8 * h);
        const uint2 v = bload8(rc, tile < a.ntiles ? coff : kOOB);
        p.code = make_uint4(v.x, v.y, 0u, 0u);
    } else {          // (tile, chunk c of 16 inputs, row r)
        const int tt = t >> 6, c = (t >> 4) & 3;
        r = t & 15;
        tile = tile0 + tt;
        g = (k0 + 16 * c) / a.G;
        coff = (uint32_t)((((int64_t)tile * a.CK + 4 * sb + c) * 16 + r) * 16);
        p.code = bload16(rc, tile < a.ntiles ? coff : kOOB);
    }
    const uint32_t zoff = tile < a.ntiles ? (uint32_t)(((int64_t)tile * a.NG + g) * 16 + r) : kOOB;
    p.zpw = bload4(rz, zoff == kOOB ? kOOB : (zoff & ~3u));
    p.zsh = 8u * (zoff & 3u);
    {   // scale of (sub-step s, row o) for threads < 2 TN, the others read past the
        // extent: no branch, so the compiler does not wait for every load at its end
        const int s = (t >> 6) & 1, o = t & 63;
        const int tl = tile0 + (o >> 4), gs = (k0 + 32 * s) / a.G;
        const bool ok = t < 2 * TN && tl < a.ntiles;
        const uint32_t soff = ok ? (uint32_t)((((int64_t)tl * a.NG + gs) * 16 + (o & 15)) * 2) : kOOB;
        p.scw = bload4(rs, soff == kOOB ? kOOB : (soff & ~3u));
        p.ssh = 8u * (soff & 2u);
    }
}

// Sub-block j of the staged block in buffer buf, from p.
template <int BITS, int NS>
__device__ __forceinline__ void stage(const Pref<BITS> &p, Lds<BITS, NS> &L, int buf, int j) {
    constexpr int RS = Lds<BITS, NS>::RS;
    const int t = threadIdx.x, col = KB0 * j;
    const uint32_t zp = (p.zpw >> p.zsh) & 255u;
    {   // activation planes: hi bytes and (lo - 128) bytes, natural input order
        const int m = t >> 2, q = t & 3;
        const uint32_t d[8] = {p.a0.x, p.a0.y, p.a0.z, p.a0.w, p.a1.x, p.a1.y, p.a1.z, p.a1.w};
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            hi[i] = __builtin_amdgcn_perm(d[2 * i + 1], d[2 * i], 0x07050301u);
            lo[i] = __builtin_amdgcn_perm(d[2 * i + 1], d[2 * i], 0x06040200u) ^ 0x80808080u;
        }
        *reinterpret_cast<uint4 *>(&L.a_hi[buf][m * RS + col + 16 * q]) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *reinterpret_cast<uint4 *>(&L.a_lo[buf][m * RS + col + 16 * q]) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    if (BITS == 4) {
        const int tt = t >> 6, c = (t >> 5) & 1, r = (t >> 1) & 15, h = t & 1;
        const int o = tt * 16 + r;
        const uint32_t zb = zp * 0x01010101u;
        uint32_t w[4];
        const uint32_t dd[2] = {p.code.x, p.code.y};
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t lo = dd[i] & 0x0F0F0F0Fu, hi = (dd[i] >> 4) & 0x0F0F0F0Fu;
            const uint32_t n0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // weights 8i+0..3
            const uint32_t n1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // weights 8i+4..7
            w[2 * i] = ((n0 | 0x80808080u) - zb) ^ 0x80808080u;               // u - zp as int8
            w[2 * i + 1] = ((n1 | 0x80808080u) - zb) ^ 0x80808080u;
        }
        *reinterpret_cast<uint4 *>(&L.w0[buf][o * RS + col + 32 * c + 16 * h]) = make_uint4(w[0], w[1], w[2], w[3]);
        int s = __builtin_amdgcn_sdot4((int)w[0], 0x01010101, 0, false);
        s = __builtin_amdgcn_sdot4((int)w[1], 0x01010101, s, false);
        s = __builtin_amdgcn_sdot4((int)w[2], 0x01010101, s, false);
        s = __builtin_amdgcn_sdot4((int)w[3], 0x01010101, s, false);
        s += __shfl_xor(s, 1);  // the other half of the chunk
        if (h == 0) L.wsum[buf][2 * j + c][o] = s;
    } else {
        const int tt = t >> 6, c = (t >> 4) & 3, r = t & 15;
        const int o = tt * 16 + r;
        const v2s zz = {(short)zp, (short)zp};
        uint32_t wl[4], wh[4];
        const uint32_t dd[4] = {p.code.x, p.code.y, p.code.z, p.code.w};
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            // 16-bit lanes (u0, u2) and (u1, u3), minus zp, split into nibble parts
            const uint32_t ue = dd[i] & 0x00FF00FFu, uo = (dd[i] >> 8) & 0x00FF00FFu;
            const v2s we = __builtin_bit_cast(v2s, ue) - zz, wo = __builtin_bit_cast(v2s, uo) - zz;
            const uint32_t le = __builtin_bit_cast(uint32_t, we) & 0x000F000Fu, lo = __builtin_bit_cast(uint32_t, wo) & 0x000F000Fu;
            const uint32_t he = __builtin_bit_cast(uint32_t, (v2s)(we >> (v2s){4, 4}));
            const uint32_t ho = __builtin_bit_cast(uint32_t, (v2s)(wo >> (v2s){4, 4}));
            wl[i] = __builtin_amdgcn_perm(lo, le, 0x06020400u);  // (w0, w1, w2, w3) low nibbles
            wh[i] = __builtin_amdgcn_perm(ho, he, 0x06020400u);  // high parts as int8
            s = __builtin_amdgcn_sdot4((int)wh[i], 0x10101010, s, false);  // 16 * wh
            s = __builtin_amdgcn_sdot4((int)wl[i], 0x01010101, s, false);
        }
        *reinterpret_cast<uint4 *>(&L.w0[buf][o * RS + col + 16 * c]) = make_uint4(wl[0], wl[1], wl[2], wl[3]);
        *reinterpret_cast<uint4 *>(&L.w1[buf][o * RS + col + 16 * c]) = make_uint4(wh[0], wh[1], wh[2], wh[3]);
        s += __shfl_xor(s, 16);  // the other chunk of the 32-input sub-step
        if ((c & 1) == 0) L.wsum[buf][2 * j + (c >> 1)][o] = s;
    }
    if (t < 2 * TN)
        L.scale[buf][2 * j + (t >> 6)][t & 63] = __half2float(__ushort_as_half((unsigned short)((p.scw >> p.ssh) & 0xFFFFu)));
}

// Accumulators of one wave: the matrix-core partial sums of the current
// segment (int4: hi, lo planes; int8: hh, hl, lh, ll), the weight sum of the
// segment, and the float outputs (16 tokens of one row per lane).
template <int BITS>
struct Acc {
    v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
    int wacc = 0;
    float acc[16] = {};
};

// The 2 NS sub-steps of 32 inputs of staged block kb (in LDS buffer buf).
template <int BITS, int NS, bool SEG32>
__device__ __forceinline__ void compute_block(const Lds<BITS, NS> &L, int buf, int kb, int arow, int brow, int orow,
                                              int seg, Acc<BITS> &c) {
    constexpr int KB = Lds<BITS, NS>::KB;
#pragma unroll
    for (int s = 0; s < 2 * NS; s++) {
        const v4i ah = *reinterpret_cast<const v4i *>(&L.a_hi[buf][arow + 32 * s]);
        const v4i al = *reinterpret_cast<const v4i *>(&L.a_lo[buf][arow + 32 * s]);
        const v4i b0 = *reinterpret_cast<const v4i *>(&L.w0[buf][brow + 32 * s]);
        if (SEG32) {  // every sub-step is a segment: the products start from zero
            c.c0 = c.c1 = c.c2 = c.c3 = (v16i){};
            c.wacc = 0;
        }
        if (BITS == 4) {
            c.c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, b0, c.c0, 0, 0, 0);
            c.c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, b0, c.c1, 0, 0, 0);
        } else {
            const v4i b1 = *reinterpret_cast<const v4i *>(&L.w1[buf][brow + 32 * s]);
            c.c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, b1, c.c0, 0, 0, 0);
            c.c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, b0, c.c1, 0, 0, 0);
            c.c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, b1, c.c2, 0, 0, 0);
            c.c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(al, b0, c.c3, 0, 0, 0);
        }
        c.wacc += L.wsum[buf][s][orow];
        if (SEG32 || (kb * KB + 32 * (s + 1)) % seg == 0) {  // end of a segment: tile_i16's flush
            const float sc = L.scale[buf][s][orow];
            const int w128 = 128 * c.wacc;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                int G;
                if (BITS == 4)
                    G = (c.c0[i] << 8) + c.c1[i] + w128;
                else
                    G = (((c.c0[i] << 4) + c.c1[i]) << 8) + ((c.c2[i] << 4) + c.c3[i]) + w128;
                c.acc[i] = fmaf((float)G, sc, c.acc[i]);
            }
            if (!SEG32) {
                c.c0 = c.c1 = c.c2 = c.c3 = (v16i){};
                c.wacc = 0;
            }
        }
    }
}

template <int BITS, int NS, bool SEG32>
__global__ __launch_bounds__(256) void gemm_i8_kernel(MfArgs a) {
    using LT = Lds<BITS, NS>;
    constexpr int KB = LT::KB, RS = LT::RS;
    extern __shared__ __align__(16) uint8_t smem_gemm[];
    LT &L = *reinterpret_cast<LT *>(smem_gemm);
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid & 1, wn = wid >> 1;
    const int tile0 = blockIdx.x * (TN / 16), out0 = blockIdx.x * TN, tok0 = blockIdx.y * TM;
    const auto rx = make_rsrc(a.xq, a.xq_bytes);
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rs = make_rsrc(a.scales, a.scales_bytes);
    const auto rz = make_rsrc(a.zps, a.zps_bytes);
    if (tid < TM) L.sx[tid] = tok0 + tid < a.T ? a.sx[tok0 + tid] : 0.0f;

    const int nkb = a.K / KB;
    // Two register sets of prefetched blocks: block kb + 1 is loaded while
    // block kb - 1 is computed, so a load has two blocks of work to arrive.
    Pref<BITS> pa[NS], pb[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) prefetch<BITS>(a, j, tok0, tile0, pa[j], rx, rc, rs, rz);
    if (nkb > 1) {
#pragma unroll
        for (int j = 0; j < NS; j++) prefetch<BITS>(a, NS + j, tok0, tile0, pb[j], rx, rc, rs, rz);
    }
#pragma unroll
    for (int j = 0; j < NS; j++) stage<BITS, NS>(pa[j], L, 0, j);
    lds_barrier();

    Acc<BITS> c;
    const int arow = (32 * wm + (lane & 31)) * RS + 16 * (lane >> 5);
    const int brow = (32 * wn + (lane & 31)) * RS + 16 * (lane >> 5);
    const int orow = 32 * wn + (lane & 31);

    for (int kb = 0; kb < nkb; kb += 2) {
        // even block kb in buffer 0; pa is free, pb holds block kb + 1
        if (kb + 2 < nkb) {
#pragma unroll
            for (int j = 0; j < NS; j++) prefetch<BITS>(a, (kb + 2) * NS + j, tok0, tile0, pa[j], rx, rc, rs, rz);
        }
        compute_block<BITS, NS, SEG32>(L, 0, kb, arow, brow, orow, a.seg, c);
        if (kb + 1 < nkb) {
#pragma unroll
            for (int j = 0; j < NS; j++) stage<BITS, NS>(pb[j], L, 1, j);
        }
        lds_barrier();
        if (kb + 1 >= nkb) break;
        // odd block kb + 1 in buffer 1; pb is free, pa holds block kb + 2
        if (kb + 3 < nkb) {
#pragma unroll
            for (int j = 0; j < NS; j++) prefetch<BITS>(a, (kb + 3) * NS + j, tok0, tile0, pb[j], rx, rc, rs, rz);
        }
        compute_block<BITS, NS, SEG32>(L, 1, kb + 1, arow, brow, orow, a.seg, c);
        if (kb + 2 < nkb) {
#pragma unroll
            for (int j = 0; j < NS; j++) stage<BITS, NS>(pa[j], L, 0, j);
        }
        lds_barrier();
    }
    const float *acc = c.acc;

    // Epilogue: lane holds output row out0 + orow for 16 tokens.
    const int o = out0 + orow;
    if (o >= a.n) return;
    const float bo = (a.flags & LLMQ_BIAS) ? a.bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int ml = 32 * wm + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        const int tok = tok0 + ml;
        if (tok >= a.T) continue;
        float v = acc[i] * L.sx[ml];
        if (a.flags & LLMQ_BIAS) v += bo;
        if (a.flags & LLMQ_GELU) v = gelu_f(v);
        float *dst = a.out + (int64_t)tok * a.ldo + o;
        if (a.flags & LLMQ_RESID) v += *dst;
        *dst = v;
    }
}

template <int BITS, int NS, bool SEG32>
int launch_ns(llmq_ctx *ctx, const MfArgs &a, dim3 grid) {
    const size_t lds = sizeof(Lds<BITS, NS>);
    static bool attr = false;
    if (!attr) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_i8_kernel<BITS, NS, SEG32>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr = true;
    }
    hipLaunchKernelGGL((gemm_i8_kernel<BITS, NS, SEG32>), grid, dim3(256), lds, ctx->stream, a);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

template <int BITS, bool SEG32>
int launch_bits(llmq_ctx *ctx, const MfArgs &a, dim3 grid, int ns) {
    if (ns == 2) return launch_ns<BITS, 2, SEG32>(ctx, a, grid);
    return launch_ns<BITS, 1, SEG32>(ctx, a, grid);
}

}  // namespace

bool gemm_mfma_supports(const llmq_mat *w, int64_t T) {
    if (w->kind != MAT_QUANT || T < 2) return false;
    const int64_t seg = w->group < 256 ? w->group : 256;
    return w->k % KB0 == 0 && w->k % seg == 0 && w->group % 32 == 0 &&
           (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256 < (int64_t)kOOB && T * w->k * 2 < (int64_t)kOOB;
}

int launch_gemm_mfma(llmq_ctx *ctx, const GemvRequest &rq, int16_t *xq, float *sx) {
    const llmq_mat *w = rq.w;
    const int64_t T = rq.T, K = w->k;
    const int64_t ldx = rq.ldx ? rq.ldx : K;
    LLMQ_REQUIRE(gemm_mfma_supports(w, T), "linear: no MFMA GEMM for this matrix");
    const int upt = (int)((K / 4 + 255) / 256);
    const bool ln = rq.ln_w != nullptr;
#define ACTQ(L, U) hipLaunchKernelGGL((act_q16_kernel<L, U>), dim3((unsigned)T), dim3(256), 0, ctx->stream, rq.x, ldx, \
                                       rq.ln_w, rq.ln_b, (int)K, xq, sx)
    if (upt <= 1) {
        if (ln) ACTQ(true, 1); else ACTQ(false, 1);
    } else if (upt <= 4) {
        if (ln) ACTQ(true, 4); else ACTQ(false, 4);
    } else if (upt <= 12) {
        if (ln) ACTQ(true, 12); else ACTQ(false, 12);
    } else {
        return llmq_set_error(LLMQ_EUNSUPPORTED, "linear: reduction axis %lld too long", (long long)K);
    }
#undef ACTQ
    LLMQ_HIP(hipGetLastError());
    MfArgs a;
    a.xq = xq;
    a.sx = sx;
    a.codes = w->codes;
    a.scales = w->scales;
    a.zps = w->zps;
    a.bias = rq.bias ? rq.bias : rq.out;
    a.out = rq.out;
    a.ldo = rq.ldo ? rq.ldo : w->n;
    a.xq_bytes = (uint32_t)(T * K * 2);
    a.codes_bytes = (uint32_t)((w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256);
    a.scales_bytes = (uint32_t)((w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS * 2);
    a.zps_bytes = (uint32_t)((w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS);
    a.T = (int)T;
    a.K = (int)K;
    a.n = (int)w->n;
    a.ntiles = (int)w->ntiles;
    a.CK = (int)w->CK;
    a.NG = (int)w->NG;
    a.G = (int)w->group;
    a.seg = (int)(w->group < 256 ? w->group : 256);
    a.flags = rq.flags;
    dim3 grid((unsigned)((w->n + TN - 1) / TN), (unsigned)((T + TM - 1) / TM));
    // staged block: int4 2 sub-blocks of 64 inputs (1 when K is an odd
    // multiple of 64), int8 1 (its registers): two workgroups fit a CU
    const int nsb = (int)(K / KB0);
    int ns = w->bits == 4 && nsb % 2 == 0 ? 2 : 1;
    if (const char *e = getenv("LLMQ_GEMM_NS")) {
        const int v = atoi(e);
        if ((v == 1 || v == 2) && nsb % v == 0) ns = v;
    }
    const bool seg32 = a.seg == 32;
    if (w->bits == 4) return seg32 ? launch_bits<4, true>(ctx, a, grid, ns) : launch_bits<4, false>(ctx, a, grid, ns);
    return seg32 ? launch_bits<8, true>(ctx, a, grid, ns) : launch_bits<8, false>(ctx, a, grid, ns);
}
