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
// Mapping: a workgroup of 4 waves owns 16 MT tokens x 64 output rows (4 row
// tiles); wave w computes rows 16 w .. 16 w + 15 for all 16 MT tokens with
// v_mfma_i32_16x16x32_i8 (A: 16 tokens x 32 inputs of one plane, B: 32
// inputs x 16 rows), the wave's weight fragment serving its MT token
// groups.  One call covers exactly one 32-input group, so the group sums
// tile_i16 scales (int4-g32: every call) come straight out of the
// accumulators; the 16x16x64 form would add two groups' products together
// before they can be scaled.  The reduction axis is walked in staged blocks
// of 128 inputs: activations, codes, zero points and scales of block kb + 2
// are loaded into registers while block kb, staged in LDS (activation
// planes, weights as int8 rows, per-row weight sums, scales), feeds the
// matrix cores; two LDS buffers alternate, one barrier per block.
//
// What bounds it: tile_i16's per-group float chain, per output and group
// of 32 inputs a shift-add, a convert and an fma (3 VALU against 2 MFMA of
// 8192 products per 16 x 16 outputs; the 128 * sum w term starts the low
// plane's accumulator), issued by two workgroups of four waves a CU: each
// staged block takes ~1 us per workgroup at 476 tokens against ~0.35 us of
// instructions (per-workgroup timestamps), and prefetching four blocks
// ahead instead of two does not shorten it.
//
// int4 weights in groups of 32 take gemm_f16_kernel instead (below): the
// same G on the fp16 matrix cores, exact in their fp32 sums, so the flush is
// one fma per output and group.
//
// Activations come from act_q16_kernel: LayerNorm (kernels.mojo:179-197) when
// asked, then quantize_rows (kernels.mojo:400-416), one workgroup per token.
#include "common.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int TN = 64;           // output rows per workgroup (a 16 x 16 block per wave)
constexpr int KB = 128;          // inputs per staged block
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

// The fp16 planes of int16 codes q (gemm_f16_kernel's A operand): q =
// 256 hi + lo with hi = q >> 8 and lo = q & 255, as fp16 values 256 hi and
// lo (both exact).  Layout for T tokens (padded to T16) and CK chunks of 32
// inputs, the 16 tokens of a token tile side by side so that a wave's
// operand load is 1 KB in one piece:
//     fp16 [T16 / 16][CK][hi, lo][4 groups][16 tokens][8]
// group g holding inputs 8 g .. 8 g + 7 of the chunk in the order 0, 2, 4,
// 6, 1, 3, 5, 7 (the order in which a code dword's nibbles decode).
__device__ __forceinline__ uint32_t f16_pair(int a, int b) {
    const _Float16 ha = (_Float16)(float)a, hb = (_Float16)(float)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}
// Unit u (inputs 4 u .. 4 u + 3) of token t, held by a lane whose
// neighbour (lane ^ 1) holds unit u ^ 1, the other half of the same group of
// 8 inputs: the pair swaps codes, then the even lane stores the group's 16
// bytes of the hi plane and the odd lane those of the lo plane.  Both lanes
// of a pair call this together (K is a multiple of 32).
__device__ __forceinline__ void store_planes(uint8_t *planes, int CK, int t, int u, int q0, int q1, int q2, int q3) {
    const int c = u >> 3, g = (u & 7) >> 1, h = u & 1;
    const int p0 = __shfl_xor(q0, 1), p1 = __shfl_xor(q1, 1), p2 = __shfl_xor(q2, 1), p3 = __shfl_xor(q3, 1);
    // inputs 0..7 of the group
    const int e0 = h ? p0 : q0, e1 = h ? p1 : q1, e2 = h ? p2 : q2, e3 = h ? p3 : q3;
    const int e4 = h ? q0 : p0, e5 = h ? q1 : p1, e6 = h ? q2 : p2, e7 = h ? q3 : p3;
    const int m = h ? 255 : ~255;  // lo plane (q & 255) from the odd lane, hi (q & ~255) from the even one
    uint4 v;
    v.x = f16_pair(e0 & m, e2 & m);  // slots 0 1: inputs 0 2
    v.y = f16_pair(e4 & m, e6 & m);  // slots 2 3: inputs 4 6
    v.z = f16_pair(e1 & m, e3 & m);  // slots 4 5: inputs 1 3
    v.w = f16_pair(e5 & m, e7 & m);  // slots 6 7: inputs 5 7
    *reinterpret_cast<uint4 *>(planes + ((int64_t)(t >> 4) * CK + c) * 2048 + h * 1024 + (g * 16 + (t & 15)) * 16) = v;
}

// One workgroup (256 threads) per token row: optional LayerNorm, then
// quantize_rows.  Values are held in registers, 4 per unit of a float4.
// With `planes` set, the codes are also written there as fp16 planes.
template <bool LN, int UPT>
__global__ __launch_bounds__(256) void act_q16_kernel(const float *__restrict__ x, int64_t ldx,
                                                      const float *__restrict__ lw, const float *__restrict__ lb,
                                                      int K, int16_t *__restrict__ xq, float *__restrict__ sx,
                                                      uint8_t *__restrict__ planes) {
    __shared__ float red[4], bc[2];
    extern __shared__ __align__(16) float xs[];  // [K] with LayerNorm
    const int t = blockIdx.x, tid = threadIdx.x, nunits = K / 4;
    const float4 *xr = reinterpret_cast<const float4 *>(x + (int64_t)t * ldx);
    float4 v[UPT];
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + 256 * i;
        v[i] = u < nunits ? xr[u] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if (LN) {
        // the statistics in layernorm's own order (16 lane partials)
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const int u = tid + 256 * i;
            if (u < nunits) reinterpret_cast<float4 *>(xs)[u] = v[i];
        }
        llmq_lds_barrier();
        float mean, rstd;
        llmq_ln_stats(xs, K, bc, mean, rstd);
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
        if (planes)  // from the stored int16 codes
            store_planes(planes, K / 32, t, u, (int16_t)q0, (int16_t)q1, (int16_t)q2, (int16_t)q3);
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

// Registers of one staged block (KB = 128 inputs), loaded ahead of its use.
// Thread t: activations of token t / 16, inputs 8 (t % 16) .. +7; int4
// codes of (tile t / 64, 32-input chunk (t / 16) % 4, row t % 16); int8
// codes of the same rows' two 16-input chunks of sub-step (t / 16) % 4; the
// scale of (sub-step t / 64, row t % 64).  Zero point and scale come as
// the aligned dwords holding them plus bit offsets, extracted where they are
// used, so no wait follows the loads.
template <int MT>
struct Pref {
    uint4 a[MT];    // 8 int16 activations of tokens t / 16 + 16 j
    uint4 c0, c1;   // int4: one chunk (c0); int8: two chunks
    uint32_t zpw, zsh, scw, ssh;
};

template <int BITS, int MT>
struct Lds {
    static constexpr int RS = KB + 16;   // row stride in bytes
    uint8_t a_hi[2][16 * MT * RS];
    uint8_t a_lo[2][16 * MT * RS];
    uint8_t w0[2][TN * RS];              // int4: u - zp; int8: wl = w & 15
    uint8_t w1[2][BITS == 8 ? TN * RS : 16];  // int8: wh = w >> 4
    int wsum[2][KB / 32][TN];            // sum of w per (32-input sub-step, row)
    float scale[2][KB / 32][TN];         // scale of the group of each (sub-step, row)
    float sx[16 * MT];
};

// Loads of block kb (inputs 128 kb ..); everything at or past K reads zeros.
template <int BITS, int MT>
__device__ __forceinline__ void prefetch(const MfArgs &a, int kb, int tok0, int tile0, Pref<MT> &p,
                                         __amdgpu_buffer_rsrc_t rx, __amdgpu_buffer_rsrc_t rc,
                                         __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rz) {
    const int t = threadIdx.x, k0 = kb * KB;
#pragma unroll
    for (int j = 0; j < MT; j++) {
        const int m = (t >> 4) + 16 * j, k = k0 + 8 * (t & 15);
        const int tok = tok0 + m;
        const uint32_t off = tok < a.T && k < a.K ? (uint32_t)(((int64_t)tok * a.K + k) * 2) : kOOB;
        p.a[j] = bload16(rx, off);
    }
    const int tt = t >> 6, sub = (t >> 4) & 3, r = t & 15;
    const int tile = tile0 + tt, ks = k0 + 32 * sub;  // this thread's 32-input sub-step
    const bool ok = tile < a.ntiles && ks < a.K;
    if (BITS == 4) {
        const uint32_t coff = (uint32_t)((((int64_t)tile * a.CK + ks / 32) * 16 + r) * 16);
        p.c0 = bload16(rc, ok ? coff : kOOB);
    } else {
        const uint32_t coff = (uint32_t)((((int64_t)tile * a.CK + ks / 16) * 16 + r) * 16);
        p.c0 = bload16(rc, ok ? coff : kOOB);
        p.c1 = bload16(rc, ok ? coff + 256u : kOOB);  // next chunk, same row
    }
    const uint32_t zoff = ok ? (uint32_t)(((int64_t)tile * a.NG + ks / a.G) * 16 + r) : kOOB;
    p.zpw = bload4(rz, zoff == kOOB ? kOOB : (zoff & ~3u));
    p.zsh = 8u * (zoff & 3u);
    {
        const int s = t >> 6, o = t & 63;
        const int tl = tile0 + (o >> 4), kss = k0 + 32 * s;
        const bool sok = tl < a.ntiles && kss < a.K;
        const uint32_t soff = sok ? (uint32_t)((((int64_t)tl * a.NG + kss / a.G) * 16 + (o & 15)) * 2) : kOOB;
        p.scw = bload4(rs, soff == kOOB ? kOOB : (soff & ~3u));
        p.ssh = 8u * (soff & 2u);
    }
}

// int8 weights w (u - zp, 9 bits) of 16 codes as low nibbles wl and high
// parts wh (w = 16 wh + wl); returns sum w.
__device__ __forceinline__ int split_w8(uint4 code, uint32_t zp, uint32_t (&wl)[4], uint32_t (&wh)[4]) {
    const v2s zz = {(short)zp, (short)zp};
    const uint32_t dd[4] = {code.x, code.y, code.z, code.w};
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
    return s;
}

// Block p into LDS buffer buf.
template <int BITS, int MT>
__device__ __forceinline__ void stage(const Pref<MT> &p, Lds<BITS, MT> &L, int buf) {
    constexpr int RS = Lds<BITS, MT>::RS;
    const int t = threadIdx.x;
    const uint32_t zp = (p.zpw >> p.zsh) & 255u;
#pragma unroll
    for (int j = 0; j < MT; j++) {  // activation planes: hi bytes and (lo - 128) bytes, natural input order
        const int m = (t >> 4) + 16 * j, col = 8 * (t & 15);
        const uint32_t hi0 = __builtin_amdgcn_perm(p.a[j].y, p.a[j].x, 0x07050301u);
        const uint32_t hi1 = __builtin_amdgcn_perm(p.a[j].w, p.a[j].z, 0x07050301u);
        const uint32_t lo0 = __builtin_amdgcn_perm(p.a[j].y, p.a[j].x, 0x06040200u) ^ 0x80808080u;
        const uint32_t lo1 = __builtin_amdgcn_perm(p.a[j].w, p.a[j].z, 0x06040200u) ^ 0x80808080u;
        *reinterpret_cast<uint2 *>(&L.a_hi[buf][m * RS + col]) = make_uint2(hi0, hi1);
        *reinterpret_cast<uint2 *>(&L.a_lo[buf][m * RS + col]) = make_uint2(lo0, lo1);
    }
    const int tt = t >> 6, sub = (t >> 4) & 3, r = t & 15;
    const int o = tt * 16 + r;
    if (BITS == 4) {
        const uint32_t zb = zp * 0x01010101u;
        const uint32_t dd[4] = {p.c0.x, p.c0.y, p.c0.z, p.c0.w};
        uint32_t w[8];
        int s = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = dd[i] & 0x0F0F0F0Fu, hi = (dd[i] >> 4) & 0x0F0F0F0Fu;
            const uint32_t n0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // weights 8i+0..3
            const uint32_t n1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // weights 8i+4..7
            w[2 * i] = ((n0 | 0x80808080u) - zb) ^ 0x80808080u;               // u - zp as int8
            w[2 * i + 1] = ((n1 | 0x80808080u) - zb) ^ 0x80808080u;
            s = __builtin_amdgcn_sdot4((int)w[2 * i], 0x01010101, s, false);
            s = __builtin_amdgcn_sdot4((int)w[2 * i + 1], 0x01010101, s, false);
        }
        uint8_t *dst = &L.w0[buf][o * RS + 32 * sub];
        *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
        *reinterpret_cast<uint4 *>(dst + 16) = make_uint4(w[4], w[5], w[6], w[7]);
        L.wsum[buf][sub][o] = s;
    } else {
        uint32_t wl[4], wh[4], wl1[4], wh1[4];
        const int s = split_w8(p.c0, zp, wl, wh) + split_w8(p.c1, zp, wl1, wh1);
        uint8_t *d0 = &L.w0[buf][o * RS + 32 * sub];
        uint8_t *d1 = &L.w1[buf][o * RS + 32 * sub];
        *reinterpret_cast<uint4 *>(d0) = make_uint4(wl[0], wl[1], wl[2], wl[3]);
        *reinterpret_cast<uint4 *>(d0 + 16) = make_uint4(wl1[0], wl1[1], wl1[2], wl1[3]);
        *reinterpret_cast<uint4 *>(d1) = make_uint4(wh[0], wh[1], wh[2], wh[3]);
        *reinterpret_cast<uint4 *>(d1 + 16) = make_uint4(wh1[0], wh1[1], wh1[2], wh1[3]);
        L.wsum[buf][sub][o] = s;
    }
    L.scale[buf][t >> 6][t & 63] = __half2float(__ushort_as_half((unsigned short)((p.scw >> p.ssh) & 0xFFFFu)));
}

// Accumulators of one wave: the matrix-core partial sums of the current
// segment (int4: hi, lo planes; int8: hh, hl, lh, ll), the weight sum of the
// segment, and the float outputs (4 tokens of one row per lane).
template <int MT>
struct Acc {
    v4i c0[MT] = {}, c1[MT] = {}, c2[MT] = {}, c3[MT] = {};
    int wacc = 0;
    float acc[MT][4] = {};
};

__device__ __forceinline__ v4i mfma16(int64_t a, int64_t b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}

// The 4 sub-steps of 32 inputs of staged block kb (in LDS buffer buf): per
// sub-step the wave's weight fragment serves its MT token groups.
template <int BITS, bool SEG32, int MT>
__device__ __forceinline__ void compute_block(const Lds<BITS, MT> &L, int buf, int kb, int arow, int brow, int orow,
                                              int seg, Acc<MT> &c) {
    constexpr int RS = Lds<BITS, MT>::RS;
#pragma unroll
    for (int s = 0; s < KB / 32; s++) {
        const int64_t b0 = *reinterpret_cast<const int64_t *>(&L.w0[buf][brow + 32 * s]);
        int64_t b1 = 0;
        if (BITS == 8) b1 = *reinterpret_cast<const int64_t *>(&L.w1[buf][brow + 32 * s]);
        if (SEG32) {  // every sub-step is a segment: the products start from zero, the
                      // lowest-weight accumulator from the 128 * sum w term
            const int w128 = 128 * L.wsum[buf][s][orow];
            const v4i wv = {w128, w128, w128, w128};
#pragma unroll
            for (int j = 0; j < MT; j++) {
                c.c0[j] = c.c2[j] = (v4i){};
                c.c1[j] = BITS == 4 ? wv : (v4i){};
                c.c3[j] = BITS == 8 ? wv : (v4i){};
            }
        }
#pragma unroll
        for (int j = 0; j < MT; j++) {
            const int64_t ah = *reinterpret_cast<const int64_t *>(&L.a_hi[buf][arow + 16 * j * RS + 32 * s]);
            const int64_t al = *reinterpret_cast<const int64_t *>(&L.a_lo[buf][arow + 16 * j * RS + 32 * s]);
            if (BITS == 4) {
                c.c0[j] = mfma16(ah, b0, c.c0[j]);
                c.c1[j] = mfma16(al, b0, c.c1[j]);
            } else {
                c.c0[j] = mfma16(ah, b1, c.c0[j]);
                c.c1[j] = mfma16(ah, b0, c.c1[j]);
                c.c2[j] = mfma16(al, b1, c.c2[j]);
                c.c3[j] = mfma16(al, b0, c.c3[j]);
            }
        }
        if (!SEG32) c.wacc += L.wsum[buf][s][orow];
        if (SEG32 || (kb * KB + 32 * (s + 1)) % seg == 0) {  // end of a segment: tile_i16's flush
            const float sc = L.scale[buf][s][orow];
            const int w128 = SEG32 ? 0 : 128 * c.wacc;  // (SEG32: already in the accumulators)
#pragma unroll
            for (int j = 0; j < MT; j++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    int G;
                    if (BITS == 4)
                        G = (c.c0[j][i] << 8) + c.c1[j][i] + w128;
                    else
                        G = (((c.c0[j][i] << 4) + c.c1[j][i]) << 8) + ((c.c2[j][i] << 4) + c.c3[j][i]) + w128;
                    c.acc[j][i] = fmaf((float)G, sc, c.acc[j][i]);
                }
            }
            if (!SEG32) {
#pragma unroll
                for (int j = 0; j < MT; j++) c.c0[j] = c.c1[j] = c.c2[j] = c.c3[j] = (v4i){};
                c.wacc = 0;
            }
        }
    }
}

template <int BITS, bool SEG32, int MT>
__global__ __launch_bounds__(256) void gemm_i8_kernel(MfArgs a) {
    using LT = Lds<BITS, MT>;
    constexpr int RS = LT::RS, TMW = 16 * MT;  // tokens of the workgroup
    __shared__ __align__(16) LT L;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int tile0 = blockIdx.x * (TN / 16), out0 = blockIdx.x * TN, tok0 = blockIdx.y * TMW;
    const auto rx = make_rsrc(a.xq, a.xq_bytes);
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rs = make_rsrc(a.scales, a.scales_bytes);
    const auto rz = make_rsrc(a.zps, a.zps_bytes);
    if (tid < TMW) L.sx[tid] = tok0 + tid < a.T ? a.sx[tok0 + tid] : 0.0f;

    const int nkb = (a.K + KB - 1) / KB;
    // Two register sets of prefetched blocks: block kb + 1 is loaded while
    // block kb - 1 is computed, so a load has two blocks of work to arrive.
    Pref<MT> pa, pb;
    prefetch<BITS, MT>(a, 0, tok0, tile0, pa, rx, rc, rs, rz);
    if (nkb > 1) prefetch<BITS, MT>(a, 1, tok0, tile0, pb, rx, rc, rs, rz);
    stage<BITS, MT>(pa, L, 0);
    lds_barrier();

    Acc<MT> c;
    // A: token 16 j + lane % 16, inputs 8 (lane / 16) ..; B: row 16 wid + lane % 16
    const int arow = (lane & 15) * RS + 8 * (lane >> 4);
    const int brow = (16 * wid + (lane & 15)) * RS + 8 * (lane >> 4);
    const int orow = 16 * wid + (lane & 15);

    for (int kb = 0; kb < nkb; kb += 2) {
        // even block kb in buffer 0; pa is free, pb holds block kb + 1
        if (kb + 2 < nkb) prefetch<BITS, MT>(a, kb + 2, tok0, tile0, pa, rx, rc, rs, rz);
        compute_block<BITS, SEG32, MT>(L, 0, kb, arow, brow, orow, a.seg, c);
        if (kb + 1 < nkb) stage<BITS, MT>(pb, L, 1);
        lds_barrier();
        if (kb + 1 >= nkb) break;
        // odd block kb + 1 in buffer 1; pb is free, pa holds block kb + 2
        if (kb + 3 < nkb) prefetch<BITS, MT>(a, kb + 3, tok0, tile0, pb, rx, rc, rs, rz);
        compute_block<BITS, SEG32, MT>(L, 1, kb + 1, arow, brow, orow, a.seg, c);
        if (kb + 2 < nkb) stage<BITS, MT>(pa, L, 0);
        lds_barrier();
    }

    // Epilogue: lane holds output row out0 + orow for tokens 16 j + 4 (lane / 16) + i.
    const int o = out0 + orow;
    if (o >= a.n) return;
    const float bo = (a.flags & LLMQ_BIAS) ? a.bias[o] : 0.0f;
#pragma unroll
    for (int j = 0; j < MT; j++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int ml = 16 * j + 4 * (lane >> 4) + i;
            const int tok = tok0 + ml;
            if (tok >= a.T) continue;
            float v = c.acc[j][i] * L.sx[ml];
            if (a.flags & LLMQ_BIAS) v += bo;
            if (a.flags & LLMQ_GELU) v = gelu_ref(v);
            float *dst = a.out + (int64_t)tok * a.ldo + o;
            if (a.flags & LLMQ_RESID) v += *dst;
            *dst = v;
        }
    }
}

// rows_i16 (kernels.mojo:576-614): the last n % 32 output rows, which the
// reference leaves out of its 32-row tiles (matmul_rows_a16, 468-476) and
// dots one at a time: per (row, token) 16 lanes in dot1_i16's order, the
// 16-lane halving sum, times sx, plus bias, then finish (GELU, residual).
// Four (row, token) items a wave; item i is row o0 + i % nrows, token
// i / nrows.
__global__ __launch_bounds__(64) void rows_i16_kernel(MfArgs a, int bits, int o0, int nrows) {
    const int L = threadIdx.x & 15;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 4);
    const bool live = item < (int64_t)nrows * a.T;
    const int o = o0 + (live ? (int)(item % nrows) : 0), tok = live ? (int)(item / nrows) : 0;
    float d = llmq_dot1_lane(a.codes, a.scales, a.zps, bits, a.K, a.G, a.CK, a.NG, o, a.xq + (int64_t)tok * a.K, L);
    d = llmq_reduce16(d);
    if (!live || L != 0) return;
    float v = d * a.sx[tok];
    if (a.flags & LLMQ_BIAS) v += a.bias[o];
    if (a.flags & LLMQ_GELU) v = gelu_ref(v);
    float *dst = a.out + (int64_t)tok * a.ldo + o;
    if (a.flags & LLMQ_RESID) v += *dst;
    *dst = v;
}

// ------------------------------------------------------- int4-g32 on fp16
//
// tile_i16 for int4 weights in groups of 32 (a segment is a group): per
// token t, output row o and group g,
//     G = sum_{k in g} q[t, k] (u[o, k] - zp[o, g]),   acc = fma(float(G), scale[o, g], acc)
// with q = 256 hi + lo from the fp16 planes and w = u - zp (|w| <= 15)
// decoded to fp16, the matrix cores (v_mfma_f32_16x16x32_f16, fp32 sums)
// form sum (256 hi) w + sum lo w.  Every product is an integer of magnitude
// <= 32768 * 15, and every partial sum is bounded by 32 * (32768 + 255) * 15
// < 2^24, so each intermediate value is exact and the result is G itself:
// the float the reference converts G to (exactly, as |G| < 2^24).  The
// flush is then one fma per output and group.
//
// Mapping: a workgroup of NW waves owns MT token tiles of 16 tokens and
// NW NR row tiles of 16 rows (wave w: row tiles w NR ..) and walks the K / 32
// groups in steps of S.  Per step it copies, with the global-to-LDS loads
// (16 bytes a lane), the token tiles' planes (MT S 2 KB), the row tiles'
// code blocks (NW NR S 256 B), zero points and scales into one of two LDS
// buffers while the waves compute the previous step from the other: one
// barrier a step.  Per group lane l of a wave reads, for each token tile, 16
// bytes of each plane (token l % 16, inputs 8 (l / 16) ..) and, for each row
// tile, the code dword of row l % 16 and inputs 8 (l / 16) .. with that
// row's zero point and scale; it then holds outputs (tokens 4 (l / 16) + i,
// row l % 16).  Workgroups go to the XCDs in an order that keeps the ones
// sharing a token block's planes on one XCD.  At 476 tokens this runs the
// GPT-2 layer GEMMs in 12-13 us (qkv, fc, proj, fcproj), against 15-19 us for
// the int8-MFMA form: the planes are read once a workgroup instead of once a
// wave (a form loading them per wave took 15-18 us), and register-staged
// copies measured slower than the global-to-LDS ones.
struct F16Args {
    const uint8_t *planes, *codes, *zps;
    const uint16_t *scales;
    const float *sx, *bias;
    float *out;
    int64_t ldo;
    int T, n, ntiles, CK, flags;
    int xcd;  // XCD-aware workgroup order
    // KV: QuantKV.store of the key / value rows (a workgroup's 64 rows are
    // one head's q, k or v: rows 64 b of the qkv matrix, b = part * heads + head)
    int8_t *k8, *v8;
    float *ks, *vs;
    int kv_layer, kv_pos0, kv_max_t, kv_heads;
};

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// 1024 + the 8 bytes of (a, b) as fp16 pairs (a0, a1), (a2, a3), (b0, b1),
// (b2, b3): 0x6400 | n is 1024 + n in fp16 for n < 1024.
__device__ __forceinline__ void bytes_f16(uint32_t a, uint32_t b, uint32_t (&d)[4]) {
    d[0] = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
    d[1] = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
    d[2] = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
    d[3] = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
}

// Bytes of one staged step (CPG code chunks of 16 bytes a row and group:
// 1 for int4, 2 for int8).
template <int MT, int NR, int S, int NW, int CPG>
struct F16Lds {
    static constexpr int A = MT * S * 2048, C = NW * NR * S * 256 * CPG, Z = NW * NR * S * 16, SC = NW * NR * S * 32;
    static constexpr int BYTES = A + C + Z + SC;
};

template <int MT, int NR, int S, int NW, int BITS, bool KV>
__global__ __launch_bounds__(NW * 64) void gemm_f16_kernel(F16Args a) {
    static_assert(!KV || (MT == 1 && NR == 1 && NW == 4), "the cache store takes 64-row workgroups");
    constexpr int CPG = BITS / 4;  // code chunks a group of 32
    using LY = F16Lds<MT, NR, S, NW, CPG>;
    constexpr int RB = NW * 1024;  // bytes a copy round: 16 a lane
    // separate arrays, so that the compiler sees a copy into one cannot alias reads of the other
    __shared__ __align__(16) uint8_t b0[LY::BYTES], b1[LY::BYTES];
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c16 = lane & 15, g = lane >> 4;
    // Workgroups go to the 8 XCDs in turn (linear id mod 8); each XCD gets
    // a contiguous run of (token block, row block) pairs in token-block
    // order, so that the workgroups sharing a token block's planes share an
    // L2.
    int bx = blockIdx.x, by = blockIdx.y;
    if (a.xcd) {
        const int nb = gridDim.x * gridDim.y, L = blockIdx.y * gridDim.x + blockIdx.x;
        const int x = L & 7, q = nb >> 3, rem = nb & 7;
        const int pos = x * q + min(x, rem) + (L >> 3);
        bx = pos % gridDim.x;
        by = pos / gridDim.x;
    }
    const int rt0 = bx * NW * NR, tt0 = by * MT, ttiles = (a.T + 15) >> 4;
    const int tile0 = rt0 + w * NR;  // this wave's row tiles
    const int NG = a.CK / CPG;       // groups of 32: one scale and zero point each; the planes' chunks
    // Copy of step s (groups s S ..) into buf, region by region: lane i of
    // wave w brings the 16 bytes at offset q RB + 1024 w + 16 i of the
    // region (the global-to-LDS load writes a wave's 64 x 16 bytes to
    // consecutive LDS).  A token tile past the planes or a row tile past the
    // matrix copies tile 0 instead (its outputs are not stored).
    auto stage = [&](int s, uint8_t *buf) {
        const int c0 = s * S;
#pragma unroll
        for (int q = 0; q < (LY::A + RB - 1) / RB; q++) {
            const int x = q * RB + tid * 16;
            if (x < LY::A) {
                const int j = x / (S * 2048), tt = tt0 + j < ttiles ? tt0 + j : 0;
                __builtin_amdgcn_global_load_lds(a.planes + ((int64_t)tt * NG + c0) * 2048 + x % (S * 2048),
                                                 (__attribute__((address_space(3))) void *)(buf + q * RB + w * 1024), 16, 0, 0);
            }
        }
#pragma unroll
        for (int q = 0; q < (LY::C + RB - 1) / RB; q++) {
            const int x = q * RB + tid * 16;
            if (x < LY::C) {
                const int r = x / (S * 256 * CPG), tile = rt0 + r < a.ntiles ? rt0 + r : 0;
                __builtin_amdgcn_global_load_lds(a.codes + ((int64_t)tile * a.CK + c0 * CPG) * 256 + x % (S * 256 * CPG),
                                                 (__attribute__((address_space(3))) void *)(buf + LY::A + q * RB + w * 1024), 16, 0,
                                                 0);
            }
        }
#pragma unroll
        for (int q = 0; q < (LY::Z + LY::SC + RB - 1) / RB; q++) {  // zero points, then scales
            const int x = q * RB + tid * 16;
            if (x < LY::Z + LY::SC) {
                const uint8_t *src;
                if (x < LY::Z) {
                    const int r = x / (S * 16), tile = rt0 + r < a.ntiles ? rt0 + r : 0;
                    src = a.zps + ((int64_t)tile * NG + c0) * 16 + x % (S * 16);
                } else {
                    const int y = x - LY::Z, r = y / (S * 32), tile = rt0 + r < a.ntiles ? rt0 + r : 0;
                    src = reinterpret_cast<const uint8_t *>(a.scales) + ((int64_t)tile * NG + c0) * 32 + y % (S * 32);
                }
                __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(buf + LY::A + LY::C + q * RB + w * 1024),
                                                 16, 0, 0);
            }
        }
    };
    // the epilogue's token scales and biases, loaded first
    float sxr[MT][4], bor[NR];
#pragma unroll
    for (int j = 0; j < MT; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tok = (tt0 + j) * 16 + 4 * g + i;
            sxr[j][i] = tok < a.T ? a.sx[tok] : 0.0f;
        }
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int o = (tile0 + r) * 16 + c16;
        bor[r] = (a.flags & LLMQ_BIAS) && o < a.n ? a.bias[o] : 0.0f;
    }
    float acc[MT][NR][4];
#pragma unroll
    for (int j = 0; j < MT; j++)
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[j][r][i] = 0.0f;
    // The S groups of a staged step.
    auto compute = [&](const uint8_t *cur) {
#pragma unroll
        for (int gi = 0; gi < S; gi++) {
            uint4 ah[MT], al[MT];
#pragma unroll
            for (int j = 0; j < MT; j++) {
                ah[j] = *reinterpret_cast<const uint4 *>(cur + (j * S + gi) * 2048 + lane * 16);
                al[j] = *reinterpret_cast<const uint4 *>(cur + (j * S + gi) * 2048 + 1024 + lane * 16);
            }
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const int e = (w * NR + r) * S + gi;  // (row tile of the workgroup, group) entry
                const uint32_t zp = cur[LY::A + LY::C + e * 16 + c16];
                const float sc = __half2float(
                    *reinterpret_cast<const __half *>(cur + LY::A + LY::C + LY::Z + e * 32 + c16 * 2));
                // w = u - zp in fp16: (1024 + u) - (1024 + zp), both exact; inputs 0 2 4 6 1 3 5 7
                const uint32_t z2 = zp * 0x10001u + 0x64006400u;
                uint32_t q4[4];
                if constexpr (BITS == 4) {  // a code dword: the 8 inputs' nibbles, even inputs low
                    const uint32_t cw = *reinterpret_cast<const uint32_t *>(cur + LY::A + e * 256 + c16 * 16 + g * 4);
                    bytes_f16(cw & 0x0F0F0F0Fu, (cw >> 4) & 0x0F0F0F0Fu, q4);
                } else {  // 8 code bytes (chunk g / 2 of the group, half g % 2), even inputs picked first
                    const uint2 cw = *reinterpret_cast<const uint2 *>(cur + LY::A + e * 512 + (g >> 1) * 256 + c16 * 16 +
                                                                      (g & 1) * 8);
                    bytes_f16(__builtin_amdgcn_perm(cw.y, cw.x, 0x06040200u), __builtin_amdgcn_perm(cw.y, cw.x, 0x07050301u),
                              q4);
                }
                v8h b;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const v2h p = __builtin_bit_cast(v2h, q4[i]) - __builtin_bit_cast(v2h, z2);
                    b[2 * i] = p[0];
                    b[2 * i + 1] = p[1];
                }
#pragma unroll
                for (int j = 0; j < MT; j++) {
                    const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (BITS == 4) {  // |G| < 2^24: one exact chain
                        v4f d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, ah[j]), b, z, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, al[j]), b, d, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[j][r][i] = fmaf(d[i], sc, acc[j][r][i]);  // tile_i16's flush
                    } else {
                        // |w| <= 255: sum 256 hi w (multiples of 256 below 2^32) and sum
                        // lo w (below 2^21) are each exact, and their one rounded
                        // sum is float(G), the reference's conversion of G
                        const v4f dh = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, ah[j]), b, z, 0, 0, 0);
                        const v4f dl = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, al[j]), b, z, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[j][r][i] = fmaf(dh[i] + dl[i], sc, acc[j][r][i]);
                    }
                }
            }
        }
    };
    const int nsteps = NG / S;  // (the launcher picks S dividing the number of groups)
    stage(0, b0);
    for (int s = 0; s < nsteps; s += 2) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies have landed
        __syncthreads();                     // every wave's copy of step s is in; b1 is free
        if (s + 1 < nsteps) stage(s + 1, b1);
        compute(b0);
        if (s + 1 >= nsteps) break;
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (s + 2 < nsteps) stage(s + 2, b0);
        compute(b1);
    }
    if constexpr (KV) {
        // QuantKV.store (kvcache.mojo:333-342) of a key / value head: per
        // token s = max|x| / 127 over its 64 rows (1 if zero), codes
        // round(x / s), from the values the epilogue below stores (bias only).
        const int blk = (rt0 * 16) >> 6, part = blk / a.kv_heads, head = blk % a.kv_heads;
        if (part >= 1 && part <= 2 && rt0 * 16 + 64 <= a.n) {  // (uniform over the workgroup)
            float xv[4], m[4];
            const int o = tile0 * 16 + c16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = acc[0][0][i] * sxr[0][i];
                if (a.flags & LLMQ_BIAS) v += bor[0];
                xv[i] = v;
                m[i] = fmaxf(0.0f, fabsf(v));  // kv_store_kernel's running max from 0
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int off = 8; off > 0; off >>= 1) m[i] = fmaxf(m[i], __shfl_xor(m[i], off));  // the 16 rows
            __shared__ float mx[4 * 16];                   // [wave][token]
            __shared__ __align__(16) int8_t cq[16 * 64];   // [token][row of the head]
            if (c16 == 0)
#pragma unroll
                for (int i = 0; i < 4; i++) mx[w * 16 + 4 * g + i] = m[i];
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tl = 4 * g + i;
                const float mm = fmaxf(fmaxf(mx[tl], mx[16 + tl]), fmaxf(mx[32 + tl], mx[48 + tl]));
                float sc = mm / 127.0f;
                if (sc == 0.0f) sc = 1.0f;
                const float inv = 1.0f / sc;
                cq[tl * 64 + (o & 63)] = (int8_t)llmq_to_int(roundf(xv[i] * inv));
                if (w == 0 && c16 == 0) {
                    const int tok = tt0 * 16 + tl;
                    const int64_t sl = ((int64_t)a.kv_layer * a.kv_max_t + a.kv_pos0 + tok) * a.kv_heads + head;
                    if (tok < a.T) (part == 1 ? a.ks : a.vs)[sl] = sc;
                }
            }
            __syncthreads();
            // each thread one dword: token tid / 16, rows 4 (tid % 16) ..
            const int tl = tid >> 4, tok = tt0 * 16 + tl;
            if (tok < a.T) {
                const int64_t sl = ((int64_t)a.kv_layer * a.kv_max_t + a.kv_pos0 + tok) * a.kv_heads + head;
                reinterpret_cast<uint32_t *>((part == 1 ? a.k8 : a.v8) + sl * 64)[tid & 15] =
                    reinterpret_cast<const uint32_t *>(cq)[tid];
            }
        }
    }
    // Epilogue (store_out): tile_i16's acc * sx + b, then GELU / residual.
    if (tile0 * 16 >= a.n) return;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int o = (tile0 + r) * 16 + c16;
        if (o >= a.n) continue;
#pragma unroll
        for (int j = 0; j < MT; j++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tok = (tt0 + j) * 16 + 4 * g + i;
                if (tok >= a.T) continue;
                float v = acc[j][r][i] * sxr[j][i];
                if (a.flags & LLMQ_BIAS) v += bor[r];
                if (a.flags & LLMQ_GELU) v = gelu_ref(v);
                float *dst = a.out + (int64_t)tok * a.ldo + o;
                if (a.flags & LLMQ_RESID) v += *dst;
                *dst = v;
            }
        }
    }
}

}  // namespace

bool gemm_mfma_supports(const llmq_mat *w, int64_t T) {
    if (w->kind != MAT_QUANT || T < 2) return false;
    const int64_t seg = w->group < 256 ? w->group : 256;
    return w->k % 32 == 0 && w->k % seg == 0 && w->group % 32 == 0 &&
           (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 256 < (int64_t)kOOB && T * w->k * 2 < (int64_t)kOOB;
}

bool gemm_f16_supports(const llmq_mat *w, int64_t T) {
    if (const char *e = getenv("LLMQ_MFMA_F16"))
        if (atoi(e) == 0) return false;
    return gemm_mfma_supports(w, T) && (w->bits == 4 || w->bits == 8) && w->group == 32 &&
           (T + 15) / 16 * 16 * w->k * 4 < (int64_t)kOOB;
}

size_t gemm_f16_planes_bytes(const llmq_mat *w, int64_t T) { return (size_t)((T + 15) / 16 * 16) * w->k * 4; }

bool gemm_kv_fold_ok(const llmq_mat *w, int64_t T, const llmq_kv *cache) {
    if (const char *e = getenv("LLMQ_KV_FOLD"))
        if (e[0] == '0') return false;
    if (const char *e = getenv("LLMQ_F16_TILE"))  // measurement tiles keep kv_store_kernel
        if (e[0]) return false;
    const int min_t = exact_order() ? 2 : 8;
    if (getenv("LLMQ_MFMA_MIN_T")) return false;
    if (!cache || cache->integer || cache->head_dim != 64 || T < min_t || !w->a16) return false;
    const int64_t C = (int64_t)cache->n_head * 64;
    return gemm_f16_supports(w, T) && w->n == 3 * C && w->n % 64 == 0;
}

int launch_gemm_mfma(llmq_ctx *ctx, const GemvRequest &rq, int16_t *xq, float *sx, uint8_t *planes) {
    const llmq_mat *w = rq.w;
    const int64_t T = rq.T, K = w->k;
    const int64_t ldx = rq.ldx ? rq.ldx : K;
    LLMQ_REQUIRE(gemm_mfma_supports(w, T), "linear: no MFMA GEMM for this matrix");
    LLMQ_REQUIRE(!planes || gemm_f16_supports(w, T), "linear: fp16 planes given for a matrix the fp16 GEMM does not take");
    LLMQ_REQUIRE(!rq.kv || planes, "linear: the key / value store needs the fp16 GEMM");
    LLMQ_REQUIRE(!rq.kv || !(rq.flags & (LLMQ_GELU | LLMQ_RESID)),
                 "linear: the key / value store takes the product plus bias only");
    const int upt = (int)((K / 4 + 255) / 256);
    const bool ln = rq.ln_w != nullptr;
#define ACTQ(L, U) hipLaunchKernelGGL((act_q16_kernel<L, U>), dim3((unsigned)T), dim3(256), L ? K * 4 : 0, ctx->stream, rq.x, ldx, \
                                       rq.ln_w, rq.ln_b, (int)K, xq, sx, planes)
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
    // the 32-row tiles; the rest (n % 32 rows: the vocabulary's last 17)
    // go through rows_i16 below
    const int full = (int)(w->n / 32 * 32);
    if (planes && full > 0) {
        F16Args f;
        f.planes = planes;
        f.codes = w->codes;
        f.zps = w->zps;
        f.scales = w->scales;
        f.sx = sx;
        f.bias = rq.bias ? rq.bias : rq.out;
        f.out = rq.out;
        f.ldo = rq.ldo ? rq.ldo : w->n;
        f.T = (int)T;
        f.n = full;
        f.ntiles = (int)w->ntiles;
        f.CK = (int)w->CK;
        f.flags = rq.flags;
        f.xcd = 1;
        if (const char *e = getenv("LLMQ_F16_XCD")) f.xcd = atoi(e) != 0;
        // a workgroup's tile: MT token tiles x NW NR row tiles, S groups a
        // step (S divides the number of groups); LLMQ_F16_TILE=MT,NR,S[,NW]
        // picks another instantiation, for measurement
        int mt = 1, nr = 1, st = 4, nw = 4;
        if (const char *e = getenv("LLMQ_F16_TILE")) {
            int x = 0, y = 0, z = 0, v = 4;
            if (sscanf(e, "%d,%d,%d,%d", &x, &y, &z, &v) >= 3) mt = x, nr = y, st = z, nw = v;
        }
        const int ngroups = (int)(w->k / 32);
        if (ngroups % st != 0) mt = 1, nr = 1, nw = 4, st = ngroups % 2 == 0 ? 2 : 1;
        const int rtiles = full / 16, ttiles = (int)((T + 15) / 16);
        bool ok = false;
        if (rq.kv) {  // the default tile with the cache store in its epilogue
            LLMQ_REQUIRE(gemm_kv_fold_ok(w, T, rq.kv->cache) && mt == 1 && nr == 1 && nw == 4 && full == w->n,
                         "linear: no key / value store in this GEMM's epilogue");
            const llmq_kv *kv = rq.kv->cache;
            LLMQ_REQUIRE(rq.kv->layer >= 0 && rq.kv->layer < kv->n_layer && rq.kv->pos0 >= 0 &&
                             rq.kv->pos0 + T <= kv->max_t,
                         "linear: cache positions %d..%lld of layer %d out of range", rq.kv->pos0,
                         (long long)(rq.kv->pos0 + T - 1), rq.kv->layer);
            f.k8 = kv->k;
            f.v8 = kv->v;
            f.ks = kv->ks;
            f.vs = kv->vs;
            f.kv_layer = rq.kv->layer;
            f.kv_pos0 = rq.kv->pos0;
            f.kv_max_t = kv->max_t;
            f.kv_heads = kv->n_head;
            const dim3 grid((unsigned)(rtiles / 4), (unsigned)ttiles);
#define F16KV(SS)                                                                                                   \
    if (!ok && st == SS) {                                                                                          \
        if (w->bits == 4)                                                                                           \
            hipLaunchKernelGGL((gemm_f16_kernel<1, 1, SS, 4, 4, true>), grid, dim3(256), 0, ctx->stream, f);        \
        else                                                                                                        \
            hipLaunchKernelGGL((gemm_f16_kernel<1, 1, SS, 4, 8, true>), grid, dim3(256), 0, ctx->stream, f);        \
        ok = true;                                                                                                  \
    }
            F16KV(4) F16KV(2) F16KV(1)
#undef F16KV
        }
#define F16K(M, R, SS, NW)                                                                                          \
    if (!ok && mt == M && nr == R && st == SS && nw == NW) {                                                         \
        const dim3 grid((unsigned)((rtiles + NW * R - 1) / (NW * R)), (unsigned)((ttiles + M - 1) / M));              \
        if (w->bits == 4)                                                                                            \
            hipLaunchKernelGGL((gemm_f16_kernel<M, R, SS, NW, 4, false>), grid, dim3(NW * 64), 0, ctx->stream, f);   \
        else                                                                                                         \
            hipLaunchKernelGGL((gemm_f16_kernel<M, R, SS, NW, 8, false>), grid, dim3(NW * 64), 0, ctx->stream, f);   \
        ok = true;                                                                                                   \
    }
        F16K(1, 1, 4, 4) F16K(1, 1, 2, 4) F16K(1, 1, 1, 4) F16K(2, 1, 4, 4) F16K(1, 2, 4, 4) F16K(1, 1, 8, 4)
        F16K(1, 1, 4, 8) F16K(2, 1, 4, 8) F16K(1, 1, 8, 8)
#undef F16K
        LLMQ_REQUIRE(ok, "linear: no fp16 GEMM instantiation for LLMQ_F16_TILE=%d,%d,%d,%d", mt, nr, st, nw);
        LLMQ_HIP(hipGetLastError());
    }
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
    a.n = full;
    a.ntiles = (int)w->ntiles;
    a.CK = (int)w->CK;
    a.NG = (int)w->NG;
    a.G = (int)w->group;
    a.seg = (int)(w->group < 256 ? w->group : 256);
    a.flags = rq.flags;
    // tokens a workgroup: 16 MT; 32 for the wide matrices (476 tokens: qkv
    // 21.0 -> 20.1 us, fc 23.3 -> 20.4 us), 16 for the narrow ones (more
    // workgroups); LLMQ_MFMA_MT overrides, for measurement
    int mt = w->n >= 2048 ? 2 : 1;
    if (const char *e = getenv("LLMQ_MFMA_MT")) mt = atoi(e) == 1 ? 1 : atoi(e) == 4 ? 4 : 2;
    dim3 grid((unsigned)((full + TN - 1) / TN), (unsigned)((T + 16 * mt - 1) / (16 * mt)));
    const bool seg32 = a.seg == 32;
#define GK(B, S, M) hipLaunchKernelGGL((gemm_i8_kernel<B, S, M>), grid, dim3(256), 0, ctx->stream, a)
#define GKM(B, S)                        \
    do {                                 \
        if (mt == 1) GK(B, S, 1);        \
        else if (mt == 2) GK(B, S, 2);   \
        else GK(B, S, 4);                \
    } while (0)
    if (full > 0 && !planes) {
        if (w->bits == 4) {
            if (seg32) GKM(4, true); else GKM(4, false);
        } else {
            if (seg32) GKM(8, true); else GKM(8, false);
        }
    }
#undef GKM
#undef GK
    LLMQ_HIP(hipGetLastError());
    if (w->n > full) {
        const int nt = (int)(w->n - full);
        hipLaunchKernelGGL(rows_i16_kernel, dim3((unsigned)(((int64_t)nt * T + 3) / 4)), dim3(64), 0, ctx->stream, a,
                           w->bits, full, nt);
        LLMQ_HIP(hipGetLastError());
    }
    return LLMQ_OK;
}
