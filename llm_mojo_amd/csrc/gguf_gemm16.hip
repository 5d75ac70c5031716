// Several-token Q4_K matmul on the fp16 matrix cores: matmul_rows for T > 1
// over a GGUFMatrix of Q4_K rows (kernels.mojo:314-349; the Q4_K decoder,
// gguf.mojo:205-250).
//
// A Q4_K weight of sub-block j (32 weights) of a superblock is
// d sc_j u - dmin m_j, with u a 4-bit code, sc_j and m_j 6-bit integers and
// d, dmin fp16.  Over a superblock of a row,
//   sum_i w_i x_i = d sum_j sum_i (sc_j u_i) x_i - dmin sum_j m_j X_j,
// X_j the sub-block's sum of x, and sc_j u_i <= 945 and m_j are exact in
// fp16.  The activations go in as an "h16 record": per token and superblock
// a power-of-two scale s (max |x s| < 2^10) and x s as two fp16 planes,
// hi = fp16(x s), lo = fp16(x s - hi) (together x s to 22 bits), and the
// same two planes of s X_j.  The matrix cores (v_mfma_f32_16x16x32_f16)
// form D = sum (sc u)(hi + lo) and D' = sum m (S hi + S lo), every product
// exact in their fp32 sums, and the kernel adds (d D - dmin D') / s.  The
// outputs agree with the reference's float matmul to fp32 rounding, not in
// its summation order.
//
// Record layout for T tokens (padded to T16, a multiple of 16), KB = K / 32
// sub-blocks and NSB = K / 256 superblocks, the 16 tokens of a token tile
// side by side so that each operand load of a wave is 1 KB in one piece:
//   planes  fp16 [T16 / 16][KB][hi, lo][4 groups][16 tokens][8]: group g
//           holds inputs 8g .. 8g + 7 of the sub-block in the order 0, 2, 4,
//           6, 1, 3, 5, 7 (the order in which a code dword's nibbles decode,
//           below);
//   sums    fp16 [T16 / 16][NSB][hi, lo][16 tokens][8]: s X_j, j = 0..7;
//   inv     float [T16 / 16][NSB][16 tokens]: 1 / s.
// A padded token's record (zeros from the record kernel, anything from
// other writers) reaches only that token's outputs, which are not stored.
//
// Mapping: a workgroup owns RT row tiles of 16 rows and a tile of 16 tokens;
// its NW waves split the row's superblocks into contiguous runs.  In a
// superblock a wave's lane l takes token / row l % 16 and input group
// l / 16 of each sub-block: the A operand is that token's group of the
// record (32 bytes), the B operand the row's code dword for the group (the
// (chunk, row) entry of the device layout) times sc_j; lane l holds outputs
// (tokens 4 (l / 16) + i, row l % 16).  The waves' partial sums are added in
// LDS in wave order.
#include "common.h"
#include "hs_rec.h"
#include <type_traits>

namespace {

constexpr uint32_t kOOB = 0x80000000u;

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

struct HArgs {
    const uint8_t *codes, *sb, *planes, *sums, *inv;
    uint32_t codes_bytes, sb_bytes, planes_bytes, sums_bytes, inv_bytes;
    int n, KB, CK, NSB, ntiles, T, flags;
    int stream;  // weights read by one token tile only: non-temporal loads
    int64_t ldo;
    const float *bias;
    float *out;
    // h16s input: the exponents (inv is then unused, sums in the h16s layout);
    // with ssq, outputs times 1 / sqrt(sum x^2 / C + eps) of their token
    const uint8_t *exps;
    uint32_t exps_bytes;
    const float *ssq;
    int C;
    float eps;
    HSRec orec;          // the h16s record an epilogue writes (planes null: none)
    const float *ogain;  // of (out + residual) * ogain
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
// Weight loads with cache policy AUX: 2 (non-temporal) when no other
// workgroup reads the same weights, else 0 (cached for the other token
// tiles).  A constant part of the offset goes in the scalar offset, so that
// the loads of one base share its vector register.
template <int AUX>
__device__ __forceinline__ uint4 wload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
template <int AUX>
__device__ __forceinline__ uint32_t wload4(__amdgpu_buffer_rsrc_t r, uint32_t off, int soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, soff, AUX);
}
__device__ __forceinline__ uint4 bload16s(__amdgpu_buffer_rsrc_t r, uint32_t off, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, soff, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

struct Rec {
    uint8_t *planes;
    _Float16 *sums;
    float *inv;
};

Rec rec_parts(void *rec, int64_t T, int64_t K) {
    const int64_t T16 = (T + 15) / 16 * 16, KB = K / 32, NSB = K / 256;
    uint8_t *p = static_cast<uint8_t *>(rec);
    return {p, reinterpret_cast<_Float16 *>(p + T16 * KB * 128),
            reinterpret_cast<float *>(p + T16 * KB * 128 + T16 * NSB * 32)};
}

// The record of x (T x K floats, row stride ldx): workgroup (blockIdx.x,
// token blockIdx.y) covers 4 superblocks, one a wave.
__global__ __launch_bounds__(256) void act_h16_kernel(const float *__restrict__ x, int64_t ldx, int T, int KB,
                                                      int NSB, uint8_t *__restrict__ planes,
                                                      _Float16 *__restrict__ sums, float *__restrict__ inv) {
    const int t = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int sb = blockIdx.x * 4 + w;
    const bool ok = sb < NSB, in = ok && t < T;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) v[q] = in ? x[(int64_t)t * ldx + sb * 256 + 64 * q + lane] : 0.0f;
    llmq_h16_store(planes, sums, inv, KB, NSB, t, sb, v, ok);
}

// 1024 + the 8 bytes of (a, b) as fp16 pairs (a0, a1), (a2, a3), (b0, b1),
// (b2, b3): 0x6400 | n is 1024 + n in fp16 for n < 1024.
__device__ __forceinline__ void bytes_f16(uint32_t a, uint32_t b, uint32_t (&d)[4]) {
    d[0] = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
    d[1] = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
    d[2] = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
    d[3] = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
}

// An h16s superblock for lane (token c16, group g): its 16 exponents ev
// (bytes), its A operands ah / al (group g of each sub-block: half
// 2u + g / 2) and sum operand sq (halves 8 (g % 2) + i) brought to the
// common scale 2^c; inv[i] = 2^-c of output token 4g + i.
__device__ __forceinline__ uint32_t pk_mul(uint32_t x, uint32_t f) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, x) * __builtin_bit_cast(v2h, f));
}
__device__ __forceinline__ uint4 pk_mul4(uint4 x, uint32_t f) {
    return make_uint4(pk_mul(x.x, f), pk_mul(x.y, f), pk_mul(x.z, f), pk_mul(x.w, f));
}
// Signed byte (shift / 8) of w, shift a multiple of 8 (may vary by lane).
__device__ __forceinline__ int sbyte(uint32_t w, uint32_t shift) { return (int)(w << (24u - shift)) >> 24; }

__device__ __forceinline__ void hs_rescale(uint4 ev, int g, uint4 (&ah)[8], uint4 (&al)[8], uint4 &sq,
                                           float (&inv)[4]) {
    const uint32_t ew[4] = {ev.x, ev.y, ev.z, ev.w};
    int c = sbyte(ew[0], 0);
#pragma unroll
    for (int i = 0; i < 16; i++) c = min(c, sbyte(ew[i >> 2], 8u * (i & 3)));
    // 2^(c - eh) as fp16 bits (v_ldexp_f16: subnormal from c - eh = -15, 0
    // from -25)
    auto f16 = [&](int eh) -> uint32_t {
        return (uint32_t)__builtin_bit_cast(unsigned short, __builtin_amdgcn_ldexph((_Float16)1.0f, c - eh));
    };
    // the lane's A operand of sub-block u: half 2u + g / 2, byte 2 (u % 2) + g / 2 of word u / 2
    const uint32_t oA = (g >> 1) ? 8u : 0u;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const uint32_t f = f16(sbyte(ew[u >> 1], 16u * (u & 1) + oA)), fp = f | (f << 16);
        ah[u] = pk_mul4(ah[u], fp);
        al[u] = pk_mul4(al[u], fp);
    }
    // its sums: halves 8 (g % 2) .. + 7, words 2 (g % 2) and 2 (g % 2) + 1
    const uint32_t s0 = (g & 1) ? ev.z : ev.x, s1 = (g & 1) ? ev.w : ev.y;
    uint32_t fs[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t wv = k < 2 ? s0 : s1;
        fs[k] = f16(sbyte(wv, 16u * (k & 1))) | (f16(sbyte(wv, 16u * (k & 1) + 8u)) << 16);
    }
    sq = make_uint4(pk_mul(sq.x, fs[0]), pk_mul(sq.y, fs[1]), pk_mul(sq.z, fs[2]), pk_mul(sq.w, fs[3]));
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int co = __shfl(c, 4 * g + i);
        inv[i] = __uint_as_float((uint32_t)(127 - co) << 23);
    }
}

// SIN: the record is an h16s record (with a.ssq: outputs RMS-normalized).
// OUT 1 (RT 1, LLMQ_RESID): the epilogue also writes the h16s record of
// (out + residual) * ogain to a.orec (when set), this matmul's 16-row tile
// being a half of the next one's input.  OUT 2 (RT 4, the rows are
// [gate; up]): slots 0, 1 take gate tiles 2b, 2b + 1, slots 2, 3 the up
// tiles of the same rows, and the epilogue writes only the h16s record of
// silu(gate) * up (a.orec).
template <int NW, int RT, bool SIN, int OUT>
__global__ __launch_bounds__(NW * 64) void gemm_h16_q4k_kernel(HArgs a) {
    static_assert(OUT != 1 || (RT == 1 && NW >= 4), "record epilogue: one row tile, a thread an output");
    static_assert(OUT != 2 || (RT == 4 && NW * 64 >= 512), "SwiGLU epilogue: two gate and two up tiles");
    __shared__ float part[NW][RT][256];
    __shared__ float s_r[16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c16 = lane & 15, g = lane >> 4;
    const int tt = blockIdx.y;
    auto tile_of = [&](int r) {
        return OUT == 2 ? (r < 2 ? 2 * (int)blockIdx.x + r : a.ntiles / 2 + 2 * (int)blockIdx.x + r - 2)
                        : (int)blockIdx.x * RT + r;
    };
    const auto rc = make_rsrc(a.codes, a.codes_bytes), rs = make_rsrc(a.sb, a.sb_bytes);
    const auto rp = make_rsrc(a.planes, a.planes_bytes), rq = make_rsrc(a.sums, a.sums_bytes);
    const auto ri = make_rsrc(a.inv, a.inv_bytes), re = make_rsrc(a.exps, a.exps_bytes);
    // epilogue operands, in flight from the start: the record gain of this
    // thread's output (OUT 1) and, wave 0, the token's sums of squares (lane:
    // token c16, quarter g of the halves)
    float og = 0.0f;
    if (OUT == 1 && a.orec.planes && tid < 256) og = a.ogain[tile_of(0) * 16 + (tid & 15)];
    // the residual of each output this thread writes (LLMQ_RESID), likewise
    constexpr int NIT = (RT * 256 + NW * 64 - 1) / (NW * 64);
    float res[NIT];
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int e = tid + it * NW * 64, r = e >> 8, q = e & 255, tk = tt * 16 + (q >> 4), o = tile_of(r) * 16 + (q & 15);
        const bool rd = OUT != 2 && (a.flags & LLMQ_RESID) && e < RT * 256 && o < a.n && tk < a.T;
        res[it] = rd ? a.out[(int64_t)tk * a.ldo + o] : 0.0f;
    }
    // (the first kSq float4 in registers, added after the main loop: wave 0
    // does not wait for them before its own loads; the record epilogue's
    // matmuls take no norm, 16-wave ones no registers to spare)
    constexpr bool NRM = SIN && OUT != 1;
    constexpr int kSq = NRM && NW < 16 ? 8 : 1;
    const bool nrm = NRM && a.ssq && w == 0;
    const int nq4 = a.C / 256;  // float4 a lane: a quarter of the token's C / 16 halves
    const float4 *p4 = reinterpret_cast<const float4 *>(a.ssq + (int64_t)(tt * 16 + c16) * (a.C / 16) + g * 4 * nq4);
    float4 sqv[kSq];  // (set and read by wave 0 only)
    if (nrm && kSq > 1) {
#pragma unroll
        for (int k = 0; k < kSq; k++) sqv[k] = k < nq4 ? p4[k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const int s0 = w * a.NSB / NW, s1 = (w + 1) * a.NSB / NW;  // the wave's superblocks (an even split)
    const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, km1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    float acc[RT][4];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[r][i] = 0.0f;
    // the weights (block fields and code dwords) of superblock sbi, the
    // cache policy chosen once for all of them
    auto load_w_pol = [&](auto pol, int sbi, uint4 (&f)[RT], uint32_t (&cw)[RT][8]) {
        constexpr int AUX = decltype(pol)::value;
#pragma unroll
        for (int r = 0; r < RT; r++) {
            const int tl = tile_of(r);
            const bool ok = tl < a.ntiles;
            f[r] = wload16<AUX>(rs, ok ? (uint32_t)(((tl * a.NSB + sbi) * 16 + c16) * 16) : kOOB);
            // chunk entries of one row tile are 256 bytes apart (kOOB + 256 u stays out of range)
            const uint32_t cb = ok ? (uint32_t)(((tl * a.CK + sbi * 8) * 16 + c16) * 16 + g * 4) : kOOB;
#pragma unroll
            for (int u = 0; u < 8; u++) cw[r][u] = wload4<AUX>(rc, cb, 256 * u);
        }
    };
    auto load_w = [&](int sbi, uint4 (&f)[RT], uint32_t (&cw)[RT][8]) {
        if (a.stream)
            load_w_pol(std::integral_constant<int, 2>{}, sbi, f, cw);
        else
            load_w_pol(std::integral_constant<int, 0>{}, sbi, f, cw);
    };
    // A wave with several superblocks (the down matrix at batch 16) has the
    // next one's weights in flight while it computes one, issued after the
    // current superblock's record loads, which it waits for (loads complete
    // in issue order): 1.190 -> 1.156 ms a batch-16 step.  Its first four
    // sub-blocks' planes in flight as well measured 1.187 ms.
    uint4 fn[RT];
    uint32_t cwn[RT][8];
    if (s0 < s1) load_w(s0, fn, cwn);
    for (int sbi = s0; sbi < s1; sbi++) {
        uint4 f[RT], ah[8], al[8];
        uint32_t cw[RT][8];
        const uint32_t ab = (uint32_t)((tt * a.KB + sbi * 8) * 2048 + lane * 16);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            ah[u] = bload16s(rp, ab, 2048 * u);
            al[u] = bload16s(rp, ab, 2048 * u + 1024);
        }
        // sums planes: hi in group 0, lo in group 1, zeros in groups 2 and 3
        // (h16s: all four groups); the scales (h16s: the token's exponents)
        uint4 sq = SIN ? bload16(rq, (uint32_t)(((tt * a.NSB + sbi) * 64 + g * 16 + c16) * 16))
                       : bload16(rq, g < 2 ? (uint32_t)((tt * a.NSB + sbi) * 512 + lane * 16) : kOOB);
        const uint4 iv = SIN ? bload16(re, (uint32_t)(((tt * a.NSB + sbi) * 16 + c16) * 16))
                             : bload16(ri, (uint32_t)(((tt * a.NSB + sbi) * 16 + 4 * g) * 4));
#pragma unroll
        for (int r = 0; r < RT; r++) {
            f[r] = fn[r];
#pragma unroll
            for (int u = 0; u < 8; u++) cw[r][u] = cwn[r][u];
        }
        __builtin_amdgcn_sched_barrier(0);
        if (sbi + 1 < s1) load_w(sbi + 1, fn, cwn);
        __builtin_amdgcn_sched_barrier(0);  // the superblock's loads all issue before its first product
        float inv[4];
        if constexpr (SIN) {
            hs_rescale(iv, g, ah, al, sq, inv);
        } else {
            inv[0] = __uint_as_float(iv.x);
            inv[1] = __uint_as_float(iv.y);
            inv[2] = __uint_as_float(iv.z);
            inv[3] = __uint_as_float(iv.w);
        }
#pragma unroll
        for (int r = 0; r < RT; r++) {
            // sc_j and m_j as bytes (k_scale_min, gguf.mojo:205-221, four at a time)
            const uint32_t sc_lo = f[r].y & 0x3F3F3F3Fu, m_lo = f[r].z & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (f[r].w & 0x0F0F0F0Fu) | ((f[r].y >> 2) & 0x30303030u);
            const uint32_t m_hi = ((f[r].w >> 4) & 0x0F0F0F0Fu) | ((f[r].z >> 2) & 0x30303030u);
            uint32_t scp[4], mp[4];
            bytes_f16(sc_lo, sc_hi, scp);
            bytes_f16(m_lo, m_hi, mp);
            v2h sc[4], nsc[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[i] = __builtin_bit_cast(v2h, scp[i]) - k1024;  // (sc_2i, sc_2i+1)
                nsc[i] = sc[i] * km1024;
            }
            v4f d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t lo = cw[r][u] & 0x0F0F0F0Fu, hi = (cw[r][u] >> 4) & 0x0F0F0F0Fu;
                uint32_t q[4];
                bytes_f16(lo, hi, q);  // 1024 + (u0, u2), (u4, u6), (u1, u3), (u5, u7)
                const _Float16 s1 = sc[u >> 1][u & 1], n1 = nsc[u >> 1][u & 1];
                const v2h sv = {s1, s1}, nv = {n1, n1};
                v8h b;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // (1024 + u) sc - 1024 sc = u sc exactly (both terms and the result fit fp16)
                    const v2h p = __builtin_elementwise_fma(__builtin_bit_cast(v2h, q[i]), sv, nv);
                    b[2 * i] = p[0];
                    b[2 * i + 1] = p[1];
                }
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, ah[u]), b, d, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, al[u]), b, d, 0, 0, 0);
            }
            // m_j in groups 0 and 1 (against the sums' hi and lo planes); h16s:
            // m of half 8 (g % 2) + i's sub-block in every group
            v8h bm;
            if constexpr (SIN) {
                const uint32_t ma = (g & 1) ? mp[2] : mp[0], mb = (g & 1) ? mp[3] : mp[1];
                const uint32_t dup[4] = {__builtin_amdgcn_perm(ma, ma, 0x01000100u), __builtin_amdgcn_perm(ma, ma, 0x03020302u),
                                         __builtin_amdgcn_perm(mb, mb, 0x01000100u), __builtin_amdgcn_perm(mb, mb, 0x03020302u)};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const v2h p = __builtin_bit_cast(v2h, dup[i]) - k1024;
                    bm[2 * i] = p[0];
                    bm[2 * i + 1] = p[1];
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const v2h p = g < 2 ? __builtin_bit_cast(v2h, mp[i]) - k1024 : (v2h){(_Float16)0.0f, (_Float16)0.0f};
                    bm[2 * i] = p[0];
                    bm[2 * i + 1] = p[1];
                }
            }
            v4f dm = {0.0f, 0.0f, 0.0f, 0.0f};
            dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, sq), bm, dm, 0, 0, 0);
            const float dd = __half2float(__ushort_as_half((unsigned short)(f[r].x & 0xFFFFu)));
            const float dmin = __half2float(__ushort_as_half((unsigned short)(f[r].x >> 16)));
#pragma unroll
            for (int i = 0; i < 4; i++) acc[r][i] = fmaf(inv[i], fmaf(-dmin, dm[i], dd * d[i]), acc[r][i]);
        }
    }
    if (nrm) {  // 1 / rms of token c16: the quarters in a fixed order
        float ssum = 0.0f;
#pragma unroll
        for (int k = 0; k < kSq; k++) ssum += (sqv[k].x + sqv[k].y) + (sqv[k].z + sqv[k].w);
        for (int k = kSq > 1 ? kSq : 0; k < nq4; k++) {
            const float4 v = p4[k];
            ssum += (v.x + v.y) + (v.z + v.w);
        }
        ssum += __shfl_xor(ssum, 16);
        ssum += __shfl_xor(ssum, 32);
        if (g == 0) s_r[c16] = 1.0f / sqrtf(ssum / (float)a.C + a.eps);
    }
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int i = 0; i < 4; i++) part[w][r][(4 * g + i) * 16 + c16] = acc[r][i];
    __syncthreads();
    if constexpr (OUT == 2) {
        // gate tile r2 and the up tile of the same rows: silu(gate) * up is
        // half 2b + r2 of the next matmul's input (zeros for padded tokens)
        if (tid < 512) {
            const int r2 = tid >> 8, q = tid & 255, tk = tt * 16 + (q >> 4);
            float gt = part[0][r2][q], up = part[0][r2 + 2][q];
#pragma unroll
            for (int p = 1; p < NW; p++) {
                gt += part[p][r2][q];
                up += part[p][r2 + 2][q];
            }
            if (NRM && a.ssq) {
                gt *= s_r[q >> 4];
                up *= s_r[q >> 4];
            }
            const float h = (gt / (1.0f + expf(-gt))) * up;
            hs_store_half(a.orec, tk, 2 * (int)blockIdx.x + r2, tk < a.T ? h : 0.0f, 0.0f);
        }
        return;
    }
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int e = tid + it * NW * 64;
        if (e >= RT * 256) break;
        const int r = e >> 8, q = e & 255, tk = tt * 16 + (q >> 4), o = tile_of(r) * 16 + (q & 15);
        float v = part[0][r][q];
#pragma unroll
        for (int p = 1; p < NW; p++) v += part[p][r][q];
        if (NRM && a.ssq) v *= s_r[q >> 4];
        const bool live = o < a.n && tk < a.T;
        if (live) {
            if (a.flags & LLMQ_BIAS) v += a.bias[o];
            if (a.flags & LLMQ_GELU) v = gelu_ref(v);
            if (a.flags & LLMQ_RESID) v += res[it];
            a.out[(int64_t)tk * a.ldo + o] = v;
        }
        // (the next matmul's input row (out + residual) * gain, zeros for
        // padded tokens and rows)
        if (OUT == 1 && a.orec.planes) hs_store_half(a.orec, tk, tile_of(r), live ? v * og : 0.0f, live ? v : 0.0f);
    }
}

// The h16s record of x * gain with the sums of squares of x (T x K floats,
// row stride ldx): workgroup (blockIdx.x, token blockIdx.y) covers a
// superblock, wave w inputs 64 w .. 64 w + 63 (four halves).
__global__ __launch_bounds__(256) void rec_h16s_kernel(const float *__restrict__ x, int64_t ldx, int T,
                                                       const float *__restrict__ gain, HSRec o) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    const float xv = t < T ? x[(int64_t)t * ldx + i] : 0.0f;
    hs_store_half(o, t, i >> 4, xv * gain[i], xv);
}

// The same matmul for many tokens (prompts): a workgroup of 8 waves owns 8
// row tiles and kPT token tiles; each superblock's record for those tokens
// (kPT x 16 KiB of planes, their sums and scales) is copied into LDS by the
// global-to-LDS loads, double-buffered so the next superblock's copy runs
// under this one's products.  Wave w decodes the codes of row tiles w % 4
// and w % 4 + 4 once and multiplies them with token tiles 2 (w / 4) and
// 2 (w / 4) + 1, each operand read from LDS serving two products.  Each
// wave covers the whole reduction axis, so no partial sums are combined.
constexpr int kPT = 4;                                        // token tiles a workgroup
constexpr int kPL = 16384;                                    // planes bytes of a token tile's superblock
constexpr int kStage = kPT * kPL + kPT * 512 + 1024;          // planes, sums, inv (padded)
constexpr int kRW = 2;                                        // row tiles a wave

__global__ __launch_bounds__(512) void gemm_h16_q4k_lds_kernel(HArgs a, int ntt) {
    // two separate buffers, so that the compiler sees a copy into one cannot alias reads of the other
    __shared__ __align__(16) uint8_t st0[kStage], st1[kStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c16 = lane & 15, g = lane >> 4;
    const int th = w >> 2, tt0 = blockIdx.y * kPT;
    int rt[kRW];
    bool rok[kRW];
#pragma unroll
    for (int r = 0; r < kRW; r++) {
        rt[r] = blockIdx.x * 4 * kRW + (w & 3) + 4 * r;
        rok[r] = rt[r] < a.ntiles;
    }
    const auto rc = make_rsrc(a.codes, a.codes_bytes), rs = make_rsrc(a.sb, a.sb_bytes);
    const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, km1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    // the copy of superblock s into buffer b: planes in 8 rounds of 512 x 16 bytes, sums by waves 0-1,
    // scales by wave 2 (tiles past the record read tile 0; their outputs are not written)
    auto stage = [&](int s, uint8_t *buf) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int t = r >> 1, tt = tt0 + t < ntt ? tt0 + t : 0;
            const uint8_t *src = a.planes + ((int64_t)tt * a.KB + 8 * s) * 2048 + (r & 1) * 8192 + tid * 16;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(buf + t * kPL + (r & 1) * 8192 + w * 1024), 16, 0, 0);
        }
        if (w < 2) {
            const int t = tid >> 5, tt = tt0 + t < ntt ? tt0 + t : 0;
            const uint8_t *src = a.sums + ((int64_t)tt * a.NSB + s) * 512 + (tid & 31) * 16;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(buf + kPT * kPL + w * 1024), 16, 0, 0);
        } else if (w == 2) {
            const int t = (lane >> 2) & 3, tt = tt0 + t < ntt ? tt0 + t : 0;
            const uint8_t *src = a.inv + ((int64_t)tt * a.NSB + s) * 64 + (lane & 3) * 16;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(buf + kPT * kPL + kPT * 512), 16, 0, 0);
        }
    };
    auto load_codes = [&](int s, uint4 (&f)[kRW], uint32_t (&cw)[kRW][8]) {
#pragma unroll
        for (int r = 0; r < kRW; r++) {
            f[r] = bload16(rs, rok[r] ? (uint32_t)(((rt[r] * a.NSB + s) * 16 + c16) * 16) : kOOB);
            const uint32_t cb = rok[r] ? (uint32_t)(((rt[r] * a.CK + s * 8) * 16 + c16) * 16 + g * 4) : kOOB;
#pragma unroll
            for (int u = 0; u < 8; u++) cw[r][u] = bload4(rc, cb + 256u * u);
        }
    };
    float acc[kRW][2][4];
#pragma unroll
    for (int r = 0; r < kRW; r++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[r][t][i] = 0.0f;
    uint4 f[kRW];
    uint32_t cw[kRW][8];
    // superblock s from buffer cur, the next one's copy into nxt
    auto step = [&](int s, const uint8_t *cur, uint8_t *nxt) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies (and codes) have landed
        __syncthreads();                     // every wave's copy of s is in; nxt is free
        // this superblock's codes times sc_j, and m_j, as fp16 (as gemm_h16_q4k_kernel)
        v8h bw[kRW][8], bm[kRW];
        float dd[kRW], dmin[kRW];
#pragma unroll
        for (int r = 0; r < kRW; r++) {
            const uint32_t sc_lo = f[r].y & 0x3F3F3F3Fu, m_lo = f[r].z & 0x3F3F3F3Fu;
            const uint32_t sc_hi = (f[r].w & 0x0F0F0F0Fu) | ((f[r].y >> 2) & 0x30303030u);
            const uint32_t m_hi = ((f[r].w >> 4) & 0x0F0F0F0Fu) | ((f[r].z >> 2) & 0x30303030u);
            uint32_t scp[4], mp[4];
            bytes_f16(sc_lo, sc_hi, scp);
            bytes_f16(m_lo, m_hi, mp);
            v2h sc[4], nsc[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sc[i] = __builtin_bit_cast(v2h, scp[i]) - k1024;
                nsc[i] = sc[i] * km1024;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t lo = cw[r][u] & 0x0F0F0F0Fu, hi = (cw[r][u] >> 4) & 0x0F0F0F0Fu;
                uint32_t q[4];
                bytes_f16(lo, hi, q);
                const _Float16 s1 = sc[u >> 1][u & 1], n1 = nsc[u >> 1][u & 1];
                const v2h sv = {s1, s1}, nv = {n1, n1};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const v2h pp = __builtin_elementwise_fma(__builtin_bit_cast(v2h, q[i]), sv, nv);
                    bw[r][u][2 * i] = pp[0];
                    bw[r][u][2 * i + 1] = pp[1];
                }
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const v2h pp = g < 2 ? __builtin_bit_cast(v2h, mp[i]) - k1024 : (v2h){(_Float16)0.0f, (_Float16)0.0f};
                bm[r][2 * i] = pp[0];
                bm[r][2 * i + 1] = pp[1];
            }
            dd[r] = __half2float(__ushort_as_half((unsigned short)(f[r].x & 0xFFFFu)));
            dmin[r] = __half2float(__ushort_as_half((unsigned short)(f[r].x >> 16)));
        }
        if (s + 1 < a.NSB) {  // the next superblock's copy and codes go out under these products
            stage(s + 1, nxt);
            load_codes(s + 1, f, cw);
        }
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
            const int t = 2 * th + t2;
            const uint8_t *base = cur + t * kPL;
            v4f d[kRW];
#pragma unroll
            for (int r = 0; r < kRW; r++) d[r] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
            // the token tile's operands read in two groups of 8 (the LDS counter's reach) ahead of their products
#pragma unroll
            for (int h = 0; h < 8; h += 4) {
                uint4 ah[4], al[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    ah[u] = *reinterpret_cast<const uint4 *>(base + (h + u) * 2048 + lane * 16);
                    al[u] = *reinterpret_cast<const uint4 *>(base + (h + u) * 2048 + 1024 + lane * 16);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int r = 0; r < kRW; r++) {
                        d[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, ah[u]), bw[r][h + u], d[r], 0,
                                                                      0, 0);
                        d[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, al[u]), bw[r][h + u], d[r], 0,
                                                                      0, 0);
                    }
            }
            uint4 sq = *reinterpret_cast<const uint4 *>(cur + kPT * kPL + t * 512 + (lane & 31) * 16);
            if (g >= 2) sq = make_uint4(0u, 0u, 0u, 0u);
            const uint4 iv = *reinterpret_cast<const uint4 *>(cur + kPT * kPL + kPT * 512 + t * 64 + g * 16);
            const float inv[4] = {__uint_as_float(iv.x), __uint_as_float(iv.y), __uint_as_float(iv.z),
                                  __uint_as_float(iv.w)};
#pragma unroll
            for (int r = 0; r < kRW; r++) {
                v4f dm = {0.0f, 0.0f, 0.0f, 0.0f};
                dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, sq), bm[r], dm, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[r][t2][i] = fmaf(inv[i], fmaf(-dmin[r], dm[i], dd[r] * d[r][i]), acc[r][t2][i]);
            }
        }
    };
    stage(0, st0);
    load_codes(0, f, cw);
    for (int s = 0; s < a.NSB; s += 2) {
        step(s, st0, st1);
        if (s + 1 < a.NSB) step(s + 1, st1, st0);
    }
#pragma unroll
    for (int r = 0; r < kRW; r++)
#pragma unroll
        for (int t2 = 0; t2 < 2; t2++) {
            const int tt = tt0 + 2 * th + t2;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tk = tt * 16 + 4 * g + i, o = rt[r] * 16 + c16;
                if (tt < ntt && rok[r] && o < a.n && tk < a.T) {
                    float v = acc[r][t2][i];
                    if (a.flags & LLMQ_BIAS) v += a.bias[o];
                    if (a.flags & LLMQ_GELU) v = gelu_ref(v);
                    float *dst = a.out + (int64_t)tk * a.ldo + o;
                    if (a.flags & LLMQ_RESID) v += *dst;
                    *dst = v;
                }
            }
        }
}

}  // namespace

int64_t h16_rec_bytes(int64_t T, int64_t K) {
    const int64_t T16 = (T + 15) / 16 * 16, KB = K / 32, NSB = K / 256;
    return T16 * KB * 128 + T16 * NSB * 32 + T16 * NSB * 4;
}

void h16_rec_parts(void *rec, int64_t T, int64_t K, uint8_t **planes, _Float16 **sums, float **inv) {
    const Rec p = rec_parts(rec, T, K);
    *planes = p.planes;
    *sums = p.sums;
    *inv = p.inv;
}

bool gguf_gemm_h16_ok(const llmq_mat *w) {
    return w && w->kind == MAT_GGUF && w->ggml_type == LLMQ_GGML_Q4_K && w->k % 256 == 0;
}

int launch_act_h16(llmq_ctx *ctx, const float *x, int64_t ldx, int64_t T, int64_t K, void *rec) {
    LLMQ_REQUIRE(x && rec && T > 0 && K % 256 == 0, "act_h16: bad arguments");
    LLMQ_REQUIRE(h16_rec_bytes(T, K) < (int64_t)kOOB, "act_h16: record too large");
    const int64_t T16 = (T + 15) / 16 * 16, NSB = K / 256;
    LLMQ_REQUIRE(T16 <= 65535, "act_h16: too many tokens");
    const Rec p = rec_parts(rec, T, K);
    hipLaunchKernelGGL(act_h16_kernel, dim3((unsigned)((NSB + 3) / 4), (unsigned)T16), dim3(256), 0, ctx->stream, x,
                       ldx, (int)T, (int)(K / 32), (int)NSB, p.planes, p.sums, p.inv);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int64_t h16s_rec_bytes(int64_t T, int64_t K) {
    const int64_t T16 = (T + 15) / 16 * 16, KB = K / 32, NSB = K / 256;
    return T16 * KB * 128 + T16 * NSB * 80 + T16 * (K / 16) * 4;
}

int launch_rec_h16s(llmq_ctx *ctx, const float *x, int64_t ldx, int64_t T, int64_t K, const float *gain, void *rec) {
    LLMQ_REQUIRE(x && gain && rec && T > 0 && K % 256 == 0, "rec_h16s: bad arguments");
    const int64_t T16 = (T + 15) / 16 * 16;
    LLMQ_REQUIRE(T16 <= 65535 && h16s_rec_bytes(T, K) < (int64_t)kOOB, "rec_h16s: record too large");
    hipLaunchKernelGGL(rec_h16s_kernel, dim3((unsigned)(K / 256), (unsigned)T16), dim3(256), 0, ctx->stream, x, ldx,
                       (int)T, gain, hs_parts(rec, T, K));
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

namespace {

// Waves of the one-token-tile matmul: a superblock each up to 16, the
// superblocks split evenly over 16 beyond (down at 22: 16 waves of one or
// two measured 1.0162 against 1.0205 ms a batch-16 step for 11 waves of two).
int h16_waves(int64_t NSB) { return (int)std::min<int64_t>(NSB, 16); }

template <bool SIN, int OUT>
void launch_rt1(hipStream_t st, int nw, unsigned nt, unsigned ntt, const HArgs &a) {
    if (nw <= 4)
        hipLaunchKernelGGL((gemm_h16_q4k_kernel<4, 1, SIN, OUT>), dim3(nt, ntt), dim3(256), 0, st, a);
    else if (nw <= 8)
        hipLaunchKernelGGL((gemm_h16_q4k_kernel<8, 1, SIN, OUT>), dim3(nt, ntt), dim3(512), 0, st, a);
    else if (nw <= 11)
        hipLaunchKernelGGL((gemm_h16_q4k_kernel<11, 1, SIN, OUT>), dim3(nt, ntt), dim3(704), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_h16_q4k_kernel<16, 1, SIN, OUT>), dim3(nt, ntt), dim3(1024), 0, st, a);
}

}  // namespace

bool gguf_gemm_h16s_ok(const llmq_mat *w, bool swiglu, int64_t T) {
    if (!gguf_gemm_h16_ok(w) || (T + 15) / 16 >= kPT || w->n % 16) return false;
    return !swiglu || (h16_waves(w->k / 256) <= 8 && w->n % 64 == 0);
}

int launch_gguf_gemm_h16(llmq_ctx *ctx, const llmq_mat *w, const void *rec, int64_t T, float *out, int64_t ldo,
                         const float *bias, int flags, const H16Fuse *fz) {
    const H16Fuse none{};
    if (!fz) fz = &none;
    const bool fused = fz->in_s || fz->out_rec || fz->swiglu;
    LLMQ_REQUIRE(gguf_gemm_h16_ok(w), "gguf_gemm_h16: not a Q4_K matrix with whole superblocks");
    LLMQ_REQUIRE(rec && (out || fz->swiglu) && T > 0, "gguf_gemm_h16: bad arguments");
    LLMQ_REQUIRE(!(flags & LLMQ_BIAS) || bias, "gguf_gemm_h16: LLMQ_BIAS without a bias");
    LLMQ_REQUIRE(!fused || gguf_gemm_h16s_ok(w, fz->swiglu, T), "gguf_gemm_h16: the fused forms take this matrix only "
                 "for fewer than %d token tiles", kPT);
    LLMQ_REQUIRE(!fz->norm || (fz->in_s && (!fz->out_rec || fz->swiglu)),
                 "gguf_gemm_h16: the RMSNorm factor comes with an h16s record and no residual record epilogue");
    LLMQ_REQUIRE(!fz->swiglu || (fz->in_s && fz->out_rec && !flags), "gguf_gemm_h16: SwiGLU takes an h16s record in "
                 "and writes one, nothing else");
    LLMQ_REQUIRE(!fz->out_rec || fz->swiglu || ((flags & LLMQ_RESID) && fz->gain), "gguf_gemm_h16: a record "
                 "epilogue needs LLMQ_RESID and the gain");
    const int64_t T16 = (T + 15) / 16 * 16, KB = w->k / 32, NSB = w->k / 256;
    const int64_t ntc = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 16;
    const int64_t nts = (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16;
    LLMQ_REQUIRE(ntc * 16 < (int64_t)kOOB && h16s_rec_bytes(T, std::max<int64_t>(w->k, w->n)) < (int64_t)kOOB &&
                     T16 <= 65535,
                 "gguf_gemm_h16: operands too large");
    HArgs a{};
    a.codes = w->codes;
    a.codes_bytes = (uint32_t)(ntc * 16);
    a.sb = reinterpret_cast<const uint8_t *>(w->g_sb16);
    a.sb_bytes = (uint32_t)(nts * 16);
    if (fz->in_s) {
        const HSRec p = hs_parts(const_cast<void *>(rec), T, w->k);
        a.planes = p.planes;
        a.sums = reinterpret_cast<const uint8_t *>(p.sums);
        a.sums_bytes = (uint32_t)(T16 * NSB * 64);
        a.exps = reinterpret_cast<const uint8_t *>(p.exps);
        a.exps_bytes = (uint32_t)(T16 * NSB * 16);
        a.ssq = fz->norm ? p.ssq : nullptr;
        a.C = (int)w->k;
        a.eps = fz->eps;
    } else {
        const Rec p = rec_parts(const_cast<void *>(rec), T, w->k);
        a.planes = p.planes;
        a.sums = reinterpret_cast<const uint8_t *>(p.sums);
        a.sums_bytes = (uint32_t)(T16 * NSB * 32);
        a.inv = reinterpret_cast<const uint8_t *>(p.inv);
        a.inv_bytes = (uint32_t)(T16 * NSB * 4);
    }
    a.planes_bytes = (uint32_t)(T16 * KB * 128);
    if (fz->out_rec) {
        a.orec = hs_parts(fz->out_rec, T, fz->swiglu ? w->n / 2 : w->n);
        if (fz->swiglu) a.orec.ssq = nullptr;  // down's input: no norm
        a.ogain = fz->gain;
    }
    a.n = (int)w->n;
    a.KB = (int)KB;
    a.CK = (int)w->CK;
    a.NSB = (int)NSB;
    a.ntiles = (int)w->ntiles;
    a.T = (int)T;
    a.flags = flags;
    a.ldo = ldo;
    a.bias = bias ? bias : out;
    a.out = out;
    const unsigned ntt = (unsigned)(T16 / 16);
    a.stream = ntt == 1;
    const int nw = h16_waves(NSB);
    const unsigned nt = (unsigned)w->ntiles;
    hipStream_t st = ctx->stream;
    if (fz->swiglu)  // two gate and two up tiles a workgroup
        hipLaunchKernelGGL((gemm_h16_q4k_kernel<8, 4, true, 2>), dim3(nt / 4, ntt), dim3(512), 0, st, a);
    else if (fused && fz->in_s)
        fz->out_rec ? launch_rt1<true, 1>(st, nw, nt, ntt, a) : launch_rt1<true, 0>(st, nw, nt, ntt, a);
    else if (fused)
        launch_rt1<false, 1>(st, nw, nt, ntt, a);
    else if (ntt >= (unsigned)kPT)  // prompts: the LDS-staged form
        hipLaunchKernelGGL(gemm_h16_q4k_lds_kernel, dim3((nt + 4 * kRW - 1) / (4 * kRW), (ntt + kPT - 1) / kPT),
                           dim3(512), 0, st, a, (int)ntt);
    // wide matrices (gate / up): 4 row tiles a workgroup share the record
    // loads (one round of 176 workgroups at 11264 rows; 1, 2 and 4 tiles
    // measured 10.5, 11.9 and 10.1 us at 16 tokens)
    else if (nw <= 8 && w->ntiles >= 512)
        hipLaunchKernelGGL((gemm_h16_q4k_kernel<8, 4, false, 0>), dim3((nt + 3) / 4, ntt), dim3(512), 0, st, a);
    else
        launch_rt1<false, 0>(st, nw, nt, ntt, a);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
