// GGUF block formats on the GPU: GGUFMatrix (gguf.mojo:344-511) with its
// float-activation decode GEMV (matmul_rows T == 1 / linear_team OUT_MAJOR,
// kernels.mojo:301-312, 817-826) and the block decoders of gguf.mojo:178-297.
//
// Blocks are uploaded as stored: every code, scale and min bit is kept; only
// their placement changes, into the row-tile layout of common.h.  Per row,
// the codes of each 32 weights (16 for Q8_0) form one 16-byte chunk in
// natural order (dword i, nibble / byte j = weight 8i + j / 4i + j), chunk-
// major within a 16-row tile; fields that are not codes go to arrays indexed
// [tile][chunk or superblock][16 rows]:
//
//   Q4_0  chunk = block          meta16[c] = d
//   Q4_1  chunk = block          meta32[c] = d | m << 16
//   Q8_0  chunk = half block     meta16[c / 2] = d
//   Q4_K  chunk = sub-block      sb16[sb] = d | dmin << 16 | 12 scale bytes
//   Q5_K  as Q4_K                + bits32[c]: the 5th bit of weight n in bit n
//   Q6_K  chunk = 2 sub-blocks   + bits64[c]: high 2 bits of weight n in bits 2n..2n+1;
//                                  sb16[sb] = the 16 int8 scales, meta16[sb] = d
//
// The device bytes per row equal the reference's row_bytes (gguf.mojo:371).
//
// Arithmetic: per chunk the kernel forms a = sum x*u over the chunk's codes
// u (float32 FMAs) and applies the block's scale and offset once:
//   Q4_0  d * (a - 8 S)        Q4_1  d * a + m * S        Q8_0  d * (a' - 128 S)  (a' over q + 128)
//   Q4_K  d*sc * a - dmin*m * S          Q5_K  the same with u = lo4 + 16 * bit5
//   Q6_K  d*sc * (a - 32 S) per 16 weights, u = lo4 + 16 * hi2
// with S = sum x over the chunk (or half chunk), computed once per token.
// This equals the reference's per-weight dequantize-then-FMA up to float32
// rounding.
#include <string.h>

#include <vector>

#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kSteps = 8;

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)bits)); }

struct GgufArgs {
    const uint4 *codes;
    const uint16_t *meta16;
    const uint32_t *meta32;
    const uint32_t *bits32;
    const uint2 *bits64;
    const uint4 *sb16;
    int n, K, ntiles, CK, NSB, ks, flags;
    const float *x, *bias;
    float *out;
    ArgmaxPart *amax;
};

// Weights per chunk and chunks per superblock of a type.
template <int TYPE>
struct Fmt {
    static constexpr int WPC = TYPE == LLMQ_GGML_Q8_0 ? 16 : 32;
    static constexpr int CPS =
        (TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K || TYPE == LLMQ_GGML_Q6_K) ? 8 : 1;
};

// k_scale_min (gguf.mojo:205-221) over the 12 scale bytes s0..s2 (dwords).
__device__ __forceinline__ void k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &sc, int &mn) {
    auto byte = [&](int i) -> int {
        const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
        return (int)((w >> (8 * (i & 3))) & 255u);
    };
    if (j < 4) {
        sc = byte(j) & 63;
        mn = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Byte k of v as float (selects v_cvt_f32_ubyte<k>).
template <int K>
__device__ __forceinline__ float ubyte(uint32_t v) { return (float)((v >> (8 * K)) & 255u); }

// sum of x[e] * u_e over a 4-bit chunk d (natural nibble order), x in LDS.
__device__ __forceinline__ float dot_nibbles(uint32_t w, const float *x) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    float a = 0.0f;
    a = fmaf(x[0], ubyte<0>(lo), a);
    a = fmaf(x[1], ubyte<0>(hi), a);
    a = fmaf(x[2], ubyte<1>(lo), a);
    a = fmaf(x[3], ubyte<1>(hi), a);
    a = fmaf(x[4], ubyte<2>(lo), a);
    a = fmaf(x[5], ubyte<2>(hi), a);
    a = fmaf(x[6], ubyte<3>(lo), a);
    a = fmaf(x[7], ubyte<3>(hi), a);
    return a;
}

// sum of x[e] * ((bits >> (S * e)) & M) over 8 weights (S = 1 or 2).
template <int S>
__device__ __forceinline__ float dot_bits(uint32_t bits, const float *x) {
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaf(x[e], (float)((bits >> (S * e)) & ((1u << S) - 1)), a);
    return a;
}

template <int TYPE, bool LOOP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void gguf_gemv_kernel(GgufArgs a) {
    using F = Fmt<TYPE>;
    constexpr int WPC = F::WPC;
    extern __shared__ __align__(16) float xs[];  // [K] activations, then [K / 16] sums of 16
    __shared__ float part[4 * 16];
    __shared__ ArgmaxPart s_best[4];
    float *xsum16 = xs + a.K;
    const int CK = a.CK;
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
    const int oc = row_ok ? o : 0;
    const float e_bias = a.bias[oc];
    const float e_res = a.out[oc];

    // Activations and their per-16 sums into LDS (issued first).
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
    float4 xv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = tid + kThreads * i;
        xv[i] = x4[q < a.K / 4 ? q : 0];
    }
    __builtin_amdgcn_sched_barrier(0);

    const int tile_c = tile_ok ? tile : 0;
    const uint32_t code_lane = (uint32_t)tile_c * CK * 16u + (uint32_t)j * 16u + (uint32_t)r;
    const uint32_t meta_lane = (uint32_t)tile_c * CK * 16u + (uint32_t)r;
    const uint32_t sb_lane = (uint32_t)tile_c * a.NSB * 16u + (uint32_t)r;
    uint4 wc[kSteps];
    uint32_t wm[kSteps];   // meta16 / meta32 / bits32
    uint2 wb[kSteps];      // bits64
    uint4 wsb[kSteps];     // superblock fields
    uint32_t wd6[kSteps];  // Q6_K d
    auto fetch = [&](int sb) {
#pragma unroll
        for (int u = 0; u < kSteps; u++) {
            const uint32_t s = (uint32_t)(sb + u);
            const uint32_t c = 4u * s + (uint32_t)j;
            wc[u] = a.codes[code_lane + s * 64u];
            if (TYPE == LLMQ_GGML_Q4_0) wm[u] = a.meta16[meta_lane + c * 16u];
            if (TYPE == LLMQ_GGML_Q8_0) wm[u] = a.meta16[meta_lane + (c >> 1) * 16u];
            if (TYPE == LLMQ_GGML_Q4_1) wm[u] = a.meta32[meta_lane + c * 16u];
            if (TYPE == LLMQ_GGML_Q5_K) wm[u] = a.bits32[meta_lane + c * 16u];
            if (TYPE == LLMQ_GGML_Q6_K) {
                wb[u] = a.bits64[meta_lane + c * 16u];
                wd6[u] = a.meta16[sb_lane + (c >> 3) * 16u];
            }
            if (F::CPS == 8) wsb[u] = a.sb16[sb_lane + (c >> 3) * 16u];
        }
    };
    __builtin_amdgcn_sched_barrier(0);
    fetch(s0);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = tid + kThreads * i;
        if (q < a.K / 4) reinterpret_cast<float4 *>(xs)[q] = xv[i];
    }
    for (int q = tid + kThreads * 4; q < a.K / 4; q += kThreads) reinterpret_cast<float4 *>(xs)[q] = x4[q];
    lds_barrier();
    for (int g = tid; g < a.K / 16; g += kThreads) {
        const float4 *p = reinterpret_cast<const float4 *>(xs + 16 * g);
        float sacc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = p[i];
            sacc += ((v.x + v.y) + v.z) + v.w;
        }
        xsum16[g] = sacc;
    }
    lds_barrier();

    float acc = 0.0f;
    for (int sbat = s0; sbat < s1; sbat += kSteps) {
        if (LOOP && sbat != s0) {
            __builtin_amdgcn_sched_barrier(0);
            fetch(sbat);
        }
#pragma unroll
        for (int u = 0; u < kSteps; u++) {
            const int ss = sbat + u;
            const bool ok = tile_ok && ss < s1 && 4 * ss + j < CK;
            const int c = ok ? 4 * ss + j : 0;
            const float *xc = xs + c * WPC;
            const uint4 d = wc[u];
            float contrib;
            if (TYPE == LLMQ_GGML_Q8_0) {
                // bytes as q + 128 (xor 0x80), then subtract 128 * S
                const uint32_t w4[4] = {d.x ^ 0x80808080u, d.y ^ 0x80808080u, d.z ^ 0x80808080u, d.w ^ 0x80808080u};
                float aa = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    aa = fmaf(xc[4 * i], ubyte<0>(w4[i]), aa);
                    aa = fmaf(xc[4 * i + 1], ubyte<1>(w4[i]), aa);
                    aa = fmaf(xc[4 * i + 2], ubyte<2>(w4[i]), aa);
                    aa = fmaf(xc[4 * i + 3], ubyte<3>(w4[i]), aa);
                }
                contrib = h2f(wm[u]) * (aa - 128.0f * xsum16[c]);
            } else {
                const float a0 = dot_nibbles(d.x, xc), a1 = dot_nibbles(d.y, xc + 8);
                const float a2 = dot_nibbles(d.z, xc + 16), a3 = dot_nibbles(d.w, xc + 24);
                const float SA = xsum16[2 * c], SB = xsum16[2 * c + 1];
                if (TYPE == LLMQ_GGML_Q4_0) {
                    contrib = h2f(wm[u]) * (((a0 + a1) + (a2 + a3)) - 8.0f * (SA + SB));
                } else if (TYPE == LLMQ_GGML_Q4_1) {
                    contrib = h2f(wm[u]) * ((a0 + a1) + (a2 + a3)) + h2f(wm[u] >> 16) * (SA + SB);
                } else if (TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K) {
                    float al = (a0 + a1) + (a2 + a3);
                    if (TYPE == LLMQ_GGML_Q5_K) {
                        const uint32_t b = wm[u];
                        al += 16.0f * ((dot_bits<1>(b, xc) + dot_bits<1>(b >> 8, xc + 8)) +
                                       (dot_bits<1>(b >> 16, xc + 16) + dot_bits<1>(b >> 24, xc + 24)));
                    }
                    const uint4 f = wsb[u];
                    int sc, mn;
                    k_scale_min(f.y, f.z, f.w, c & 7, sc, mn);
                    const float dd = h2f(f.x) * (float)sc, mm = h2f(f.x >> 16) * (float)mn;
                    contrib = dd * al - mm * (SA + SB);
                } else {  // Q6_K: two 16-weight sub-blocks with their own int8 scales
                    const uint2 hb = wb[u];
                    const float hA = (dot_bits<2>(hb.x, xc) + dot_bits<2>(hb.x >> 16, xc + 8));
                    const float hB = (dot_bits<2>(hb.y, xc + 16) + dot_bits<2>(hb.y >> 16, xc + 24));
                    const uint4 f = wsb[u];
                    const int si = 2 * (c & 7);  // scale index of the first half
                    const uint32_t sw = si < 4 ? f.x : (si < 8 ? f.y : (si < 12 ? f.z : f.w));
                    const float scA = (float)(int8_t)((sw >> (8 * (si & 3))) & 255u);
                    const float scB = (float)(int8_t)((sw >> (8 * ((si + 1) & 3))) & 255u);
                    const float dq = h2f(wd6[u]);
                    contrib = dq * (scA * ((a0 + a1) + 16.0f * hA - 32.0f * SA) +
                                    scB * ((a2 + a3) + 16.0f * hB - 32.0f * SB));
                }
            }
            acc += ok ? contrib : 0.0f;
            __builtin_amdgcn_sched_barrier(0);
        }
        if (!LOOP) break;
    }

    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    if (a.ks > 1) {
        if (j == 0) part[wid * 16 + r] = acc;
        lds_barrier();
        if (kpart == 0) {
            float v = 0.0f;
            for (int q = 0; q < a.ks; q++) v += part[(wid + q) * 16 + r];
            acc = v;
        }
    }
    float best_v = -INFINITY;
    int best_i = 0x7fffffff;
    if (kpart == 0 && row_ok) {
        float v = acc;
        if (a.flags & LLMQ_BIAS) v += e_bias;
        if (a.flags & LLMQ_GELU) {
            const float sg = 0.7978845608028654f;
            float t = 0.044715f * v;
            t = t * v;
            t = t * v;
            v = (0.5f * v) * (1.0f + tanhf(sg * (v + t)));
        }
        if (a.flags & LLMQ_RESID) v += e_res;
        if (j == 0) a.out[o] = v;
        best_v = v;
        best_i = o;
    }
    if (a.amax) {
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
                ArgmaxPart cc = s_best[q];
                if (cc.v > b.v || (cc.v == b.v && cc.idx < b.idx)) b = cc;
            }
            a.amax[blockIdx.x] = b;
        }
    }
}

// Dequantize one row into float32 (GGUFMatrix.dequant_row, gguf.mojo:381-382).
template <int TYPE>
__global__ void gguf_dequant_row_kernel(GgufArgs a, int64_t row, float *dst) {
    using F = Fmt<TYPE>;
    const int64_t tile = row / 16, r = row % 16;
    for (int k = threadIdx.x; k < a.K; k += blockDim.x) {
        const int c = k / F::WPC, e = k % F::WPC;
        const uint4 d = a.codes[((size_t)tile * a.CK + c) * 16 + r];
        const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
        const size_t mi = ((size_t)tile * a.CK + c) * 16 + r;
        const size_t sbi = ((size_t)tile * a.NSB + c / F::CPS) * 16 + r;
        float v;
        if (TYPE == LLMQ_GGML_Q8_0) {
            const int q = (int)(int8_t)((dw[e >> 2] >> (8 * (e & 3))) & 255u);
            v = h2f(a.meta16[((size_t)tile * a.CK + (c >> 1)) * 16 + r]) * (float)q;
        } else {
            int u = (int)((dw[e >> 3] >> (4 * (e & 7))) & 15u);
            if (TYPE == LLMQ_GGML_Q4_0) {
                v = ((float)u - 8.0f) * h2f(a.meta16[mi]);
            } else if (TYPE == LLMQ_GGML_Q4_1) {
                const uint32_t m = a.meta32[mi];
                v = h2f(m) * (float)u + h2f(m >> 16);
            } else if (TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K) {
                if (TYPE == LLMQ_GGML_Q5_K) u |= (int)((a.bits32[mi] >> e) & 1u) << 4;
                const uint4 f = a.sb16[sbi];
                int sc, mn;
                k_scale_min(f.y, f.z, f.w, c & 7, sc, mn);
                v = (h2f(f.x) * (float)sc) * (float)u - h2f(f.x >> 16) * (float)mn;
            } else {
                const uint2 hb = a.bits64[mi];
                const uint32_t hw = e < 16 ? hb.x : hb.y;
                u |= (int)((hw >> (2 * (e & 15))) & 3u) << 4;
                const uint4 f = a.sb16[sbi];
                const int si = 2 * (c & 7) + (e >= 16);
                const uint32_t sw = si < 4 ? f.x : (si < 8 ? f.y : (si < 12 ? f.z : f.w));
                const float sc = (float)(int8_t)((sw >> (8 * (si & 3))) & 255u);
                v = (h2f(a.meta16[sbi]) * sc) * ((float)u - 32.0f);
            }
        }
        dst[k] = v;
    }
}

int gguf_block_size(int t) {
    if (t == LLMQ_GGML_Q4_0 || t == LLMQ_GGML_Q4_1 || t == LLMQ_GGML_Q8_0) return 32;
    if (t == LLMQ_GGML_Q4_K || t == LLMQ_GGML_Q5_K || t == LLMQ_GGML_Q6_K) return 256;
    return 0;
}
int gguf_block_bytes(int t) {
    switch (t) {
    case LLMQ_GGML_Q4_0: return 18;
    case LLMQ_GGML_Q4_1: return 20;
    case LLMQ_GGML_Q8_0: return 34;
    case LLMQ_GGML_Q4_K: return 144;
    case LLMQ_GGML_Q5_K: return 176;
    case LLMQ_GGML_Q6_K: return 210;
    default: return 0;
    }
}

GgufArgs make_args(const llmq_mat *m) {
    GgufArgs a{};
    a.codes = reinterpret_cast<const uint4 *>(m->codes);
    a.meta16 = reinterpret_cast<const uint16_t *>(m->g_meta16);
    a.meta32 = reinterpret_cast<const uint32_t *>(m->g_meta32);
    a.bits32 = reinterpret_cast<const uint32_t *>(m->g_bits32);
    a.bits64 = reinterpret_cast<const uint2 *>(m->g_bits64);
    a.sb16 = reinterpret_cast<const uint4 *>(m->g_sb16);
    a.n = (int)m->n;
    a.K = (int)m->k;
    a.ntiles = (int)m->ntiles;
    a.CK = (int)m->CK;
    a.NSB = (int)m->NG;
    return a;
}

template <int TYPE>
void launch_type(llmq_ctx *ctx, const GgufArgs &a, dim3 grid, size_t lds, bool loop) {
    if (loop)
        hipLaunchKernelGGL((gguf_gemv_kernel<TYPE, true>), grid, dim3(kThreads), lds, ctx->stream, a);
    else
        hipLaunchKernelGGL((gguf_gemv_kernel<TYPE, false>), grid, dim3(kThreads), lds, ctx->stream, a);
}

}  // namespace

int gguf_is_supported(int t) { return gguf_block_size(t) != 0; }

// GGUFMatrix(data, kind, rows, cols): re-place the blocks of a [rows][row
// bytes] buffer into the device arrays (see the header comment).
int gguf_upload(llmq_ctx *ctx, llmq_mat *m, int t, const uint8_t *blocks, int64_t rows, int64_t cols) {
    const int bs = gguf_block_size(t), bb = gguf_block_bytes(t);
    LLMQ_REQUIRE(bs > 0, "from_gguf: unsupported type %d", t);
    LLMQ_REQUIRE(rows > 0 && cols > 0 && cols % bs == 0, "from_gguf: cols %lld not a multiple of %d", (long long)cols,
                 bs);
    const int wpc = t == LLMQ_GGML_Q8_0 ? 16 : 32;
    m->kind = MAT_GGUF;
    m->ggml_type = t;
    m->n = rows;
    m->k = cols;
    m->group = t == LLMQ_GGML_Q6_K ? 256 : 32;
    m->row_bytes = cols / bs * bb;
    m->ntiles = (rows + 15) / 16;
    m->CK = cols / wpc;
    m->NG = (t == LLMQ_GGML_Q4_K || t == LLMQ_GGML_Q5_K || t == LLMQ_GGML_Q6_K) ? cols / 256 : 0;  // superblocks
    const int64_t ntc = (m->ntiles * m->CK + LLMQ_PAD_CHUNKS) * 16;   // per-chunk entries (with padding)
    const int64_t nts = (m->ntiles * m->NG + LLMQ_PAD_CHUNKS) * 16;   // per-superblock entries
    std::vector<uint8_t> codes((size_t)ntc * 16, 0);
    std::vector<uint16_t> meta16;
    std::vector<uint32_t> meta32, bits32;
    std::vector<uint64_t> bits64;
    std::vector<uint8_t> sb16;
    if (t == LLMQ_GGML_Q4_0 || t == LLMQ_GGML_Q8_0) meta16.assign((size_t)ntc, 0);
    if (t == LLMQ_GGML_Q6_K) meta16.assign((size_t)nts, 0);
    if (t == LLMQ_GGML_Q4_1) meta32.assign((size_t)ntc, 0);
    if (t == LLMQ_GGML_Q5_K) bits32.assign((size_t)ntc, 0);
    if (t == LLMQ_GGML_Q6_K) bits64.assign((size_t)ntc, 0);
    if (m->NG) sb16.assign((size_t)nts * 16, 0);
    auto u16 = [](const uint8_t *p) -> uint32_t { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); };
    for (int64_t o = 0; o < rows; o++) {
        const int64_t tile = o / 16, r = o % 16;
        const uint8_t *row = blocks + o * m->row_bytes;
        auto chunk_at = [&](int64_t c) -> uint8_t * { return codes.data() + ((tile * m->CK + c) * 16 + r) * 16; };
        auto put4 = [&](int64_t c, int e, int u) { chunk_at(c)[e >> 1] |= (uint8_t)((u & 15) << (4 * (e & 1))); };
        auto cidx = [&](int64_t c) { return (size_t)((tile * m->CK + c) * 16 + r); };
        auto sidx = [&](int64_t sb) { return (size_t)((tile * m->NG + sb) * 16 + r); };
        for (int64_t b = 0; b < cols / bs; b++) {
            const uint8_t *p = row + b * bb;
            if (t == LLMQ_GGML_Q4_0 || t == LLMQ_GGML_Q4_1) {  // gguf.mojo:178-193
                const uint8_t *q = p + (t == LLMQ_GGML_Q4_0 ? 2 : 4);
                for (int i = 0; i < 16; i++) {
                    put4(b, i, q[i] & 15);
                    put4(b, 16 + i, q[i] >> 4);
                }
                if (t == LLMQ_GGML_Q4_0)
                    meta16[cidx(b)] = (uint16_t)u16(p);
                else
                    meta32[cidx(b)] = u16(p) | (u16(p + 2) << 16);
            } else if (t == LLMQ_GGML_Q8_0) {  // gguf.mojo:196-202
                for (int h = 0; h < 2; h++) memcpy(chunk_at(2 * b + h), p + 2 + 16 * h, 16);
                meta16[cidx(b)] = (uint16_t)u16(p);
            } else if (t == LLMQ_GGML_Q4_K || t == LLMQ_GGML_Q5_K) {  // gguf.mojo:224-268
                const bool five = t == LLMQ_GGML_Q5_K;
                uint8_t *f = sb16.data() + sidx(b) * 16;
                memcpy(f, p, 4);        // d, dmin
                memcpy(f + 4, p + 4, 12);  // 6-bit scales and mins
                const uint8_t *qs = p + (five ? 48 : 16), *qh = p + 16;
                for (int j = 0; j < 4; j++)
                    for (int l = 0; l < 32; l++) {
                        const int lo = qs[32 * j + l] & 15, hi = qs[32 * j + l] >> 4;
                        const int64_t c0 = 8 * b + 2 * j, c1 = c0 + 1;  // sub-blocks 2j, 2j+1
                        put4(c0, l, lo);
                        put4(c1, l, hi);
                        if (five) {
                            bits32[cidx(c0)] |= (uint32_t)((qh[l] >> (2 * j)) & 1) << l;
                            bits32[cidx(c1)] |= (uint32_t)((qh[l] >> (2 * j + 1)) & 1) << l;
                        }
                    }
            } else {  // Q6_K, gguf.mojo:271-297
                for (int n = 0; n < 2; n++)
                    for (int l = 0; l < 32; l++) {
                        const uint8_t ql0 = p[64 * n + l], ql1 = p[64 * n + 32 + l], qh = p[128 + 32 * n + l];
                        const int q[4] = {ql0 & 15, ql1 & 15, ql0 >> 4, ql1 >> 4};
                        for (int k = 0; k < 4; k++) {
                            const int w = 128 * n + 32 * k + l;  // weight within the superblock
                            const int64_t c = 8 * b + w / 32;
                            const int e = w % 32;
                            put4(c, e, q[k]);
                            bits64[cidx(c)] |= (uint64_t)((qh >> (2 * k)) & 3) << (2 * e);
                        }
                    }
                memcpy(sb16.data() + sidx(b) * 16, p + 192, 16);
                meta16[sidx(b)] = (uint16_t)u16(p + 208);
            }
        }
    }
    auto up = [&](void **dptr, const void *src, size_t bytes) -> int {
        if (!bytes) return LLMQ_OK;
        if (hipMalloc(dptr, bytes) != hipSuccess) return llmq_set_error(LLMQ_ENOMEM, "from_gguf: %zu bytes", bytes);
        if (hipMemcpyAsync(*dptr, src, bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
            return llmq_set_error(LLMQ_EHIP, "from_gguf: copy failed");
        return LLMQ_OK;
    };
    int rc;
    if ((rc = up((void **)&m->codes, codes.data(), codes.size())) != LLMQ_OK) return rc;
    if ((rc = up(&m->g_meta16, meta16.data(), meta16.size() * 2)) != LLMQ_OK) return rc;
    if ((rc = up(&m->g_meta32, meta32.data(), meta32.size() * 4)) != LLMQ_OK) return rc;
    if ((rc = up(&m->g_bits32, bits32.data(), bits32.size() * 4)) != LLMQ_OK) return rc;
    if ((rc = up(&m->g_bits64, bits64.data(), bits64.size() * 8)) != LLMQ_OK) return rc;
    if ((rc = up(&m->g_sb16, sb16.data(), sb16.size())) != LLMQ_OK) return rc;
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

static int pick_ks_gguf(const llmq_mat *w) {
    if (const char *e = getenv("LLMQ_GEMV_KS")) {
        int v = atoi(e);
        if (v == 1 || v == 2 || v == 4) return v;
    }
    if (w->ntiles <= 1024) return 4;
    const int64_t S = (w->CK + 3) / 4;
    for (int ks = 1; ks < 4; ks *= 2)
        if ((S + ks - 1) / ks <= kSteps) return ks;
    return 4;
}

int gguf_num_parts(const llmq_mat *w) {
    const int tpw = 4 / pick_ks_gguf(w);
    return (int)((w->ntiles + tpw - 1) / tpw);
}

int launch_gguf_gemv(llmq_ctx *ctx, const llmq_mat *w, const float *x, float *out, const float *bias, int flags,
                     ArgmaxPart *amax, int amax_cap) {
    LLMQ_REQUIRE(w && w->kind == MAT_GGUF, "gguf_gemv: not a GGUF matrix");
    LLMQ_REQUIRE(x && out, "gguf_gemv: null pointer");
    LLMQ_REQUIRE(!(flags & LLMQ_BIAS) || bias, "gguf_gemv: LLMQ_BIAS without a bias");
    const size_t lds = sizeof(float) * ((size_t)w->k + w->k / 16);
    // dynamic LDS plus the kernel's static part (partials, argmax slots) within 64 KiB
    LLMQ_REQUIRE(lds <= 64 * 1024 - 1024, "gguf_gemv: reduction axis %lld too long", (long long)w->k);
    LLMQ_REQUIRE(w->k % 16 == 0, "gguf_gemv: cols must be a multiple of 16");
    GgufArgs a = make_args(w);
    a.ks = pick_ks_gguf(w);
    a.flags = flags;
    a.x = x;
    a.bias = bias ? bias : out;
    a.out = out;
    a.amax = amax;
    const int tpw = 4 / a.ks;
    dim3 grid((unsigned)((w->ntiles + tpw - 1) / tpw));
    LLMQ_REQUIRE(!amax || (int)grid.x <= amax_cap, "gguf_gemv: argmax capacity");
    const int64_t S = (w->CK + 3) / 4;
    const bool loop = (S + a.ks - 1) / a.ks > kSteps;
    switch (w->ggml_type) {
    case LLMQ_GGML_Q4_0: launch_type<LLMQ_GGML_Q4_0>(ctx, a, grid, lds, loop); break;
    case LLMQ_GGML_Q4_1: launch_type<LLMQ_GGML_Q4_1>(ctx, a, grid, lds, loop); break;
    case LLMQ_GGML_Q8_0: launch_type<LLMQ_GGML_Q8_0>(ctx, a, grid, lds, loop); break;
    case LLMQ_GGML_Q4_K: launch_type<LLMQ_GGML_Q4_K>(ctx, a, grid, lds, loop); break;
    case LLMQ_GGML_Q5_K: launch_type<LLMQ_GGML_Q5_K>(ctx, a, grid, lds, loop); break;
    case LLMQ_GGML_Q6_K: launch_type<LLMQ_GGML_Q6_K>(ctx, a, grid, lds, loop); break;
    default: return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf_gemv: type %d", w->ggml_type);
    }
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_gguf_dequant_row(llmq_ctx *ctx, const llmq_mat *w, int64_t row, float *dst) {
    GgufArgs a = make_args(w);
    switch (w->ggml_type) {
    case LLMQ_GGML_Q4_0: hipLaunchKernelGGL(gguf_dequant_row_kernel<LLMQ_GGML_Q4_0>, dim3(1), dim3(256), 0, ctx->stream, a, row, dst); break;
    case LLMQ_GGML_Q4_1: hipLaunchKernelGGL(gguf_dequant_row_kernel<LLMQ_GGML_Q4_1>, dim3(1), dim3(256), 0, ctx->stream, a, row, dst); break;
    case LLMQ_GGML_Q8_0: hipLaunchKernelGGL(gguf_dequant_row_kernel<LLMQ_GGML_Q8_0>, dim3(1), dim3(256), 0, ctx->stream, a, row, dst); break;
    case LLMQ_GGML_Q4_K: hipLaunchKernelGGL(gguf_dequant_row_kernel<LLMQ_GGML_Q4_K>, dim3(1), dim3(256), 0, ctx->stream, a, row, dst); break;
    case LLMQ_GGML_Q5_K: hipLaunchKernelGGL(gguf_dequant_row_kernel<LLMQ_GGML_Q5_K>, dim3(1), dim3(256), 0, ctx->stream, a, row, dst); break;
    case LLMQ_GGML_Q6_K: hipLaunchKernelGGL(gguf_dequant_row_kernel<LLMQ_GGML_Q6_K>, dim3(1), dim3(256), 0, ctx->stream, a, row, dst); break;
    default: return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf dequant: type %d", w->ggml_type);
    }
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
