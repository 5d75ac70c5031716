// One-token GEMV over GGUF blocks with float activations: GGUFMatrix.dot_row
// (gguf.mojo:389-417, the block decoders of gguf.mojo:178-297 with DOT=True)
// as driven by matmul_rows / linear_team's OUT_MAJOR branch for T == 1
// (kernels.mojo:285-312, 817-826), with store_out's bias / GELU / residual.
//
// Device layout (gguf.hip): per 16-row tile, each row's codes in 16-byte
// chunks (32 4-bit codes, or 16 int8 codes for Q8_0), chunk-major; side
// arrays per chunk (Q5_K 5th bits, Q6_K high bits), per block (Q4_0 / Q4_1 /
// Q8_0 d, m) and per 256-weight superblock (K-quant d, dmin, 6-bit scales;
// Q6_K int8 scales and d), each indexed [tile][index][16 rows].  The global
// index of chunk c of tile t is t * CK + c, and block / superblock indices
// are that >> 1 (Q8_0) or >> 3 (K-quants), so every field a wave needs is
// one contiguous run even when the wave crosses a tile boundary.
//
// Arithmetic per chunk: a = sum x*u over its codes u (float32 FMAs on the
// activations in LDS), with the block's scale and offset applied once:
//   Q4_0  d * (a - 8 S)        Q4_1  d * a + m * S        Q8_0  d * (a' - 128 S)  (a' over q + 128)
//   Q4_K  d*sc * a - dmin*m * S          Q5_K  the same with u = lo4 + 16 * bit5
//   Q6_K  d*sc * (a - 32 S) per 16 weights, u = lo4 + 16 * hi2
// with S = sum x over the chunk (or half chunk) from a per-16 table.  This
// equals the reference's dequantize-then-FMA up to float32 rounding.
//
// Work mapping, loads and reductions follow the one-token integer kernel
// (gemv1.hip): one 16-wave workgroup per CU with a contiguous run of whole
// row tiles (4-wave workgroups of one tile for small matrices), a wave step
// = 16 rows x 4 consecutive chunks read as one contiguous KiB, every load of
// a wave issued up front as buffer loads (no-data lanes read past the extent:
// zeros, no traffic), per-wave fields staged through LDS, fixed-order sums.
#include "common.h"

namespace {

constexpr int kMaxSteps = 8;   // code steps a wave holds (16 for Q8_0, whose decode needs fewer registers)
constexpr int kMaxTiles = 4;
constexpr uint32_t kOOB = 0x80000000u;

struct G1Args {
    const uint8_t *codes, *meta, *bits, *sb, *d6;
    uint32_t codes_bytes, meta_bytes, bits_bytes, sb_bytes, d6_bytes;
    int n, K, ntiles, CK, tmax, flags;
    int NG, cpg_shift;   // QuantMatrix: group of chunk c of tile t is t * NG + (c >> cpg_shift)
    const float *x, *bias;
    float *out;
    ArgmaxPart *amax;
    const float *rms_g;  // optional RMSNorm gain: x -> x / sqrt(mean(x^2) + eps) * g first
    float rms_eps;
    int swiglu;          // x holds [gate | up] of 2K floats: the row is silu(gate) * up
    const float *ln_w, *ln_b;  // optional LayerNorm (eps 1e-5) of the row first
    const float *apart;        // attention splits to combine into the row (AC kernels)
    const int *astate;         // decode position: astate[0] + 1 positions
    int asplit, ans_max;       // positions a split covers, splits a head in apart
};

// Attention splits: per head, ans_max split records of kAPart floats (the
// layout common.h fixes; a head's 64 sums are 16 float4 units).
constexpr int kAPart = kLlmqSplitRec;
constexpr int kACMax = kLlmqMaxSplits;  // splits an AC kernel combines
static_assert(kLlmqSplitHD == 64, "the staging maps a row unit u to head u >> 4 (16 float4 units a head)");
constexpr int kACUnits = 2;  // float4 row units a thread combines (K <= 2 * 4 * threads)

// silu(g) * u per lane of two activation vectors (llama.hip's swiglu).
__device__ __forceinline__ uint4 swiglu4(uint4 g, uint4 u) {
    auto f = [](uint32_t gb, uint32_t ub) {
        const float x = __uint_as_float(gb), y = __uint_as_float(ub);
        return __float_as_uint((x / (1.0f + expf(-x))) * y);
    };
    return make_uint4(f(g.x, u.x), f(g.y, u.y), f(g.z, u.z), f(g.w, u.w));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
// Streamed weight codes: non-temporal (no reuse expected; the caches keep
// the activations instead).
__device__ __forceinline__ uint4 bload16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2);
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

__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)bits)); }

// Type traits: weights per chunk, and the staged per-wave fields (global
// chunk index >> shift, bytes per (index, row)).
// QuantMatrix (kQmFloat4 / kQmFloat8): its f16 scales take the place of the
// meta array and its u8 zero points that of the second staged array; the
// group index comes from the matrix's own group size (META_SHIFT is the
// smallest one, a 32-weight group, for the staging bound).
template <int TYPE>
struct T1 {
    static constexpr bool QM = TYPE == kQmFloat4 || TYPE == kQmFloat8;
    static constexpr bool KQ = TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K || TYPE == LLMQ_GGML_Q6_K;
    static constexpr bool BYTES = TYPE == LLMQ_GGML_Q8_0 || TYPE == kQmFloat8;  // 16 one-byte codes per chunk
    static constexpr int WPC = BYTES ? 16 : 32;
    static constexpr int META_SHIFT = BYTES ? 1 : (KQ ? 3 : 0);
    // bytes per (index, row) of the main staged array: meta16 / meta32 / sb16
    static constexpr int META_ESZ = KQ ? 16 : (TYPE == LLMQ_GGML_Q4_1 ? 4 : 2);
    static constexpr int BITS_ESZ = TYPE == LLMQ_GGML_Q5_K ? 4 : (TYPE == LLMQ_GGML_Q6_K ? 8 : 0);  // per chunk
    // bytes per (index, row) of the second staged array: Q6_K's d, QuantMatrix's zero points
    static constexpr int D6_ESZ = TYPE == LLMQ_GGML_Q6_K ? 2 : (QM ? 1 : 0);
};

// Staged bytes per wave: the most indices a wave's 4 * STEPS chunks can
// touch (plus one for a run that starts mid-block), 16 rows each, in whole
// 1 KiB loads.
template <int TYPE, int STEPS>
struct Stage {
    using T = T1<TYPE>;
    static constexpr int IDX = (4 * STEPS >> T::META_SHIFT) + 2;
    static constexpr int LOADS = (IDX * 16 * T::META_ESZ + 1023) / 1024;
    static constexpr int D6_LOADS = (IDX * 16 * T::D6_ESZ + 1023) / 1024;
};

// k_scale_min (gguf.mojo:205-221) of sub-block j over the 12 scale bytes
// s0..s2 (dwords), branch-free.
__device__ __forceinline__ void k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j, int &sc, int &mn) {
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    const uint32_t b0 = (s0 >> sh) & 255u, b1 = (s1 >> sh) & 255u, b2 = (s2 >> sh) & 255u;
    // j < 4: bytes j (b0) and j + 4 (b1); j >= 4: bytes j + 4 (b2), j - 4 (b0), j (b1)
    const int sc_lo = (int)(b0 & 63u), mn_lo = (int)(b1 & 63u);
    const int sc_hi = (int)((b2 & 15u) | ((b0 >> 6) << 4)), mn_hi = (int)((b2 >> 4) | ((b1 >> 6) << 4));
    sc = j < 4 ? sc_lo : sc_hi;
    mn = j < 4 ? mn_lo : mn_hi;
}

// Byte k of v as float (v_cvt_f32_ubyte<k>).
template <int K>
__device__ __forceinline__ float ub(uint32_t v) { return (float)((v >> (8 * K)) & 255u); }

// a += sum of x[e] * byte e of w4 over the 4 bytes.
__device__ __forceinline__ float dot4b(uint32_t w, float4 x, float a) {
    a = fmaf(x.x, ub<0>(w), a);
    a = fmaf(x.y, ub<1>(w), a);
    a = fmaf(x.z, ub<2>(w), a);
    return fmaf(x.w, ub<3>(w), a);
}

// Codes of 8 weights (dword i of a chunk: weight e in nibble e) as two byte
// vectors: lo = weights 0, 2, 4, 6 and hi = weights 1, 3, 5, 7.  extra holds
// per-weight high bits already in place (bits 4.. of each byte).
// (The masks go through v_and_or_b32 as inline assembly: with the masked
// bits visible the compiler turns each byte's conversion into a bit-field
// extract plus v_cvt_f32_ubyte0 instead of one v_cvt_f32_ubyte<k>.)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
    return r;
}
__device__ __forceinline__ void split8(uint32_t w, uint32_t extra_lo, uint32_t extra_hi, uint32_t &lo, uint32_t &hi) {
    lo = and_or(w, 0x0F0F0F0Fu, extra_lo);
    hi = and_or(w >> 4, 0x0F0F0F0Fu, extra_hi);
}

// sum x[e] * u_e over 8 weights whose x are x[0..7] (two float4): u from the
// two byte vectors of split8.
__device__ __forceinline__ float dot8w(uint32_t lo, uint32_t hi, float4 xa, float4 xb, float a) {
    a = fmaf(xa.x, ub<0>(lo), a);
    a = fmaf(xa.y, ub<0>(hi), a);
    a = fmaf(xa.z, ub<1>(lo), a);
    a = fmaf(xa.w, ub<1>(hi), a);
    a = fmaf(xb.x, ub<2>(lo), a);
    a = fmaf(xb.y, ub<2>(hi), a);
    a = fmaf(xb.z, ub<3>(lo), a);
    return fmaf(xb.w, ub<3>(hi), a);
}

// Spread 4 bit fields of width W at positions 2W*k (k = 0..3, i.e. the even
// weights of 8) of f to bit 4 of byte k.  W = 1 (Q5_K's 5th bits) or 2
// (Q6_K's high bits).
template <int W>
__device__ __forceinline__ uint32_t spread4(uint32_t f) {
    if (W == 1) {
        uint32_t x = f & 0x55u;                 // bits 0, 2, 4, 6
        x = (x | (x << 12)) & 0x00050005u;      // 0, 2, 16, 18
        x = (x | (x << 6)) & 0x01010101u;       // 0, 8, 16, 24
        return x << 4;
    } else {
        uint32_t x = f & 0x3333u;               // pairs at 0, 4, 8, 12
        x = (x | (x << 8)) & 0x00330033u;       // 0, 4, 16, 20
        x = (x | (x << 4)) & 0x03030303u;       // 0, 8, 16, 24
        return x << 4;
    }
}

template <int TYPE, int NW, int STEPS, int WIN, bool AC>
__global__ __launch_bounds__(NW * 64) void gguf1_kernel(G1Args a) {
    using T = T1<TYPE>;
    using St = Stage<TYPE, STEPS>;
    constexpr int NT = NW * 64;
    constexpr int WPC = T::WPC;
    extern __shared__ __align__(16) float smem_f[];
    __shared__ __align__(16) uint8_t s_meta[NW][St::LOADS * 1024];
    __shared__ __align__(16) uint8_t s_d6[NW][St::D6_LOADS > 0 ? St::D6_LOADS * 1024 : 16];
    __shared__ ArgmaxPart s_best[NW];
    __shared__ float s_red[NW], s_red2[NW];

    const int K = a.K, CK = a.CK;
    float *xs = smem_f;                                // [K] activations
    float *xsum16 = xs + K;                            // [K / 16] sums of 16
    float *part = xsum16 + ((K / 16 + 3) & ~3);        // [tmax][NW][16 rows][4], 16-byte aligned
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, j = lane >> 4;
    const int S = (CK + 3) >> 2;
    const int t0 = (int)((blockIdx.x * (uint32_t)a.ntiles) / gridDim.x);
    const int nt = (int)(((blockIdx.x + 1) * (uint32_t)a.ntiles) / gridDim.x) - t0;
    const int W = nt * S;
    const int g0 = (wid * W) / NW;
    const int ns = ((wid + 1) * W) / NW - g0;
    const int tA = ns > 0 ? (int)((uint32_t)g0 / (uint32_t)S) : 0;
    const int sA = ns > 0 ? g0 - tA * S : 0;

    // 1. Activations (four per thread and round), then the wave's staged
    //    fields, codes and high bits, then the epilogue operands.
    const int nunits = K / 4;
    constexpr int UPT = 4;  // up to 16 KiB of activations per round of 1024 threads
    const auto rx = make_rsrc(a.x, (uint32_t)K * (a.swiglu ? 8u : 4u));
    uint4 xv[UPT], xu[UPT];
    if constexpr (AC) {
        // The row is the attention output: per head h = u / 16 and dims
        // 4 (u % 16).., out = sum_j acc_j exp(m_j - M) / sum_j t_j exp(m_j -
        // M) over the ns valid splits, in order (attend_combine_kernel's
        // arithmetic).
        // (every split of the head is loaded, used or not: the loads go out
        // with the position's, which they do not wait for)
        const auto rp = make_rsrc(a.apart, (uint32_t)(K / 64) * (uint32_t)a.ans_max * kAPart * 4u);
        float2 mt[kACUnits][kACMax];
        uint4 av[kACUnits][kACMax];
#pragma unroll
        for (int i = 0; i < kACUnits; i++) {
            const int u = tid + NT * i;
            const bool ok = u < nunits;
            const uint32_t base = (uint32_t)((u >> 4) * a.ans_max) * kAPart * 4u;
#pragma unroll
            for (int jj = 0; jj < kACMax; jj++) {
                const bool lj = ok && jj < a.ans_max;
                const uint2 w2 = bload8(rp, lj ? base + (uint32_t)jj * kAPart * 4u : kOOB);
                mt[i][jj] = make_float2(__uint_as_float(w2.x), __uint_as_float(w2.y));
                av[i][jj] = bload16(rp, lj ? base + (uint32_t)jj * kAPart * 4u + 16u + 16u * (uint32_t)(u & 15) : kOOB);
            }
        }
        const int ns = min(a.ans_max, (a.astate[0] + a.asplit) / a.asplit);
#pragma unroll
        for (int i = 0; i < UPT; i++) xv[i] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int i = 0; i < kACUnits && i < UPT; i++) {
            float M = ns > 0 ? mt[i][0].x : -INFINITY;
#pragma unroll
            for (int jj = 1; jj < kACMax; jj++) M = fmaxf(M, jj < ns ? mt[i][jj].x : -INFINITY);
            float T = 0.0f, o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
#pragma unroll
            for (int jj = 0; jj < kACMax; jj++) {
                if (jj < ns) {
                    const float f = expf(mt[i][jj].x - M);
                    T = fmaf(mt[i][jj].y, f, T);
                    o0 = fmaf(__uint_as_float(av[i][jj].x), f, o0);
                    o1 = fmaf(__uint_as_float(av[i][jj].y), f, o1);
                    o2 = fmaf(__uint_as_float(av[i][jj].z), f, o2);
                    o3 = fmaf(__uint_as_float(av[i][jj].w), f, o3);
                }
            }
            xv[i] = make_uint4(__float_as_uint(o0 / T), __float_as_uint(o1 / T), __float_as_uint(o2 / T),
                               __float_as_uint(o3 / T));
        }
    } else {
#pragma unroll
        for (int i = 0; i < UPT; i++) {
            const uint32_t u = (uint32_t)(tid + NT * i);
            xv[i] = bload16(rx, u < (uint32_t)nunits ? u * 16u : kOOB);
            if (a.swiglu) xu[i] = bload16(rx, u < (uint32_t)nunits ? (u + (uint32_t)nunits) * 16u : kOOB);
        }
    }
    // the RMSNorm gain of the same units, with the row (it is not needed before
    // the norm); 16-wave forms (128 registers a lane) load it in the norm's loop
    constexpr int GU = NW <= 8 ? UPT : 0;
    uint4 gv[GU > 0 ? GU : 1];
    {
        const auto rg = make_rsrc(a.rms_g, a.rms_g ? (uint32_t)K * 4u : 0u);
#pragma unroll
        for (int i = 0; i < GU; i++) {
            const uint32_t u = (uint32_t)(tid + NT * i);
            gv[i] = bload16(rg, a.rms_g && u < (uint32_t)nunits ? u * 16u : kOOB);
        }
    }
    // Global chunk indices of the wave's first and last valid chunks.
    const int gE = g0 + max(ns, 1) - 1;
    const int tE = (int)((uint32_t)gE / (uint32_t)S), sE = gE - tE * S;
    const int cg_lo = (t0 + tA) * CK + 4 * sA;
    const int cg_hi = (t0 + tE) * CK + min(4 * sE + 3, CK - 1);
    int mi_lo, mi_hi;
    if constexpr (T::QM) {  // groups [tile][group]: contiguous over the wave's run as well
        mi_lo = (t0 + tA) * a.NG + ((4 * sA) >> a.cpg_shift);
        mi_hi = (t0 + tE) * a.NG + (min(4 * sE + 3, CK - 1) >> a.cpg_shift);
    } else {
        mi_lo = cg_lo >> T::META_SHIFT;
        mi_hi = cg_hi >> T::META_SHIFT;
    }
    const int mcount = ns > 0 ? mi_hi - mi_lo + 1 : 1;
    const auto rm = make_rsrc(T::KQ ? a.sb : a.meta, T::KQ ? a.sb_bytes : a.meta_bytes);
    uint4 wm[St::LOADS];
#pragma unroll
    for (int i = 0; i < St::LOADS; i++) {
        const uint32_t off = (uint32_t)(i * 1024 + lane * 16);
        wm[i] = bload16(rm, off < (uint32_t)(mcount * 16 * T::META_ESZ) ? (uint32_t)mi_lo * 16u * T::META_ESZ + off : kOOB);
    }
    uint4 wd6[St::D6_LOADS > 0 ? St::D6_LOADS : 1];
    if constexpr (St::D6_LOADS > 0) {
        const auto rd = make_rsrc(a.d6, a.d6_bytes);
#pragma unroll
        for (int i = 0; i < St::D6_LOADS; i++) {
            const uint32_t off = (uint32_t)(i * 1024 + lane * 16);
            wd6[i] = bload16(rd, off < (uint32_t)(mcount * 16 * T::D6_ESZ) ? (uint32_t)mi_lo * 16u * T::D6_ESZ + off
                                                                            : kOOB);
        }
    }
    const uint32_t offA = ((uint32_t)(t0 + tA) * (uint32_t)CK + 4u * (uint32_t)sA) * 16u;  // chunk-row index
    const uint32_t wrap_adj = (uint32_t)(CK - 4 * S) * 16u;
    const uint32_t lane_cr = (uint32_t)j * 16u + (uint32_t)r;
    // Codes (and high bits) of step u; the first WIN steps go out now, step
    // u + WIN as step u is consumed (WIN < STEPS for matrices streamed from
    // HBM: fewer bytes queued ahead of the activation row's fetch).
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rb = make_rsrc(a.bits, a.bits_bytes);
    uint4 wc[STEPS];
    uint2 wb[T::BITS_ESZ > 0 ? STEPS : 1];
    auto load_step = [&](int u) {
        const uint32_t cr = offA + (uint32_t)u * 64u + (sA + u >= S ? wrap_adj : 0u) + lane_cr;
        wc[u] = bload16_nt(rc, u < ns ? cr * 16u : kOOB);
        if constexpr (T::BITS_ESZ == 8) wb[u] = bload8(rb, u < ns ? cr * 8u : kOOB);
        if constexpr (T::BITS_ESZ == 4) wb[u] = make_uint2(bload4(rb, u < ns ? cr * 4u : kOOB), 0u);
    };
#pragma unroll
    for (int u = 0; u < WIN; u++) load_step(u);
    const int o = (t0 + wid) * 16 + r;
    const bool row_ok = wid < nt && o < a.n;
    const auto rbias = make_rsrc(a.bias, (uint32_t)a.n * 4u);
    const auto rout = make_rsrc(a.out, (uint32_t)a.n * 4u);
    const float e_bias = __uint_as_float(bload4(rbias, row_ok ? (uint32_t)o * 4u : kOOB));
    const float e_res = __uint_as_float(bload4(rout, row_ok ? (uint32_t)o * 4u : kOOB));

    // 2. Activations and their sums of 16 into LDS; the wave's fields into
    //    its slot.
#pragma unroll
    for (int i = 0; i < UPT; i++) {
        const int u = tid + NT * i;
        if (u < nunits) reinterpret_cast<uint4 *>(xs)[u] = a.swiglu ? swiglu4(xv[i], xu[i]) : xv[i];
    }
    for (int u = tid + NT * UPT; u < nunits; u += NT) {
        const uint4 v = bload16(rx, (uint32_t)u * 16u);
        reinterpret_cast<uint4 *>(xs)[u] = a.swiglu ? swiglu4(v, bload16(rx, (uint32_t)(u + nunits) * 16u)) : v;
    }
#pragma unroll
    for (int i = 0; i < St::LOADS; i++) reinterpret_cast<uint4 *>(s_meta[wid])[i * 64 + lane] = wm[i];
    if constexpr (St::D6_LOADS > 0) {
#pragma unroll
        for (int i = 0; i < St::D6_LOADS; i++) reinterpret_cast<uint4 *>(s_d6[wid])[i * 64 + lane] = wd6[i];
    }
    lds_barrier();
    if (a.rms_g) {  // RMSNorm of the staged row (llama.hip's rmsnorm, fused)
        float ss = 0.0f;
        for (int u = tid; u < nunits; u += NT) {
            const float4 v = reinterpret_cast<const float4 *>(xs)[u];
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
        ss = llmq_wave_sum_all(ss);
        if (lane == 0) s_red[wid] = ss;
        lds_barrier();
        ss = s_red[0];
#pragma unroll
        for (int i = 1; i < NW; i++) ss += s_red[i];
        const float r = 1.0f / sqrtf(ss / (float)K + a.rms_eps);
        const float4 *g4 = reinterpret_cast<const float4 *>(a.rms_g);
        auto norm = [&](int u, const float4 g) {
            float4 v = reinterpret_cast<const float4 *>(xs)[u];
            v.x = (v.x * r) * g.x;
            v.y = (v.y * r) * g.y;
            v.z = (v.z * r) * g.z;
            v.w = (v.w * r) * g.w;
            reinterpret_cast<float4 *>(xs)[u] = v;
        };
#pragma unroll
        for (int i = 0; i < GU; i++) {
            const int u = tid + NT * i;
            if (u < nunits)
                norm(u, make_float4(__uint_as_float(gv[i].x), __uint_as_float(gv[i].y), __uint_as_float(gv[i].z),
                                    __uint_as_float(gv[i].w)));
        }
        for (int u = tid + NT * GU; u < nunits; u += NT) norm(u, g4[u]);
        lds_barrier();
    }
    if (a.ln_w) {  // LayerNorm of the staged row (kernels.layernorm, kernels.mojo:179-197), fused
        float sum = 0.0f;
        for (int u = tid; u < nunits; u += NT) {
            const float4 v = reinterpret_cast<const float4 *>(xs)[u];
            sum += (v.x + v.y) + (v.z + v.w);
        }
        sum = llmq_wave_sum_all(sum);
        if (lane == 0) s_red[wid] = sum;
        lds_barrier();
        sum = s_red[0];
#pragma unroll
        for (int i = 1; i < NW; i++) sum += s_red[i];
        const float mean = sum / (float)K;
        float sq = 0.0f;
        for (int u = tid; u < nunits; u += NT) {
            const float4 v = reinterpret_cast<const float4 *>(xs)[u];
            const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
            sq += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
        sq = llmq_wave_sum_all(sq);
        if (lane == 0) s_red2[wid] = sq;
        lds_barrier();
        sq = s_red2[0];
#pragma unroll
        for (int i = 1; i < NW; i++) sq += s_red2[i];
        const float rstd = 1.0f / sqrtf(sq / (float)K + 1e-5f);
        const float4 *w4 = reinterpret_cast<const float4 *>(a.ln_w);
        const float4 *b4 = reinterpret_cast<const float4 *>(a.ln_b);
        for (int u = tid; u < nunits; u += NT) {
            float4 v = reinterpret_cast<const float4 *>(xs)[u];
            const float4 g = w4[u], c = b4[u];
            v.x = ((v.x - mean) * rstd) * g.x + c.x;
            v.y = ((v.y - mean) * rstd) * g.y + c.y;
            v.z = ((v.z - mean) * rstd) * g.z + c.z;
            v.w = ((v.w - mean) * rstd) * g.w + c.w;
            reinterpret_cast<float4 *>(xs)[u] = v;
        }
        lds_barrier();
    }
    for (int g = tid; g < K / 16; g += NT) {
        const float4 *p = reinterpret_cast<const float4 *>(xs + 16 * g);
        const float4 v0 = p[0], v1 = p[1], v2 = p[2], v3 = p[3];
        xsum16[g] = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w)) +
                    (((v2.x + v2.y) + (v2.z + v2.w)) + ((v3.x + v3.y) + (v3.z + v3.w)));
    }
    lds_barrier();

    // 3. Per step: the block's factors, then sum x*u over the chunk's codes.
    //    contribution = pA * aA + pB * aB + qA * SA + qB * SB over the chunk's
    //    halves (16 weights each; Q8_0's chunk is one half).
    float accA = 0.0f, accB = 0.0f;
#pragma unroll
    for (int u = 0; u < STEPS; u++) {
        if (u < ns) {  // wave-uniform: steps past the wave's range carry no codes
            if (u + WIN < STEPS) {
                __builtin_amdgcn_sched_barrier(0);
                load_step(u + WIN);
                __builtin_amdgcn_sched_barrier(0);
            }
            const bool second = sA + u >= S;
            const int tl = tA + (second ? 1 : 0);
            const int ss = sA + u - (second ? S : 0);
            const int c_raw = 4 * ss + j;
            const bool ok = c_raw < CK;
            const int c = ok ? c_raw : 0;
            int mi;
            if constexpr (T::QM)
                mi = ok ? (t0 + tl) * a.NG + (c >> a.cpg_shift) - mi_lo : 0;
            else
                mi = ok ? (((t0 + tl) * CK + c) >> T::META_SHIFT) - mi_lo : 0;
            float pA, pB, qA, qB;
            if (T::QM) {  // s * (a - zp * S) over the chunk: pA = s, qA = -zp
                pA = pB = h2f(reinterpret_cast<const uint16_t *>(s_meta[wid])[mi * 16 + r]);
                qA = qB = -(float)s_d6[wid][mi * 16 + r];
            } else if (TYPE == LLMQ_GGML_Q4_0 || TYPE == LLMQ_GGML_Q8_0) {
                const float d = h2f(reinterpret_cast<const uint16_t *>(s_meta[wid])[mi * 16 + r]);
                pA = pB = d;
                qA = qB = (TYPE == LLMQ_GGML_Q4_0 ? -8.0f : -128.0f) * d;
            } else if (TYPE == LLMQ_GGML_Q4_1) {
                const uint32_t dm = reinterpret_cast<const uint32_t *>(s_meta[wid])[mi * 16 + r];
                pA = pB = h2f(dm);
                qA = qB = h2f(dm >> 16);
            } else if (TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K) {
                const uint4 f = reinterpret_cast<const uint4 *>(s_meta[wid])[mi * 16 + r];
                int sc, mn;
                k_scale_min(f.y, f.z, f.w, c & 7, sc, mn);
                pA = pB = h2f(f.x) * (float)sc;
                qA = qB = -(h2f(f.x >> 16) * (float)mn);
            } else {  // Q6_K: int8 scales 2(c & 7) and 2(c & 7) + 1, d of the superblock
                const uint16_t sp = reinterpret_cast<const uint16_t *>(s_meta[wid])[(mi * 16 + r) * 8 + (c & 7)];
                const float d = h2f(reinterpret_cast<const uint16_t *>(s_d6[wid])[mi * 16 + r]);
                pA = d * (float)(int8_t)(sp & 255u);
                pB = d * (float)(int8_t)(sp >> 8);
                qA = -32.0f * pA;
                qB = -32.0f * pB;
            }
            if (!ok) pA = pB = qA = qB = 0.0f;
            const uint4 d4 = wc[u];
            const float4 *xc = reinterpret_cast<const float4 *>(xs + c * WPC);
            float aA = 0.0f, aB = 0.0f, SA, SB;
            if (T::BYTES) {
                // 16 one-byte codes: Q8_0's int8 as q + 128, QuantMatrix's u8 as they are
                const uint32_t flip = TYPE == LLMQ_GGML_Q8_0 ? 0x80808080u : 0u;
                aA = dot4b(d4.x ^ flip, xc[0], aA);
                aA = dot4b(d4.y ^ flip, xc[1], aA);
                aA = dot4b(d4.z ^ flip, xc[2], aA);
                aA = dot4b(d4.w ^ flip, xc[3], aA);
                SA = xsum16[c];
                SB = 0.0f;
            } else {
                uint32_t e[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};  // high bits per dword: even / odd weights
                if (TYPE == LLMQ_GGML_Q5_K) {
                    const uint32_t b = wb[u].x;
    #pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t f = (b >> (8 * i)) & 255u;
                        e[i][0] = spread4<1>(f);
                        e[i][1] = spread4<1>(f >> 1);
                    }
                } else if (TYPE == LLMQ_GGML_Q6_K) {
                    const uint2 b = wb[u];
    #pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t f = ((i < 2 ? b.x : b.y) >> (16 * (i & 1))) & 0xFFFFu;
                        e[i][0] = spread4<2>(f);
                        e[i][1] = spread4<2>(f >> 2);
                    }
                }
                const uint32_t dw[4] = {d4.x, d4.y, d4.z, d4.w};
    #pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t lo, hi;
                    split8(dw[i], e[i][0], e[i][1], lo, hi);
                    if (i < 2)
                        aA = dot8w(lo, hi, xc[2 * i], xc[2 * i + 1], aA);
                    else
                        aB = dot8w(lo, hi, xc[2 * i], xc[2 * i + 1], aB);
                }
                SA = xsum16[2 * c];
                SB = xsum16[2 * c + 1];
            }
            // QuantMatrix's chunk lies in one group: s * (a - zp S), the
            // zero-point product exact inside the FMA
            const float contrib = T::QM ? pA * fmaf(qA, SA + SB, aA + aB) : (pA * aA + qA * SA) + (pB * aB + qB * SB);
            accA += second ? 0.0f : contrib;
            accB += second ? contrib : 0.0f;
        }
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
            if (a.flags & LLMQ_BIAS) v += e_bias;
            if (a.flags & LLMQ_GELU) v = gelu_ref(v);
            if (a.flags & LLMQ_RESID) v += e_res;
            a.out[o] = v;
            best_v = v;
            best_i = o;
        }
    }
    if (a.amax) {
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
    int nw, tmax, spw, steps, grid, win;
};

// Matrices whose codes take at least this many bytes are taken as streamed
// from HBM and keep kStreamWin steps in flight per wave.
constexpr int64_t kStreamBytes = 20ll << 20;
constexpr int kStreamWin = 2;

int steps_for(int spw) { return spw <= 2 ? 2 : spw <= 4 ? 4 : spw <= 8 ? 8 : 16; }
int max_steps(const llmq_mat *w) {
    const int t = float_act_type(w);
    return t == LLMQ_GGML_Q8_0 || t == kQmFloat8 ? 2 * kMaxSteps : kMaxSteps;
}

// As the one-token integer kernel's plan: 4-wave workgroups of one tile for
// small matrices, else one 16-wave workgroup per CU with whole-tile runs.
Plan make_plan(const llmq_mat *w) {
    Plan p{};
    const int S = (int)((w->CK + 3) / 4);
    const int64_t bytes = w->ntiles * w->CK * 256;
    // 4-wave workgroups of one row tile for matrices up to 4 steps a wave
    // (they launch faster; with 8 steps a wave the K-quants' decode work
    // runs one wave per SIMD and is slower: Q5_K 4096x4096 7.22 -> 7.84 us),
    // and for matrices streamed from HBM up to 8 steps a wave (4096 inputs:
    // 688-2000 workgroups; Q4_K 4096x11008 10.3 -> 9.7 us, Q6_K 12.6 ->
    // 11.8 us, Q4_K 4096x32000 23.4 -> 21.9 us against the 16-wave form);
    // 16 waves otherwise.  LLMQ_GEMV1_NW=4|8|16 forces the shape, for
    // measurement.
    const int cap4 = bytes >= kStreamBytes ? 8 : 4;
    int nw = (S + 3) / 4 <= cap4 ? 4 : 16;
    const char *force = getenv("LLMQ_GEMV1_NW");
    if (force) {
        const int v = atoi(force);
        if (v == 4 || v == 8 || v == 16) nw = v;
        if (nw < 16 && (S + nw - 1) / nw > 8) nw = 16;
    }
    int64_t grid = w->ntiles;
    if (nw == 16) {
        grid = std::min<int64_t>(w->ntiles, 256);
        const int cap = std::min(max_steps(w), S + 1);
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
    // Two code steps in flight a wave, the next issued as each is consumed
    // (fewer bytes queued ahead of the activation row's fetch), where it
    // measured faster: 4-wave plans of 8 MB or more (config 4's gate / up
    // 6.70 -> 6.62 us), 16-wave plans from 20 MB and below 8 MB (long rows of
    // few tiles: config 4's down 6.90 -> 6.75 us); every step up front
    // otherwise (qkv-sized matrices: 4.18 against 4.33 us; Q8_0 4096 x 4096
    // 7.64 against 8.24 us).  LLMQ_GGUF1_WIN=2 forces the window, any other
    // value every step up front.
    const bool win2 = nw == 16 ? (bytes >= kStreamBytes || bytes < (8ll << 20)) : bytes >= (8ll << 20);
    p.win = win2 ? kStreamWin : p.steps;
    if (const char *e = getenv("LLMQ_GGUF1_WIN")) p.win = atoi(e) == kStreamWin ? kStreamWin : p.steps;
    if (p.win > p.steps) p.win = p.steps;
    return p;
}

size_t lds_bytes(const llmq_mat *w, const Plan &p) {
    return (size_t)w->k * 4 + (size_t)((w->k / 16 + 3) & ~3) * 4 + (size_t)p.tmax * p.nw * 64 * 4;
}

template <int TYPE, int NW, int STEPS, int WIN, bool AC = false>
int launch_w(llmq_ctx *ctx, const G1Args &a, const Plan &p, size_t lds) {
    auto kern = gguf1_kernel<TYPE, NW, STEPS, WIN, AC>;
    hipFuncAttributes fa{};
    LLMQ_HIP(hipFuncGetAttributes(&fa, reinterpret_cast<const void *>(kern)));
    if (fa.sharedSizeBytes + lds > ctx->prop.sharedMemPerBlock)
        return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf_gemv: reduction axis %d needs %zu bytes of LDS (%zu available)",
                              a.K, fa.sharedSizeBytes + lds, (size_t)ctx->prop.sharedMemPerBlock);
    static size_t lds_set = 0;  // the kernel's dynamic-LDS limit raised so far (one host thread per context)
    if (lds > lds_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess)
            return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf_gemv: %zu bytes of LDS not available", lds);
        lds_set = lds;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)p.grid), dim3(NW * 64), lds, ctx->stream, a);
    return LLMQ_OK;
}

template <int TYPE, int NW, int STEPS>
int launch_t(llmq_ctx *ctx, const G1Args &a, const Plan &p, size_t lds) {
    if constexpr (STEPS > kStreamWin)
        if (p.win == kStreamWin) return launch_w<TYPE, NW, STEPS, kStreamWin>(ctx, a, p, lds);
    return launch_w<TYPE, NW, STEPS, STEPS>(ctx, a, p, lds);
}

template <int TYPE>
int launch_type(llmq_ctx *ctx, const G1Args &a, const Plan &p, size_t lds) {
    if (p.nw == 4) {
        if (a.apart) {  // attention-combine staging: 4- and 8-wave plans only (gguf_gemv_attn_ok)
            if (p.steps == 2) return launch_w<TYPE, 4, 2, 2, true>(ctx, a, p, lds);
            if (p.steps == 4) return launch_w<TYPE, 4, 4, 4, true>(ctx, a, p, lds);
        }
        if (p.steps == 2) return launch_t<TYPE, 4, 2>(ctx, a, p, lds);
        if (p.steps == 4) return launch_t<TYPE, 4, 4>(ctx, a, p, lds);
        if (p.steps == 8) return launch_t<TYPE, 4, 8>(ctx, a, p, lds);
    } else if (p.nw == 8) {
        if (a.apart) {
            if (p.steps == 2) return launch_w<TYPE, 8, 2, 2, true>(ctx, a, p, lds);
            if (p.steps == 4) return launch_w<TYPE, 8, 4, 4, true>(ctx, a, p, lds);
        }
        if (p.steps == 2) return launch_t<TYPE, 8, 2>(ctx, a, p, lds);
        if (p.steps == 4) return launch_t<TYPE, 8, 4>(ctx, a, p, lds);
        if (p.steps == 8) return launch_t<TYPE, 8, 8>(ctx, a, p, lds);
    } else {
        if (p.steps == 2) return launch_t<TYPE, 16, 2>(ctx, a, p, lds);
        if (p.steps == 4) return launch_t<TYPE, 16, 4>(ctx, a, p, lds);
        if (p.steps == 8) return launch_t<TYPE, 16, 8>(ctx, a, p, lds);
        if constexpr (T1<TYPE>::BYTES)
            if (p.steps == 16) return launch_t<TYPE, 16, 16>(ctx, a, p, lds);
    }
    return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf_gemv: no kernel for %d waves x %d steps", p.nw, p.steps);
}

}  // namespace

int qm_cpg_shift(const llmq_mat *w) {
    if (w->NG == 1) return 31;  // per-channel: every chunk is group 0
    const int64_t cpg = w->group / (w->bits == 4 ? 32 : 16);  // chunks per group
    if ((cpg & (cpg - 1)) != 0) return -1;
    return __builtin_ctzll((unsigned long long)cpg);
}

int gguf_num_parts(const llmq_mat *w) { return make_plan(w).grid; }

bool gguf_gemv_attn_ok(const llmq_mat *w, int ns_max, int head_dim) {
    if (head_dim != kLlmqSplitHD) return false;
    if (!w || !is_float_act(w) || w->k % 64 != 0 || ns_max < 1 || ns_max > kACMax) return false;
    const Plan p = make_plan(w);
    return (p.nw == 4 || p.nw == 8) && (p.steps == 2 || p.steps == 4) && w->k / 4 <= (int64_t)kACUnits * 4 * 64;
}

int launch_gguf_gemv(llmq_ctx *ctx, const llmq_mat *w, const float *x, float *out, const float *bias, int flags,
                     ArgmaxPart *amax, int amax_cap, const float *rms_g, float rms_eps, int swiglu,
                     const float *ln_w, const float *ln_b, const float *apart, const int *astate, int asplit,
                     int ans_max) {
    LLMQ_REQUIRE(w && is_float_act(w), "gguf_gemv: not a GGUF or float-activation QuantMatrix");
    LLMQ_REQUIRE((x || apart) && out, "gguf_gemv: null pointer");
    LLMQ_REQUIRE(!apart || (gguf_gemv_attn_ok(w, ans_max, kLlmqSplitHD) && astate && asplit > 0 && !rms_g && !swiglu && !ln_w),
                 "gguf_gemv: attention-split input not supported for %lld x %lld", (long long)w->n, (long long)w->k);
    LLMQ_REQUIRE(!(flags & LLMQ_BIAS) || bias, "gguf_gemv: LLMQ_BIAS without a bias");
    LLMQ_REQUIRE(w->k % 16 == 0, "gguf_gemv: cols must be a multiple of 16");
    const Plan p = make_plan(w);
    const size_t lds = lds_bytes(w, p);
    LLMQ_REQUIRE(p.spw <= max_steps(w) && p.spw <= (w->CK + 3) / 4 + 1,
                 "gguf_gemv: no one-token kernel for %lld x %lld", (long long)w->n, (long long)w->k);
    LLMQ_REQUIRE(!amax || p.grid <= amax_cap, "gguf_gemv: argmax capacity");
    const int64_t ntc = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 16;  // (chunk, row) entries incl. padding
    const int64_t nts = (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16;  // (superblock, row) entries
    G1Args a{};
    const int type = float_act_type(w);
    a.codes = w->codes;
    a.codes_bytes = (uint32_t)(ntc * 16);
    if (w->kind == MAT_QUANT) {
        const int64_t ntg = (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16;  // (group, row) entries incl. padding
        a.meta = reinterpret_cast<const uint8_t *>(w->scales);
        a.meta_bytes = (uint32_t)(ntg * 2);
        a.d6 = w->zps;
        a.d6_bytes = (uint32_t)ntg;
        a.NG = (int)w->NG;
        a.cpg_shift = qm_cpg_shift(w);
        LLMQ_REQUIRE(a.cpg_shift >= 0, "linear: group %lld is not a power of two times 32", (long long)w->group);
    } else {
        a.meta = reinterpret_cast<const uint8_t *>(w->ggml_type == LLMQ_GGML_Q4_1 ? w->g_meta32 : w->g_meta16);
        a.meta_bytes = (uint32_t)(w->ggml_type == LLMQ_GGML_Q4_1 ? ntc * 4 : ntc * 2);
        a.bits = reinterpret_cast<const uint8_t *>(w->ggml_type == LLMQ_GGML_Q6_K ? w->g_bits64 : w->g_bits32);
        a.bits_bytes = (uint32_t)(w->ggml_type == LLMQ_GGML_Q6_K ? ntc * 8 : ntc * 4);
        a.sb = reinterpret_cast<const uint8_t *>(w->g_sb16);
        a.sb_bytes = (uint32_t)(nts * 16);
        a.d6 = reinterpret_cast<const uint8_t *>(w->g_meta16);
        a.d6_bytes = (uint32_t)(nts * 2);
    }
    a.n = (int)w->n;
    a.K = (int)w->k;
    a.ntiles = (int)w->ntiles;
    a.CK = (int)w->CK;
    a.tmax = p.tmax;
    a.flags = flags;
    a.x = x;
    a.bias = bias ? bias : out;  // read (and ignored) without LLMQ_BIAS
    a.out = out;
    a.amax = amax;
    a.rms_g = rms_g;
    a.rms_eps = rms_eps;
    a.ln_w = ln_w;
    a.ln_b = ln_b;
    a.swiglu = swiglu;
    a.apart = apart;
    a.astate = astate;
    a.asplit = asplit;
    a.ans_max = ans_max;
    int rc;
    switch (type) {
    case kQmFloat4: rc = launch_type<kQmFloat4>(ctx, a, p, lds); break;
    case kQmFloat8: rc = launch_type<kQmFloat8>(ctx, a, p, lds); break;
    case LLMQ_GGML_Q4_0: rc = launch_type<LLMQ_GGML_Q4_0>(ctx, a, p, lds); break;
    case LLMQ_GGML_Q4_1: rc = launch_type<LLMQ_GGML_Q4_1>(ctx, a, p, lds); break;
    case LLMQ_GGML_Q8_0: rc = launch_type<LLMQ_GGML_Q8_0>(ctx, a, p, lds); break;
    case LLMQ_GGML_Q4_K: rc = launch_type<LLMQ_GGML_Q4_K>(ctx, a, p, lds); break;
    case LLMQ_GGML_Q5_K: rc = launch_type<LLMQ_GGML_Q5_K>(ctx, a, p, lds); break;
    case LLMQ_GGML_Q6_K: rc = launch_type<LLMQ_GGML_Q6_K>(ctx, a, p, lds); break;
    default: return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf_gemv: type %d", type);
    }
    if (rc != LLMQ_OK) return rc;
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
