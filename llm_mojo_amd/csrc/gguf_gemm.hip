// Several-token GGUF matmul: matmul_rows for T > 1 over a GGUFMatrix
// (kernels.mojo:314-349: rows dequantized, gguf.mojo:178-297, then a float
// tile matmul, with store_out's bias / GELU / residual), on the fp32 matrix
// cores (v_mfma_f32_16x16x4f32).
//
// Each weight is dequantized with the reference decoder's float operations
// (the values equal GGUFMatrix.dequant_row bit for bit); products and sums
// are float32, in the matrix cores' order rather than mm_tile's.
//
// Mapping: a workgroup of NW waves owns 16 output rows (one row tile of the
// device layout) and 16 tokens; the reduction axis goes in blocks of 256
// inputs, block b to wave b % NW.  In a block, lane l takes row / token
// l % 16 and the 64-input run 64 (l / 16) ..: it decodes its row's 64
// weights and loads its token's 64 activations into registers, and MFMA
// step t multiplies input 64 (l / 16) + t of both.  The waves' 16 x 16
// partial sums are added in LDS in wave order.
#include "common.h"

namespace {

constexpr uint32_t kOOB = 0x80000000u;

typedef float v4f __attribute__((ext_vector_type(4)));

struct GArgs {
    const uint8_t *codes, *meta, *bits, *sb;
    uint32_t codes_bytes, meta_bytes, bits_bytes, sb_bytes, x_bytes;
    int n, K, CK, NSB, T, flags;
    int NG, cpg_shift;   // QuantMatrix: meta = f16 scales, bits = u8 zero points per (group, row)
    int64_t ldx, ldo;
    const float *x, *bias;
    float *out;
};

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
// The 16-bit element at index e of a buffer (via its aligned dword).
__device__ __forceinline__ uint32_t bload_h(__amdgpu_buffer_rsrc_t r, uint32_t e, bool ok) {
    const uint32_t w = bload4(r, ok ? (e * 2u) & ~3u : kOOB);
    return (w >> (16 * (e & 1u))) & 0xFFFFu;
}
__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)bits)); }

// k_scale_min (gguf.mojo:205-221) of sub-block j over the 12 scale bytes.
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

// The WPC weights of chunk c of row r of tile `tile` (zeros when !ok), as
// the reference decoders compute them (the expressions of gguf.hip's row
// dequantizer).
template <int TYPE>
__device__ __forceinline__ void decode_chunk(const GArgs &a, uint32_t tile, uint32_t c, uint32_t r, bool ok,
                                             float *w) {
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rm = make_rsrc(a.meta, a.meta_bytes);
    const uint32_t e = (tile * (uint32_t)a.CK + c) * 16u + r;  // (chunk, row) entry
    const uint4 q4 = bload16(rc, ok ? e * 16u : kOOB);
    const uint32_t dw[4] = {q4.x, q4.y, q4.z, q4.w};
    if (TYPE == kQmFloat4 || TYPE == kQmFloat8) {
        // QuantMatrix.row_op (tensor.mojo:431-479): (f32(u) - f32(zp)) * f32(scale)
        const uint32_t gi = (tile * (uint32_t)a.NG + (c >> a.cpg_shift)) * 16u + r;
        const float s = h2f(bload_h(rm, gi, ok));
        const uint32_t zw = bload4(make_rsrc(a.bits, a.bits_bytes), ok ? gi & ~3u : kOOB);
        const float zp = (float)((zw >> (8 * (gi & 3u))) & 255u);
        if (TYPE == kQmFloat8) {
#pragma unroll
            for (int i = 0; i < 16; i++) w[i] = ((float)((dw[i >> 2] >> (8 * (i & 3))) & 255u) - zp) * s;
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) w[i] = ((float)((dw[i >> 3] >> (4 * (i & 7))) & 15u) - zp) * s;
        }
        return;
    }
    if (TYPE == LLMQ_GGML_Q8_0) {
        const float d = h2f(bload_h(rm, (tile * (uint32_t)(a.CK / 2) + (c >> 1)) * 16u + r, ok));
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = d * (float)(int)(int8_t)((dw[i >> 2] >> (8 * (i & 3))) & 255u);
        return;
    }
    if (TYPE == LLMQ_GGML_Q4_0) {
        const float d = h2f(bload_h(rm, e, ok));
#pragma unroll
        for (int i = 0; i < 32; i++) w[i] = ((float)((dw[i >> 3] >> (4 * (i & 7))) & 15u) - 8.0f) * d;
        return;
    }
    if (TYPE == LLMQ_GGML_Q4_1) {
        const uint32_t m = bload4(rm, ok ? e * 4u : kOOB);
        const float d = h2f(m), mm = h2f(m >> 16);
#pragma unroll
        for (int i = 0; i < 32; i++) w[i] = d * (float)((dw[i >> 3] >> (4 * (i & 7))) & 15u) + mm;
        return;
    }
    const auto rs = make_rsrc(a.sb, a.sb_bytes);
    const uint32_t se = (tile * (uint32_t)a.NSB + (c >> 3)) * 16u + r;  // (superblock, row) entry
    const uint4 f = bload16(rs, ok ? se * 16u : kOOB);
    if (TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K) {
        uint32_t hb = 0;
        if (TYPE == LLMQ_GGML_Q5_K) hb = bload4(make_rsrc(a.bits, a.bits_bytes), ok ? e * 4u : kOOB);
        int sc, mn;
        k_scale_min(f.y, f.z, f.w, (int)(c & 7u), sc, mn);
        const float ds = h2f(f.x) * (float)sc, dm = h2f(f.x >> 16) * (float)mn;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            int u = (int)((dw[i >> 3] >> (4 * (i & 7))) & 15u);
            if (TYPE == LLMQ_GGML_Q5_K) u |= (int)((hb >> i) & 1u) << 4;
            w[i] = ds * (float)u - dm;
        }
        return;
    }
    // Q6_K
    const uint2 hb = bload8(make_rsrc(a.bits, a.bits_bytes), ok ? e * 8u : kOOB);
    const float d = h2f(bload_h(rm, se, ok));
    const uint32_t sw[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const uint32_t hw = i < 16 ? hb.x : hb.y;
        const int u = (int)((dw[i >> 3] >> (4 * (i & 7))) & 15u) | ((int)((hw >> (2 * (i & 15))) & 3u) << 4);
        const int si = 2 * (int)(c & 7u) + (i >= 16);
        const float sc = (float)(int8_t)((sw[si >> 2] >> (8 * (si & 3))) & 255u);
        w[i] = (d * sc) * ((float)u - 32.0f);
    }
}

template <int TYPE, int NW>
__global__ __launch_bounds__(NW * 64) void gguf_gemm_kernel(GArgs a) {
    constexpr int WPC = TYPE == LLMQ_GGML_Q8_0 || TYPE == kQmFloat8 ? 16 : 32;
    __shared__ float part[NW][256];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t tile = blockIdx.x;
    const int t0 = blockIdx.y * 16;
    const int m = lane & 15, j = lane >> 4;
    const auto rx = make_rsrc(a.x, a.x_bytes);
    const int tok = t0 + m;
    const int nblk = (a.K + 255) / 256;
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int blk = w; blk < nblk; blk += NW) {
        const int k = blk * 256 + 64 * j;  // this lane's run of 64 inputs
        float xa[64], wb[64];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const bool ok = tok < a.T && k + 4 * i < a.K;
            const uint4 v = bload16(rx, ok ? (uint32_t)(((int64_t)tok * a.ldx + k + 4 * i) * 4) : kOOB);
            xa[4 * i] = __uint_as_float(v.x);
            xa[4 * i + 1] = __uint_as_float(v.y);
            xa[4 * i + 2] = __uint_as_float(v.z);
            xa[4 * i + 3] = __uint_as_float(v.w);
        }
#pragma unroll
        for (int cc = 0; cc < 64 / WPC; cc++) {
            const int kc = k + WPC * cc;
            decode_chunk<TYPE>(a, tile, (uint32_t)(kc / WPC), (uint32_t)m, kc < a.K, wb + WPC * cc);
        }
#pragma unroll
        for (int t = 0; t < 64; t++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[t], wb[t], acc, 0, 0, 0);
    }
    // lane holds C[token 4 j + i][row m]
#pragma unroll
    for (int i = 0; i < 4; i++) part[w][(4 * j + i) * 16 + m] = acc[i];
    __syncthreads();
    if (tid < 256) {
        const int tt = tid >> 4, rr = tid & 15;
        float v = part[0][tid];
#pragma unroll
        for (int q = 1; q < NW; q++) v += part[q][tid];
        const int o = (int)tile * 16 + rr, tk = t0 + tt;
        if (o < a.n && tk < a.T) {
            if (a.flags & LLMQ_BIAS) v += a.bias[o];
            if (a.flags & LLMQ_GELU) v = gelu_ref(v);
            float *dst = a.out + (int64_t)tk * a.ldo + o;
            if (a.flags & LLMQ_RESID) v += *dst;
            *dst = v;
        }
    }
}

template <int TYPE>
int launch_t(llmq_ctx *ctx, const GArgs &a, dim3 grid, int nw) {
    if (nw == 8)
        hipLaunchKernelGGL((gguf_gemm_kernel<TYPE, 8>), grid, dim3(512), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL((gguf_gemm_kernel<TYPE, 4>), grid, dim3(256), 0, ctx->stream, a);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

}  // namespace

int launch_gguf_gemm(llmq_ctx *ctx, const llmq_mat *w, const float *x, int64_t ldx, int64_t T, float *out,
                     int64_t ldo, const float *bias, int flags, void *rec, int64_t rec_cap) {
    LLMQ_REQUIRE(w && is_float_act(w), "gguf_gemm: not a GGUF or float-activation QuantMatrix");
    LLMQ_REQUIRE(x && out && T > 0, "gguf_gemm: bad arguments");
    const char *he = getenv("LLMQ_GEMM_H16");
    if (rec_cap != 0 && gguf_gemm_h16_ok(w) && !(he && he[0] == '0')) {
        const int64_t need = h16_rec_bytes(T, w->k);
        if (rec_cap < 0)
            RC(ctx_workspace(ctx, (size_t)need, &rec, 1));
        else
            LLMQ_REQUIRE(rec && need <= rec_cap, "gguf_gemm: %lld tokens need a %lld-byte record, %lld given",
                         (long long)T, (long long)need, (long long)rec_cap);
        RC(launch_act_h16(ctx, x, ldx, T, w->k, rec));
        return launch_gguf_gemm_h16(ctx, w, rec, T, out, ldo, bias, flags);
    }
    LLMQ_REQUIRE(!(flags & LLMQ_BIAS) || bias, "gguf_gemm: LLMQ_BIAS without a bias");
    LLMQ_REQUIRE(w->k % 32 == 0, "gguf_gemm: cols must be a multiple of 32");
    const int64_t ntc = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 16;
    const int64_t nts = (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16;
    LLMQ_REQUIRE(ntc * 16 < (int64_t)kOOB && T * ldx * 4 < (int64_t)kOOB, "gguf_gemm: operands too large");
    LLMQ_REQUIRE(T <= 16 * 65535LL, "gguf_gemm: too many tokens");
    GArgs a{};
    const int t = float_act_type(w);
    a.codes = w->codes;
    a.codes_bytes = (uint32_t)(ntc * 16);
    if (w->kind == MAT_QUANT) {
        const int64_t ntg = (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16;  // (group, row) entries incl. padding
        a.meta = reinterpret_cast<const uint8_t *>(w->scales);
        a.meta_bytes = (uint32_t)(ntg * 2);
        a.NG = (int)w->NG;
        a.cpg_shift = qm_cpg_shift(w);
        LLMQ_REQUIRE(a.cpg_shift >= 0, "linear: group %lld is not a power of two times 32", (long long)w->group);
    } else if (t == LLMQ_GGML_Q4_1) {
        a.meta = reinterpret_cast<const uint8_t *>(w->g_meta32);
        a.meta_bytes = (uint32_t)(ntc * 4);
    } else if (t == LLMQ_GGML_Q6_K) {
        a.meta = reinterpret_cast<const uint8_t *>(w->g_meta16);
        a.meta_bytes = (uint32_t)(nts * 2);
    } else {
        a.meta = reinterpret_cast<const uint8_t *>(w->g_meta16);
        a.meta_bytes = w->g_meta16 ? (uint32_t)(ntc * 2) : 0u;
    }
    a.bits = reinterpret_cast<const uint8_t *>(t == LLMQ_GGML_Q6_K ? w->g_bits64 : w->g_bits32);
    a.bits_bytes = (uint32_t)(t == LLMQ_GGML_Q6_K ? ntc * 8 : (t == LLMQ_GGML_Q5_K ? ntc * 4 : 0));
    if (w->kind == MAT_QUANT) {
        a.bits = w->zps;
        a.bits_bytes = (uint32_t)((w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16);
    }
    a.sb = reinterpret_cast<const uint8_t *>(w->g_sb16);
    a.sb_bytes = w->g_sb16 ? (uint32_t)(nts * 16) : 0u;
    a.n = (int)w->n;
    a.K = (int)w->k;
    a.CK = (int)w->CK;
    a.NSB = (int)w->NG;
    a.T = (int)T;
    a.flags = flags;
    a.ldx = ldx;
    a.ldo = ldo;
    a.x = x;
    a.x_bytes = (uint32_t)(T * ldx * 4);
    a.bias = bias ? bias : out;
    a.out = out;
    const int nblk = (int)((w->k + 255) / 256);
    const int nw = nblk >= 8 ? 8 : 4;
    dim3 grid((unsigned)w->ntiles, (unsigned)((T + 15) / 16));
    switch (t) {
    case kQmFloat4: return launch_t<kQmFloat4>(ctx, a, grid, nw);
    case kQmFloat8: return launch_t<kQmFloat8>(ctx, a, grid, nw);
    case LLMQ_GGML_Q4_0: return launch_t<LLMQ_GGML_Q4_0>(ctx, a, grid, nw);
    case LLMQ_GGML_Q4_1: return launch_t<LLMQ_GGML_Q4_1>(ctx, a, grid, nw);
    case LLMQ_GGML_Q8_0: return launch_t<LLMQ_GGML_Q8_0>(ctx, a, grid, nw);
    case LLMQ_GGML_Q4_K: return launch_t<LLMQ_GGML_Q4_K>(ctx, a, grid, nw);
    case LLMQ_GGML_Q5_K: return launch_t<LLMQ_GGML_Q5_K>(ctx, a, grid, nw);
    case LLMQ_GGML_Q6_K: return launch_t<LLMQ_GGML_Q6_K>(ctx, a, grid, nw);
    default: return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf_gemm: type %d", t);
    }
}
