// The output head in integers for GGUF matrices with an int16 kernel (Q6_K,
// Q8_0): head_i16 (kernels.mojo:693-736) / head_team's has_i16 branch
// (kernels.mojo:886-896) over GGUFMatrix.dot_row_i16 (gguf.mojo:462-487).
//
// Per token t: h[t] is quantized to int16 (quantize_rows, kernels.mojo:
// 400-416) and every vocabulary row v gets
//   logits[t, v] = red16(accf) * sx,   accf[L] = fma(f32(acc_u[L]), d_u, accf[L]) over units u
// where a unit is a Q6_K superblock (256 weights, d at byte 208) or a Q8_0
// block (32 weights), and lane L (0..15) of a unit's int32 accumulator holds
// the products of weight pairs 2L, 2L+1 of each 32 weights of the unit
// (dot_pairs, tensor.mojo:34-46): Q6_K weights are (q - 32) * sc as int16,
// Q8_0's the int8 codes.  The lane sums are integers, so any order of
// adding them is exact; the float steps (per-lane conversion, the fma chain
// over units in order, the 16-lane halving sum) are the reference's, so a
// row's logit is the same float whatever the tile or token count.
//
// Work mapping: one workgroup per (16-row tile, up to 8 tokens taken one
// after another), 4 waves.  Thread
// (r, q) of a wave (r = lane % 16, q = lane / 16) computes lanes 4q..4q+3 of
// row r for a unit: Q6_K reads dword q of each of the unit's 8 chunks of 32
// codes (weights 8q..8q+7) and the matching 16 high bits; Q8_0 reads bytes
// 8(q%2)..+7 of half 2u + q/2.  Units go through LDS in rounds of R: the
// waves write each unit's 16 x 16 lane values as floats, then thread (r, L)
// of the workgroup runs lane L's fma chain over the round's units.
#include "common.h"

namespace {

constexpr uint32_t kOOB = 0x80000000u;
constexpr int kNW = 4;  // waves per workgroup

typedef short short2v __attribute__((ext_vector_type(2)));

struct H16Args {
    const uint8_t *codes, *bits, *sb, *d;
    uint32_t codes_bytes, bits_bytes, sb_bytes, d_bytes;
    int V, C, CK, NU, T, tpb;  // tpb: tokens a workgroup takes, one after another
    const float *h;
    float *logits;
    const float *rms_g;  // optional RMSNorm gain applied to h first
    float rms_eps;
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

__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)bits)); }

// Int(round(v)) of quantize_rows: half away from zero, NaN -> 0, saturated.
__device__ __forceinline__ int round_to_int(float v) {
    float r = roundf(v);
    r = r != r ? 0.0f : r;
    r = fminf(fmaxf(r, -1.0e9f), 1.0e9f);
    return (int)r;
}

__device__ __forceinline__ int sdot2(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(short2v, a), __builtin_bit_cast(short2v, b), c, false);
}

// Bits 4k..4k+1 (k = 0..3) of f to bits 4..5 of byte k.
__device__ __forceinline__ uint32_t spread2(uint32_t f) {
    uint32_t x = f & 0x3333u;               // pairs at 0, 4, 8, 12
    x = (x | (x << 8)) & 0x00330033u;       // 0, 4, 16, 20
    x = (x | (x << 4)) & 0x03030303u;       // 0, 8, 16, 24
    return x << 4;
}

template <int TYPE>
struct Unit {
    static constexpr int WEIGHTS = TYPE == LLMQ_GGML_Q6_K ? 256 : 32;
    static constexpr int UPW = TYPE == LLMQ_GGML_Q6_K ? 1 : 4;  // units a wave takes per round
    static constexpr int R = kNW * UPW;                         // units per round
};

// Lanes 4q..4q+3 of row r's int32 accumulator for Q6_K superblock u of
// tile `tile`, and its d.  xq32: the token's int16 activations as pairs.
__device__ __forceinline__ void q6k_unit(const H16Args &a, int tile, int u, int r, int q, const uint32_t *xq32,
                                         int (&acc)[4], float &d) {
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rb = make_rsrc(a.bits, a.bits_bytes);
    const auto rs = make_rsrc(a.sb, a.sb_bytes);
    const auto rd = make_rsrc(a.d, a.d_bytes);
    const uint32_t c0 = (uint32_t)tile * (uint32_t)a.CK + 8u * (uint32_t)u;  // global index of the unit's first chunk
    uint32_t cw[8], hw[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const uint32_t e = (c0 + c) * 16u + (uint32_t)r;  // (chunk, row) entry
        cw[c] = bload4(rc, e * 16u + 4u * (uint32_t)q);
        hw[c] = bload4(rb, e * 8u + 4u * (uint32_t)(q >> 1));
    }
    const uint32_t se = ((uint32_t)tile * (uint32_t)a.NU + (uint32_t)u) * 16u + (uint32_t)r;
    const uint4 sc4 = bload16(rs, se * 16u);
    const uint32_t dw = bload4(rd, (se * 2u) & ~3u);
    d = h2f(dw >> (16 * (se & 1u)));
    const uint32_t scw[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        // int8 scale of this chunk's half: scale 2c + (weights >= 16)
        const uint32_t sbyte = (scw[c >> 1] >> (8 * (2 * (c & 1) + (q >> 1)))) & 255u;
        const uint32_t s16 = (uint32_t)(int)(int8_t)sbyte & 0xFFFFu;
        const uint32_t spair = s16 | (s16 << 16);
        const uint32_t hb = hw[c] >> (16 * (q & 1));  // 2 high bits of weight 8q + i at bits 2i
        const uint32_t qe = (cw[c] & 0x0F0F0F0Fu) | spread2(hb);             // even weights, 6-bit codes
        const uint32_t qo = ((cw[c] >> 4) & 0x0F0F0F0Fu) | spread2(hb >> 2);  // odd weights
        const uint4 xv = *reinterpret_cast<const uint4 *>(xq32 + 128 * u + 16 * c + 4 * q);
        const uint32_t xp[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // [q_e, 0, q_o, 0]: the pair as two 16-bit codes
            const uint32_t sel = (uint32_t)j | (0x0Cu << 8) | ((uint32_t)(4 + j) << 16) | (0x0Cu << 24);
            const uint32_t p = __builtin_amdgcn_perm(qo, qe, sel);
            short2v w = __builtin_bit_cast(short2v, p) - (short2v){32, 32};
            w = w * __builtin_bit_cast(short2v, spair);  // (q - 32) * sc, |.| <= 4096
            acc[j] = sdot2(xp[j], __builtin_bit_cast(uint32_t, w), acc[j]);
        }
    }
}

// Lanes 4q..4q+3 of row r's int32 accumulator for Q8_0 block u, and its d.
// The codes are placed in the high byte of each 16-bit half (256 * code),
// so one dot gives 256 * (x0 w0 + x1 w1); |that| <= 2 * 32767 * 128 * 256 <
// 2^31, and the arithmetic shift by 8 is exact.
__device__ __forceinline__ void q80_unit(const H16Args &a, int tile, int u, int r, int q, const uint32_t *xq32,
                                         int (&acc)[4], float &d) {
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rd = make_rsrc(a.d, a.d_bytes);
    const uint32_t e = ((uint32_t)tile * (uint32_t)a.CK + 2u * (uint32_t)u + (uint32_t)(q >> 1)) * 16u + (uint32_t)r;
    const uint2 cw = bload8(rc, e * 16u + 8u * (uint32_t)(q & 1));
    const uint32_t de = ((uint32_t)tile * (uint32_t)(a.CK / 2) + (uint32_t)u) * 16u + (uint32_t)r;
    const uint32_t dw = bload4(rd, (de * 2u) & ~3u);
    d = h2f(dw >> (16 * (de & 1u)));
    const uint4 xv = *reinterpret_cast<const uint4 *>(xq32 + 16 * u + 4 * q);
    const uint32_t xp[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t ww[2] = {cw.x, cw.y};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t b = 2u * (uint32_t)(j & 1);  // pair j: bytes 2j, 2j + 1 of the 8
        const uint32_t sel = 0x0Cu | (b << 8) | (0x0Cu << 16) | ((b + 1u) << 24);
        const uint32_t p = __builtin_amdgcn_perm(0u, ww[j >> 1], sel);
        acc[j] = sdot2(xp[j], p, 0) >> 8;
    }
}

template <int TYPE>
__global__ __launch_bounds__(kNW * 64) void gguf_head16_kernel(H16Args a) {
    using U = Unit<TYPE>;
    extern __shared__ __align__(16) uint32_t smem_u[];
    __shared__ float red[kNW];
    uint32_t *xq32 = smem_u;                                               // [C / 2] int16 pairs
    float *lanev = reinterpret_cast<float *>(smem_u + a.C / 2);            // [R][16 rows][16 lanes]
    float *dv = lanev + U::R * 256;                                        // [R][16 rows]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x;
    const int tb = blockIdx.y * a.tpb, te = min(a.T, tb + a.tpb);
    // Tokens one after another: the tile's weights come from HBM for the
    // first and from L2 for the rest.
    for (int t = tb; t < te; t++) {
    const float *h = a.h + (size_t)t * a.C;

    const int n4 = a.C / 4;
    // optional RMSNorm: h -> (h * rn) * g, rn = 1 / sqrt(mean(h^2) + eps)
    float rn = 1.0f;
    const float4 *g4 = reinterpret_cast<const float4 *>(a.rms_g);
    if (a.rms_g) {
        float ss = 0.0f;
        for (int i = tid; i < n4; i += kNW * 64) {
            const float4 v = reinterpret_cast<const float4 *>(h)[i];
            ss = fmaf(v.x, v.x, ss);
            ss = fmaf(v.y, v.y, ss);
            ss = fmaf(v.z, v.z, ss);
            ss = fmaf(v.w, v.w, ss);
        }
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if (lane == 0) red[wid] = ss;
        __syncthreads();
        ss = ((red[0] + red[1]) + red[2]) + red[3];
        rn = 1.0f / sqrtf(ss / (float)a.C + a.rms_eps);
        __syncthreads();
    }
    auto row4 = [&](int i) {
        float4 v = reinterpret_cast<const float4 *>(h)[i];
        if (a.rms_g) {
            const float4 g = g4[i];
            v.x = (v.x * rn) * g.x;
            v.y = (v.y * rn) * g.y;
            v.z = (v.z * rn) * g.z;
            v.w = (v.w * rn) * g.w;
        }
        return v;
    };
    // quantize_rows for this token: s = max|h| / 32767, q = round(h / s)
    float m = 0.0f;
    for (int i = tid; i < n4; i += kNW * 64) {
        const float4 v = row4(i);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) red[wid] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sx = m / 32767.0f;
    if (sx == 0.0f) sx = 1.0f;
    const float inv = 1.0f / sx;
    for (int i = tid; i < n4; i += kNW * 64) {
        const float4 v = row4(i);
        const int q0 = round_to_int(v.x * inv), q1 = round_to_int(v.y * inv);
        const int q2 = round_to_int(v.z * inv), q3 = round_to_int(v.w * inv);
        xq32[2 * i] = ((uint32_t)q0 & 0xFFFFu) | ((uint32_t)q1 << 16);
        xq32[2 * i + 1] = ((uint32_t)q2 & 0xFFFFu) | ((uint32_t)q3 << 16);
    }
    __syncthreads();

    const int r = lane & 15, q = lane >> 4;  // phase 1: row r, lanes 4q..4q+3
    const int pr = tid >> 4, pl = tid & 15;  // phase 2: row pr, lane pl
    float accf = 0.0f;
    for (int u0 = 0; u0 < a.NU; u0 += U::R) {
#pragma unroll
        for (int i = 0; i < U::UPW; i++) {
            const int ul = wid * U::UPW + i, u = u0 + ul;
            if (u >= a.NU) break;
            int acc[4];
            float d;
            if (TYPE == LLMQ_GGML_Q6_K)
                q6k_unit(a, tile, u, r, q, xq32, acc, d);
            else
                q80_unit(a, tile, u, r, q, xq32, acc, d);
            *reinterpret_cast<float4 *>(lanev + (ul * 16 + r) * 16 + 4 * q) =
                make_float4((float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]);
            if (q == 0) dv[ul * 16 + r] = d;
        }
        __syncthreads();
        const int nu = min(U::R, a.NU - u0);
        for (int ul = 0; ul < nu; ul++) accf = fmaf(lanev[(ul * 16 + pr) * 16 + pl], dv[ul * 16 + pr], accf);
        __syncthreads();
    }
    // red16: v[i] + v[i + 8], then + 4, + 2, + 1 (lane pl < 8, 4, 2, 1 keeps the sums)
    accf += __shfl_xor(accf, 8);
    accf += __shfl_xor(accf, 4);
    accf += __shfl_xor(accf, 2);
    accf += __shfl_xor(accf, 1);
    const int row = tile * 16 + pr;
    if (pl == 0 && row < a.V) a.logits[(size_t)t * a.V + row] = accf * sx;
    __syncthreads();  // before the next token's codes overwrite the LDS
    }
}

size_t head16_lds(const llmq_mat *w) {
    const int R = w->ggml_type == LLMQ_GGML_Q6_K ? Unit<LLMQ_GGML_Q6_K>::R : Unit<LLMQ_GGML_Q8_0>::R;
    return (size_t)w->k * 2 + (size_t)R * 256 * 4 + (size_t)R * 16 * 4;
}

template <int TYPE>
int launch_t(llmq_ctx *ctx, const H16Args &a, int ntiles, int T, size_t lds) {
    static size_t granted = 64 * 1024;
    if (lds > granted) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gguf_head16_kernel<TYPE>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    hipLaunchKernelGGL(gguf_head16_kernel<TYPE>, dim3(ntiles, (T + a.tpb - 1) / a.tpb), dim3(kNW * 64), lds,
                       ctx->stream, a);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

}  // namespace

int gguf_has_i16(const llmq_mat *w) {
    return w && w->kind == MAT_GGUF && (w->ggml_type == LLMQ_GGML_Q6_K || w->ggml_type == LLMQ_GGML_Q8_0);
}

int launch_gguf_head16(llmq_ctx *ctx, const llmq_mat *w, const float *h, float *logits, int64_t T,
                       const float *rms_g, float rms_eps) {
    LLMQ_REQUIRE(gguf_has_i16(w), "gguf head: only Q6_K and Q8_0 have an int16 kernel");
    LLMQ_REQUIRE(h && logits && T > 0 && T <= 65535, "gguf head: bad arguments");
    const size_t lds = head16_lds(w);
    int dev = 0, cap = 0;
    LLMQ_HIP(hipGetDevice(&dev));
    LLMQ_HIP(hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    LLMQ_REQUIRE(lds <= (size_t)cap, "gguf head: %lld columns need %zu bytes of LDS (have %d)", (long long)w->k, lds,
                 cap);
    const int64_t ntc = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 16;
    const int64_t nts = (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16;
    LLMQ_REQUIRE(ntc * 16 < (int64_t)kOOB, "gguf head: matrix too large for 32-bit offsets");
    H16Args a{};
    a.codes = w->codes;
    a.codes_bytes = (uint32_t)(ntc * 16);
    a.V = (int)w->n;
    a.C = (int)w->k;
    a.CK = (int)w->CK;
    a.h = h;
    a.logits = logits;
    a.T = (int)T;
    a.tpb = T < 8 ? (int)T : 8;
    a.rms_g = rms_g;
    a.rms_eps = rms_eps;
    if (w->ggml_type == LLMQ_GGML_Q6_K) {
        a.bits = reinterpret_cast<const uint8_t *>(w->g_bits64);
        a.bits_bytes = (uint32_t)(ntc * 8);
        a.sb = reinterpret_cast<const uint8_t *>(w->g_sb16);
        a.sb_bytes = (uint32_t)(nts * 16);
        a.d = reinterpret_cast<const uint8_t *>(w->g_meta16);
        a.d_bytes = (uint32_t)(nts * 2);
        a.NU = (int)w->NG;
        return launch_t<LLMQ_GGML_Q6_K>(ctx, a, (int)w->ntiles, (int)T, lds);
    }
    a.d = reinterpret_cast<const uint8_t *>(w->g_meta16);
    a.d_bytes = (uint32_t)(ntc * 2);
    a.NU = (int)(w->k / 32);
    return launch_t<LLMQ_GGML_Q8_0>(ctx, a, (int)w->ntiles, (int)T, lds);
}
