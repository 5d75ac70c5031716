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
// Work mapping: 4-wave workgroups, a wave per 16-row tile at a time
// (gguf_head16_kernel).  Thread (r, q) of a wave (r = lane % 16, q = lane /
// 16) computes lanes 4q..4q+3 of row r for every unit in order, so each
// lane's float chain and the 16-lane sum stay in registers; Q6_K reads dword
// q of each of the unit's 8 chunks of 32 codes (weights 8q..8q+7) and the
// matching 16 high bits, Q8_0 bytes 8(q%2)..+7 of half 2u + q/2.
#include "common.h"

namespace {

constexpr uint32_t kOOB = 0x80000000u;
constexpr int kNW = 4;    // waves per workgroup
constexpr int kMaxC = 4096;  // longest row the kernel takes

typedef short short2v __attribute__((ext_vector_type(2)));

struct H16Args {
    const uint8_t *codes, *bits, *sb, *d;
    uint32_t codes_bytes, bits_bytes, sb_bytes, d_bytes;
    int V, C, CK, NU, T, ntiles;
    const float *h;
    float *logits;
    const float *rms_g;  // optional RMSNorm gain applied to h first
    float rms_eps;
    ArgmaxPart *amax;    // optional per-workgroup argmax partials
    int vgrid;           // gguf_head16_mf_kernel: the workgroups of gguf_head16_kernel it stands in for
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
// The head's weights, read once a step: non-temporal loads (the caches keep
// the activations and the small tensors instead).
__device__ __forceinline__ uint4 bload16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 bload8_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 2);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t bload4_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 2);
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

// A unit's raw fields as thread (r, q) of a wave reads them: row r of the
// tile, lanes 4q..4q+3 of the unit's int32 accumulator.  Q6_K: dword q of
// each of the superblock's 8 chunks of 32 codes (weights 8q..8q+7 of the
// chunk) and the matching 16 high bits, the 16 int8 scales, d; Q8_0: bytes
// 8(q%2)..+7 of half 2u + q/2 of the block (weights 8q..8q+7) and d.
template <int TYPE>
struct RawUnit;
template <>
struct RawUnit<LLMQ_GGML_Q6_K> {
    uint32_t cw[8], hw[8];
    uint4 sc;
    uint32_t dw;
};
template <>
struct RawUnit<LLMQ_GGML_Q8_0> {
    uint2 cw;
    uint32_t dw;
};

// Loads of unit u of tile `tile` (nothing read when !ok: out-of-range
// offsets return zeros).
template <int TYPE>
__device__ __forceinline__ RawUnit<TYPE> load_unit(const H16Args &a, bool ok, int tile, int u, int r, int q) {
    RawUnit<TYPE> w;
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rd = make_rsrc(a.d, a.d_bytes);
    if constexpr (TYPE == LLMQ_GGML_Q6_K) {
        const auto rb = make_rsrc(a.bits, a.bits_bytes);
        const auto rs = make_rsrc(a.sb, a.sb_bytes);
        const uint32_t c0 = (uint32_t)tile * (uint32_t)a.CK + 8u * (uint32_t)u;  // the unit's first chunk
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const uint32_t e = (c0 + c) * 16u + (uint32_t)r;  // (chunk, row) entry
            w.cw[c] = bload4_nt(rc, ok ? e * 16u + 4u * (uint32_t)q : kOOB);
            w.hw[c] = bload4_nt(rb, ok ? e * 8u + 4u * (uint32_t)(q >> 1) : kOOB);
        }
        const uint32_t se = ((uint32_t)tile * (uint32_t)a.NU + (uint32_t)u) * 16u + (uint32_t)r;
        w.sc = bload16_nt(rs, ok ? se * 16u : kOOB);
        w.dw = bload4_nt(rd, ok ? (se * 2u) & ~3u : kOOB);
    } else {
        const uint32_t e = ((uint32_t)tile * (uint32_t)a.CK + 2u * (uint32_t)u + (uint32_t)(q >> 1)) * 16u + (uint32_t)r;
        w.cw = bload8_nt(rc, ok ? e * 16u + 8u * (uint32_t)(q & 1) : kOOB);
        const uint32_t de = ((uint32_t)tile * (uint32_t)(a.CK / 2) + (uint32_t)u) * 16u + (uint32_t)r;
        w.dw = bload4_nt(rd, ok ? (de * 2u) & ~3u : kOOB);
    }
    return w;
}

// Q6_K: the unit's weights (q - 32) * sc as int16 pairs, wp[c][j] = weights
// 8q + 2j, 8q + 2j + 1 of chunk c, |.| <= 4096.
__device__ __forceinline__ void q6k_pairs(const RawUnit<LLMQ_GGML_Q6_K> &w, int q, uint32_t (&wp)[8][4]) {
    const uint32_t scw[4] = {w.sc.x, w.sc.y, w.sc.z, w.sc.w};
#pragma unroll
    for (int c = 0; c < 8; c++) {
        // int8 scale of this chunk's half: scale 2c + (weights >= 16)
        const uint32_t sbyte = (scw[c >> 1] >> (8 * (2 * (c & 1) + (q >> 1)))) & 255u;
        const uint32_t s16 = (uint32_t)(int)(int8_t)sbyte & 0xFFFFu;
        const uint32_t spair = s16 | (s16 << 16);
        const uint32_t hb = w.hw[c] >> (16 * (q & 1));  // 2 high bits of weight 8q + i at bits 2i
        const uint32_t qe = (w.cw[c] & 0x0F0F0F0Fu) | spread2(hb);             // even weights, 6-bit codes
        const uint32_t qo = ((w.cw[c] >> 4) & 0x0F0F0F0Fu) | spread2(hb >> 2);  // odd weights
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // [q_e, 0, q_o, 0]: the pair as two 16-bit codes
            const uint32_t sel = (uint32_t)j | (0x0Cu << 8) | ((uint32_t)(4 + j) << 16) | (0x0Cu << 24);
            short2v v = __builtin_bit_cast(short2v, __builtin_amdgcn_perm(qo, qe, sel)) - (short2v){32, 32};
            v = v * __builtin_bit_cast(short2v, spair);
            wp[c][j] = __builtin_bit_cast(uint32_t, v);
        }
    }
}

// quantize_rows (kernels.mojo:400-416) of a token's row (after the
// optional RMSNorm): s = max|h| / 32767 (1 if zero), codes round(h / s) as
// int16 pairs into xt, s into *sx.  COOP: the whole workgroup (me = thread),
// else one wave (me = lane); the row stays in registers, RV float4 a thread
// (load_token).
template <int RV, bool G>
struct TokenRow {
    float4 v[RV], g[G ? RV : 1];  // the thread's part of the row (and of the RMSNorm gain, G)
};

template <int RV, bool COOP>
__device__ __forceinline__ TokenRow<RV, COOP> load_token(const H16Args &a, int t, int me) {
    constexpr int NTH = COOP ? kNW * 64 : 64;
    const int n4 = a.C / 4;
    const float4 *h4 = reinterpret_cast<const float4 *>(a.h + (size_t)t * a.C);
    const float4 *g4 = reinterpret_cast<const float4 *>(a.rms_g);
    TokenRow<RV, COOP> row;
#pragma unroll
    for (int k = 0; k < RV; k++) {
        const int i = me + k * NTH;
        row.v[k] = i < n4 ? h4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (COOP) row.g[k] = a.rms_g && i < n4 ? g4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    return row;
}

template <int RV, bool COOP, class ST>
__device__ __forceinline__ void quantize_token(const H16Args &a, TokenRow<RV, COOP> row, int me, ST &&store,
                                               float *s_red, float *sx_out) {
    constexpr int NTH = COOP ? kNW * 64 : 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int n4 = a.C / 4;
    float4 *v = row.v;
    if (a.rms_g) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < RV; k++) {
            ss = fmaf(v[k].x, v[k].x, ss);
            ss = fmaf(v[k].y, v[k].y, ss);
            ss = fmaf(v[k].z, v[k].z, ss);
            ss = fmaf(v[k].w, v[k].w, ss);
        }
        ss = llmq_wave_sum_all(ss);
        if (COOP) {
            if (lane == 0) s_red[wid] = ss;
            __syncthreads();
            ss = ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];
            __syncthreads();
        }
        const float rn = 1.0f / sqrtf(ss / (float)a.C + a.rms_eps);
#pragma unroll
        for (int k = 0; k < RV; k++) {
            const int i = me + k * NTH;
            if (i < n4) {
                float4 gg;
                if constexpr (COOP)
                    gg = row.g[k];
                else
                    gg = reinterpret_cast<const float4 *>(a.rms_g)[i];
                v[k].x = (v[k].x * rn) * gg.x;
                v[k].y = (v[k].y * rn) * gg.y;
                v[k].z = (v[k].z * rn) * gg.z;
                v[k].w = (v[k].w * rn) * gg.w;
            }
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < RV; k++)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)), fmaxf(fabsf(v[k].z), fabsf(v[k].w))));
    m = llmq_wave_max_all(m);
    if (COOP) {
        if (lane == 0) s_red[wid] = m;
        __syncthreads();
        m = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
        __syncthreads();
    }
    float sx = m / 32767.0f;
    if (sx == 0.0f) sx = 1.0f;
    const float inv = 1.0f / sx;
#pragma unroll
    for (int k = 0; k < RV; k++) {
        const int i = me + k * NTH;
        if (i < n4) {
            const int q0 = round_to_int(v[k].x * inv), q1 = round_to_int(v[k].y * inv);
            const int q2 = round_to_int(v[k].z * inv), q3 = round_to_int(v[k].w * inv);
            store(i, q0, q1, q2, q3);
        }
    }
    if (me == 0) *sx_out = sx;
}

// quantize_token's store into int16 pairs: inputs 4 i .. 4 i + 3 of the row.
struct PairStore {
    uint32_t *xt;
    __device__ __forceinline__ void operator()(int i, int q0, int q1, int q2, int q3) const {
        *reinterpret_cast<uint2 *>(xt + 2 * i) = make_uint2(((uint32_t)q0 & 0xFFFFu) | ((uint32_t)q1 << 16),
                                                            ((uint32_t)q2 & 0xFFFFu) | ((uint32_t)q3 << 16));
    }
};

// One workgroup of kNW waves; wave g = blockIdx.x * kNW + wid takes tiles
// g, g + G, .. (G = gridDim.x * kNW) and streams their units in order, the
// loads of the next PD units in flight while one is computed.  Thread
// (r = lane % 16, q = lane / 16) keeps lanes 4q..4q+3 of row r's float
// chain for each of up to TM tokens (tokens blockIdx.y * TM ..): the chain
// over units and the 16-lane sum stay in registers and shuffles.  The
// tokens are normalized and quantized once per workgroup, a wave a token.
// With amax set, each workgroup also leaves the largest logit of each token
// over its tiles (and its smallest row) in amax[token * gridDim.x + wg].
template <int TYPE, int TM>
__global__ __launch_bounds__(kNW * 64) void gguf_head16_kernel(H16Args a) {
    extern __shared__ __align__(16) uint32_t xq32[];  // [TM][C / 2] int16 pairs
    __shared__ float s_sx[TM], s_red[kNW];
    __shared__ ArgmaxPart s_best[kNW][TM];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int t0 = blockIdx.y * TM, nt = min(TM, a.T - t0);
    const int C2 = a.C / 2, NU = a.NU;
    const int g = blockIdx.x * kNW + wid, G = gridDim.x * kNW;
    // unit stream: item s is unit s % NU of tile g + (s / NU) * G
    auto item_tile = [&](int s) { return g + (s / NU) * G; };
    auto load_item = [&](int s) {
        const int tile = item_tile(s);
        return load_unit<TYPE>(a, tile < a.ntiles, tile, s % NU, r, q);
    };
    constexpr int PD = TM <= 2 ? 3 : 2;  // units in flight behind the one computed
    constexpr int RVC = kMaxC / 4 / (kNW * 64);
    // The first token's row goes out before the weights when the workgroup
    // takes fewer tokens than it has waves (loads complete in issue order).
    const bool coop = TM < kNW || nt < kNW;
    TokenRow<RVC, true> first;
    if constexpr (TM < kNW) first = load_token<RVC, true>(a, t0, tid);
    RawUnit<TYPE> ring[PD];
#pragma unroll
    for (int k = 0; k < PD; k++) ring[k] = load_item(k);

    // Tokens: optional RMSNorm, then quantize_rows (kernels.mojo:400-416).
    // Fewer tokens than waves: the workgroup takes them one by one; else a
    // wave per token.
    if (coop) {
        for (int t = 0; t < nt; t++)
            quantize_token<RVC, true>(a, TM < kNW && t == 0 ? first : load_token<RVC, true>(a, t0 + t, tid), tid,
                                      PairStore{xq32 + (size_t)t * C2}, s_red, &s_sx[t]);
    } else {
        for (int t = wid; t < nt; t += kNW)
            quantize_token<kMaxC / 4 / 64, false>(a, load_token<kMaxC / 4 / 64, false>(a, t0 + t, lane), lane,
                                                  PairStore{xq32 + (size_t)t * C2}, s_red, &s_sx[t]);
    }
    __syncthreads();
    float sx[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) sx[t] = s_sx[t < nt ? t : 0];

    float accf[TM][4];
    float best_v[TM];
    int best_i[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) {
#pragma unroll
        for (int j = 0; j < 4; j++) accf[t][j] = 0.0f;
        best_v[t] = -INFINITY;
        best_i[t] = 0x7fffffff;
    }
    for (int s0 = 0;; s0 += PD) {
#pragma unroll
    for (int k = 0; k < PD; k++) {
        const int s = s0 + k;
        const int tile = item_tile(s);
        if (tile >= a.ntiles) goto done;  // uniform over the wave
        const int u = s % NU;
        const RawUnit<TYPE> b0 = ring[k];
        ring[k] = load_item(s + PD);
        if constexpr (TYPE == LLMQ_GGML_Q6_K) {
            const float d = h2f(b0.dw >> (16 * (r & 1)));
            uint32_t wp[8][4];
            q6k_pairs(b0, q, wp);
#pragma unroll
            for (int t = 0; t < TM; t++) {
                if (t < nt) {
                    const uint32_t *xt = xq32 + (size_t)t * C2 + 128 * u + 4 * q;
                    int acc[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int c = 0; c < 8; c++) {
                        const uint4 xv = *reinterpret_cast<const uint4 *>(xt + 16 * c);
                        acc[0] = sdot2(xv.x, wp[c][0], acc[0]);
                        acc[1] = sdot2(xv.y, wp[c][1], acc[1]);
                        acc[2] = sdot2(xv.z, wp[c][2], acc[2]);
                        acc[3] = sdot2(xv.w, wp[c][3], acc[3]);
                    }
#pragma unroll
                    for (int j = 0; j < 4; j++) accf[t][j] = fmaf((float)acc[j], d, accf[t][j]);
                }
            }
        } else {
            // codes in the high byte of each 16-bit half (256 * code): one
            // dot gives 256 * (x0 w0 + x1 w1), |.| < 2^31, and the shift by
            // 8 is exact
            const float d = h2f(b0.dw >> (16 * (r & 1)));
            const uint32_t ww[2] = {b0.cw.x, b0.cw.y};
            uint32_t wp[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t bb = 2u * (uint32_t)(j & 1);  // pair j: bytes 2j, 2j + 1 of the 8
                wp[j] = __builtin_amdgcn_perm(0u, ww[j >> 1], 0x0Cu | (bb << 8) | (0x0Cu << 16) | ((bb + 1u) << 24));
            }
#pragma unroll
            for (int t = 0; t < TM; t++) {
                if (t < nt) {
                    const uint4 xv = *reinterpret_cast<const uint4 *>(xq32 + (size_t)t * C2 + 16 * u + 4 * q);
                    const uint32_t xp[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                    for (int j = 0; j < 4; j++) accf[t][j] = fmaf((float)(sdot2(xp[j], wp[j], 0) >> 8), d, accf[t][j]);
                }
            }
        }
        if (u == NU - 1) {
            // red16 (lane L = 4q + j): v[L] + v[L + 8] (q ^ 2), then + 4
            // (q ^ 1), + 2 and + 1 (j) on q == 0
            const int row = tile * 16 + r;
#pragma unroll
            for (int t = 0; t < TM; t++) {
                if (t < nt) {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        // lane ^ 32, then lane ^ 16: gfx950's half-wave and row-pair swaps
                        const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(accf[t][j]),
                                                                          __float_as_uint(accf[t][j]), false, false);
                        v[j] = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
                        const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j]),
                                                                          false, false);
                        v[j] = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
                        accf[t][j] = 0.0f;
                    }
                    const float lg = ((v[0] + v[2]) + (v[1] + v[3])) * sx[t];
                    if (q == 0 && row < a.V) {
                        a.logits[(size_t)(t0 + t) * a.V + row] = lg;
                        if (lg > best_v[t] || (lg == best_v[t] && row < best_i[t])) {
                            best_v[t] = lg;
                            best_i[t] = row;
                        }
                    }
                }
            }
        }
    }
    }
done:
    if (!a.amax) return;
#pragma unroll
    for (int t = 0; t < TM; t++) {
        float bv = best_v[t];
        int bi = best_i[t];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bi, o);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) s_best[wid][t] = ArgmaxPart{bv, bi};
    }
    __syncthreads();
    if (tid < nt) {
        ArgmaxPart b = s_best[0][tid];
#pragma unroll
        for (int w = 1; w < kNW; w++) {
            const ArgmaxPart c = s_best[w][tid];
            if (c.v > b.v || (c.v == b.v && c.idx < b.idx)) b = c;
        }
        a.amax[(size_t)(t0 + tid) * gridDim.x + blockIdx.x] = b;
    }
}

// ------------------------------------------- Q6_K on the fp16 matrix cores
//
// A token tile of 9 to 16 tokens (the rest zero) over a Q6_K head of up to
// 2048 columns, with the integers and float steps of gguf_head16_kernel and
// the lane sums on the matrix cores.  Lane L of superblock u sums
// acc[L] = sum x_k w_k over the 16 inputs k = 32 c + 2 L + i (chunks c =
// 0..7, i = 0, 1), w = (q - 32) s with s the int8 scale of the input's
// 16-weight half.  Split x = 256 xh + xl (xh = x >> 8, xl = x & 255) and
// s = 8 sh + sl (sh = s >> 3, sl = s & 7): xh, xl, q' (8 sh) and q' sl
// (q' = q - 32) are exact in fp16 and w = q' (8 sh) + q' sl, so two
// chained v_mfma_f32_16x16x16_f16 a plane form
//     P = sum xh w  (|P| <= 16 * 128 * 4096 = 2^23)
//     Q = sum xl w  (|Q| <= 16 * 255 * 4096 < 2^24; every partial sum stays
//                    below 2^24 too: |q' (8 sh)| >= |q' sl| wherever the
//                    two differ in sign)
// exactly, and fma(256, P, Q) is acc rounded once, the reference's
// (float)acc[L]; then accf[L] = fma(., d, accf[L]) and red16 as there.
//
// Lane l (r = l % 16, g = l / 16), lane sum L: A (tokens x the 16 inputs)
// holds 4 fp16 of token r, inputs m = 0..3 = (chunk 2 g + m / 2, weight
// 2 L + m % 2); B the same inputs of row r; D rows r, tokens 4 g .. 4 g + 3.
// The tokens' hi / lo planes sit in LDS as fp16 [plane][u][L][g][token][4]
// (128 KB at 2048 columns), written by the prologue (a wave a token, the
// arithmetic of gguf_head16_kernel's).  Workgroups of 8 waves: waves 0-3
// and 4-7 stand in for workgroups 2 b and 2 b + 1 of gguf_head16_kernel's
// grid (a.vgrid), taking its tiles and leaving its argmax partials.
constexpr int kMfNW = 8;
constexpr int kMfMaxC = 2048;

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// The prologue's store: codes q of inputs 4 i .. 4 i + 3 of token t as
// their hi and lo fp16 values at the A operand's places.
struct PlaneStore {
    uint32_t *pl;  // [2][plane_dw]
    uint32_t plane_dw;
    int t;
    __device__ __forceinline__ static uint32_t pair(int a, int b) {
        const _Float16 ha = (_Float16)(float)a, hb = (_Float16)(float)b;
        return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
    }
    __device__ __forceinline__ void operator()(int i, int q0, int q1, int q2, int q3) const {
        const int k = 4 * i, u = k >> 8, c = (k >> 5) & 7, L = (k & 31) >> 1;
        // fp16 index of (u, L, g = c / 2, t, m = 2 (c % 2)); pair L + 1 is 256 further
        const uint32_t f = ((((uint32_t)u * 16u + (uint32_t)L) * 4u + (uint32_t)(c >> 1)) * 16u + (uint32_t)t) * 4u +
                           2u * (uint32_t)(c & 1);
        pl[f / 2] = pair(q0 >> 8, q1 >> 8);
        pl[f / 2 + 128] = pair(q2 >> 8, q3 >> 8);
        pl[plane_dw + f / 2] = pair(q0 & 255, q1 & 255);
        pl[plane_dw + f / 2 + 128] = pair(q2 & 255, q3 & 255);
    }
};

// A unit's fields for lane (r, g): chunks 2 g and 2 g + 1 of row r (codes
// and high bits), the four scales of their halves, d.
struct MfUnit {
    uint4 c0, c1;
    uint2 h0, h1;
    uint32_t sc, dw;
};

__global__ __launch_bounds__(kMfNW * 64) void gguf_head16_mf_kernel(H16Args a) {
    extern __shared__ __align__(16) uint32_t pl[];  // fp16 [2][NU][16][4][16][4]
    __shared__ float s_sx[16];
    __shared__ ArgmaxPart s_best[kMfNW][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int t0 = blockIdx.y * 16, nt = min(16, a.T - t0);
    const int NU = a.NU;
    const uint32_t plane_dw = (uint32_t)NU * 2048u;
    const int v = 2 * (int)blockIdx.x + (wid >> 2);  // the gguf_head16_kernel workgroup this wave belongs to
    const bool vlive = v < a.vgrid;
    const int vw = v * kNW + (wid & 3), G = a.vgrid * kNW;
    const auto rc = make_rsrc(a.codes, a.codes_bytes);
    const auto rb = make_rsrc(a.bits, a.bits_bytes);
    const auto rs = make_rsrc(a.sb, a.sb_bytes);
    const auto rd = make_rsrc(a.d, a.d_bytes);
    auto item_tile = [&](int s) { return vw + (s / NU) * G; };
    auto load_mf = [&](int s) {
        const int tile = item_tile(s), u = s % NU;
        const bool ok = vlive && tile < a.ntiles;
        const uint32_t e0 = ((uint32_t)tile * (uint32_t)a.CK + 8u * (uint32_t)u + 2u * (uint32_t)g) * 16u + (uint32_t)r;
        const uint32_t se = ((uint32_t)tile * (uint32_t)NU + (uint32_t)u) * 16u + (uint32_t)r;
        MfUnit w;
        w.c0 = bload16_nt(rc, ok ? e0 * 16u : kOOB);
        w.c1 = bload16_nt(rc, ok ? (e0 + 16u) * 16u : kOOB);
        w.h0 = bload8_nt(rb, ok ? e0 * 8u : kOOB);
        w.h1 = bload8_nt(rb, ok ? (e0 + 16u) * 8u : kOOB);
        w.sc = bload4_nt(rs, ok ? se * 16u + 4u * (uint32_t)g : kOOB);
        w.dw = bload4_nt(rd, ok ? (se * 2u) & ~3u : kOOB);
        return w;
    };
    constexpr int PD = 2;
    MfUnit ring[PD];
#pragma unroll
    for (int k = 0; k < PD; k++) ring[k] = load_mf(k);

    // Tokens wid and wid + 8: optional RMSNorm, quantize_rows, the planes
    // (zeros for tokens past the batch).
    for (int t = wid; t < 16; t += kMfNW) {
        if (t < nt) {
            quantize_token<kMaxC / 4 / 64, false>(a, load_token<kMaxC / 4 / 64, false>(a, t0 + t, lane), lane,
                                                  PlaneStore{pl, plane_dw, t}, nullptr, &s_sx[t]);
        } else {
            for (uint32_t e = (uint32_t)lane; e < (uint32_t)NU * 64u; e += 64u) {  // entries (u, L, g) of token t
                const uint32_t f = (e * 16u + (uint32_t)t) * 2u;
                pl[f] = 0u;
                pl[f + 1] = 0u;
                pl[plane_dw + f] = 0u;
                pl[plane_dw + f + 1] = 0u;
            }
            if (lane == 0) s_sx[t] = 0.0f;
        }
    }
    __syncthreads();
    float sxl[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sxl[i] = s_sx[4 * g + i];

    float accf[16][4];
    float best_v[4];
    int best_i[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int L = 0; L < 16; L++) accf[L][i] = 0.0f;
        best_v[i] = -INFINITY;
        best_i[i] = 0x7fffffff;
    }
    const v4h k1056 = {(_Float16)1056.0f, (_Float16)1056.0f, (_Float16)1056.0f, (_Float16)1056.0f};
    for (int s0 = 0;; s0 += PD) {
#pragma unroll
    for (int k = 0; k < PD; k++) {
        const int s = s0 + k;
        const int tile = item_tile(s);
        if (!vlive || tile >= a.ntiles) goto done;  // uniform over the wave
        const int u = s % NU;
        const MfUnit w = ring[k];
        ring[k] = load_mf(s + PD);
        const float d = h2f(w.dw >> (16 * (r & 1)));
        // scale pieces of half h of chunks 2 g, 2 g + 1 (bytes h, 2 + h of sc),
        // laid out as B's four inputs
        v4h m1[2], m2[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int s0 = (int)(int8_t)((w.sc >> (8 * h)) & 255u), s1 = (int)(int8_t)((w.sc >> (8 * (2 + h))) & 255u);
            const _Float16 a0 = (_Float16)(float)(8 * (s0 >> 3)), a1 = (_Float16)(float)(8 * (s1 >> 3));
            const _Float16 b0 = (_Float16)(float)(s0 & 7), b1 = (_Float16)(float)(s1 & 7);
            m1[h] = (v4h){a0, a0, a1, a1};
            m2[h] = (v4h){b0, b0, b1, b1};
        }
        // 6-bit codes, bytes: qe[cc][j] byte k = weight 2 (4 j + k), qo the next one
        uint32_t qe[2][4], qo[2][4];
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
            const uint32_t cw[4] = {cc ? w.c1.x : w.c0.x, cc ? w.c1.y : w.c0.y, cc ? w.c1.z : w.c0.z,
                                    cc ? w.c1.w : w.c0.w};
            const uint32_t hw[2] = {cc ? w.h1.x : w.h0.x, cc ? w.h1.y : w.h0.y};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t hb = hw[j >> 1] >> (16 * (j & 1));
                qe[cc][j] = (cw[j] & 0x0F0F0F0Fu) | spread2(hb);
                qo[cc][j] = ((cw[j] >> 4) & 0x0F0F0F0Fu) | spread2(hb >> 2);
            }
        }
        const uint32_t *ph = pl + (uint32_t)u * 2048u + (uint32_t)lane * 2u;  // (u, L = 0, g, token r)
#pragma unroll
        for (int L = 0; L < 16; L++) {
            const int j = L >> 2, kk = L & 3, h = L >> 3;
            const uint32_t sel = (uint32_t)kk | (0x0Cu << 8) | ((uint32_t)(4 + kk) << 16) | (0x0Cu << 24);
            // q' of B's inputs m = 0..3 (chunk 2 g + m / 2, weight 2 L + m % 2)
            const uint2 raw = make_uint2(__builtin_amdgcn_perm(qo[0][j], qe[0][j], sel) | 0x64006400u,
                                         __builtin_amdgcn_perm(qo[1][j], qe[1][j], sel) | 0x64006400u);
            const v4h q4 = __builtin_bit_cast(v4h, raw) - k1056;
            const v4h B1 = q4 * m1[h], B2 = q4 * m2[h];
            const uint2 xh = *reinterpret_cast<const uint2 *>(ph + L * 128);
            const uint2 xl = *reinterpret_cast<const uint2 *>(ph + plane_dw + L * 128);
            const v4h Ah = __builtin_bit_cast(v4h, xh), Al = __builtin_bit_cast(v4h, xl);
            const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
            v4f P = __builtin_amdgcn_mfma_f32_16x16x16f16(Ah, B1, z, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x16f16(Ah, B2, P, 0, 0, 0);
            v4f Q = __builtin_amdgcn_mfma_f32_16x16x16f16(Al, B1, z, 0, 0, 0);
            Q = __builtin_amdgcn_mfma_f32_16x16x16f16(Al, B2, Q, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) accf[L][i] = fmaf(fmaf(256.0f, P[i], Q[i]), d, accf[L][i]);
        }
        if (u == NU - 1) {  // red16 (kernels.mojo red16's halving order), times sx
            const int row = tile * 16 + r;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 4 * g + i;
                float a8[8], b4[4];
#pragma unroll
                for (int L = 0; L < 8; L++) a8[L] = accf[L][i] + accf[L + 8][i];
#pragma unroll
                for (int L = 0; L < 4; L++) b4[L] = a8[L] + a8[L + 4];
                const float lg = ((b4[0] + b4[2]) + (b4[1] + b4[3])) * sxl[i];
#pragma unroll
                for (int L = 0; L < 16; L++) accf[L][i] = 0.0f;
                if (t < nt && row < a.V) {
                    a.logits[(size_t)(t0 + t) * a.V + row] = lg;
                    if (lg > best_v[i] || (lg == best_v[i] && row < best_i[i])) {
                        best_v[i] = lg;
                        best_i[i] = row;
                    }
                }
            }
        }
    }
    }
done:
    if (!a.amax) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float bv = best_v[i];
        int bi = best_i[i];
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {  // over the 16 rows of the lane group
            const float ov = __shfl_xor(bv, o);
            const int oi = __shfl_xor(bi, o);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (r == 0) s_best[wid][4 * g + i] = ArgmaxPart{bv, bi};
    }
    __syncthreads();
    if (tid < 32) {
        const int half = tid >> 4, t = tid & 15, vv = 2 * (int)blockIdx.x + half;
        if (vv < a.vgrid && t < nt) {
            ArgmaxPart b = s_best[4 * half][t];
#pragma unroll
            for (int w = 1; w < kNW; w++) {
                const ArgmaxPart c = s_best[4 * half + w][t];
                if (c.v > b.v || (c.v == b.v && c.idx < b.idx)) b = c;
            }
            a.amax[(size_t)(t0 + t) * a.vgrid + vv] = b;
        }
    }
}

// Tokens a workgroup takes (the register chains per thread).
int head16_tm(int64_t T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : T <= 8 ? 8 : 16; }

// Workgroups: enough waves for every tile once, at most 512 workgroups
// (then waves take several tiles); LLMQ_HEAD16_GRID overrides.
int head16_grid(const llmq_mat *w) {
    int g = (int)std::min<int64_t>((w->ntiles + kNW - 1) / kNW, 512);
    if (const char *e = getenv("LLMQ_HEAD16_GRID")) {
        const int v = atoi(e);
        if (v >= 1 && v <= 4096) g = v;
    }
    return std::max(g, 1);
}

template <int TYPE, int TM>
int launch_tm(llmq_ctx *ctx, const H16Args &a, int grid, int T) {
    const size_t lds = (size_t)TM * a.C * 2;
    static size_t granted = 64 * 1024;  // one host thread per context
    if (lds > granted) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gguf_head16_kernel<TYPE, TM>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    hipLaunchKernelGGL((gguf_head16_kernel<TYPE, TM>), dim3(grid, (T + TM - 1) / TM), dim3(kNW * 64), lds,
                       ctx->stream, a);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

// gguf_head16_mf_kernel for 9 to 16 tokens a tile of a Q6_K head of up to
// 2048 columns (LLMQ_HEAD16_MF=0: gguf_head16_kernel throughout).
int launch_mf(llmq_ctx *ctx, H16Args a, int grid, int T) {
    a.vgrid = grid;
    const size_t lds = (size_t)a.NU * 16384;  // two fp16 planes of 16 tokens
    static size_t granted = 64 * 1024;      // one host thread per context
    if (lds > granted) {
        LLMQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(gguf_head16_mf_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        granted = lds;
    }
    hipLaunchKernelGGL(gguf_head16_mf_kernel, dim3((grid + 1) / 2, (T + 15) / 16), dim3(kMfNW * 64), lds, ctx->stream,
                       a);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

bool mf_ok(const H16Args &a, int T, int lds_cap) {
    if (const char *e = getenv("LLMQ_HEAD16_MF"))
        if (e[0] == '0') return false;
    return head16_tm(T) == 16 && a.C <= kMfMaxC && a.C % 256 == 0 && (size_t)a.NU * 16384 + 2048 <= (size_t)lds_cap;
}

template <int TYPE>
int launch_t(llmq_ctx *ctx, const H16Args &a, int grid, int T, int lds_cap) {
    if constexpr (TYPE == LLMQ_GGML_Q6_K)
        if (mf_ok(a, T, lds_cap)) return launch_mf(ctx, a, grid, T);
    switch (head16_tm(T)) {
    case 1: return launch_tm<TYPE, 1>(ctx, a, grid, T);
    case 2: return launch_tm<TYPE, 2>(ctx, a, grid, T);
    case 4: return launch_tm<TYPE, 4>(ctx, a, grid, T);
    case 8: return launch_tm<TYPE, 8>(ctx, a, grid, T);
    default: return launch_tm<TYPE, 16>(ctx, a, grid, T);
    }
}

}  // namespace

int gguf_has_i16(const llmq_mat *w) {
    return w && w->kind == MAT_GGUF && (w->ggml_type == LLMQ_GGML_Q6_K || w->ggml_type == LLMQ_GGML_Q8_0);
}

int gguf_head16_parts(const llmq_mat *w) { return head16_grid(w); }

int launch_gguf_head16(llmq_ctx *ctx, const llmq_mat *w, const float *h, float *logits, int64_t T,
                       const float *rms_g, float rms_eps, ArgmaxPart *amax, int amax_cap) {
    LLMQ_REQUIRE(gguf_has_i16(w), "gguf head: only Q6_K and Q8_0 have an int16 kernel");
    LLMQ_REQUIRE(h && logits && T > 0 && (T + 15) / 16 <= 65535, "gguf head: bad arguments");
    LLMQ_REQUIRE(w->k <= kMaxC, "gguf head: %lld columns beyond %d", (long long)w->k, kMaxC);
    const int grid = head16_grid(w);
    LLMQ_REQUIRE(!amax || (int64_t)grid * T <= amax_cap, "gguf head: argmax capacity %d below %lld", amax_cap,
                 (long long)grid * T);
    const size_t lds = (size_t)head16_tm(T) * w->k * 2;
    int dev = 0, cap = 0;
    LLMQ_HIP(hipGetDevice(&dev));
    LLMQ_HIP(hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    LLMQ_REQUIRE(lds + 1024 <= (size_t)cap, "gguf head: %lld columns need %zu bytes of LDS (have %d)",
                 (long long)w->k, lds, cap);
    const int64_t ntc = (w->ntiles * w->CK + LLMQ_PAD_CHUNKS) * 16;
    const int64_t nts = (w->ntiles * w->NG + LLMQ_PAD_CHUNKS) * 16;
    LLMQ_REQUIRE(ntc * 16 < (int64_t)kOOB, "gguf head: matrix too large for 32-bit offsets");
    H16Args a{};
    a.codes = w->codes;
    a.codes_bytes = (uint32_t)(ntc * 16);
    a.V = (int)w->n;
    a.C = (int)w->k;
    a.CK = (int)w->CK;
    a.ntiles = (int)w->ntiles;
    a.h = h;
    a.logits = logits;
    a.T = (int)T;
    a.rms_g = rms_g;
    a.rms_eps = rms_eps;
    a.amax = amax;
    if (w->ggml_type == LLMQ_GGML_Q6_K) {
        a.bits = reinterpret_cast<const uint8_t *>(w->g_bits64);
        a.bits_bytes = (uint32_t)(ntc * 8);
        a.sb = reinterpret_cast<const uint8_t *>(w->g_sb16);
        a.sb_bytes = (uint32_t)(nts * 16);
        a.d = reinterpret_cast<const uint8_t *>(w->g_meta16);
        a.d_bytes = (uint32_t)(nts * 2);
        a.NU = (int)w->NG;
        return launch_t<LLMQ_GGML_Q6_K>(ctx, a, grid, (int)T, cap);
    }
    a.d = reinterpret_cast<const uint8_t *>(w->g_meta16);
    a.d_bytes = (uint32_t)(ntc * 2);
    a.NU = (int)(w->k / 32);
    return launch_t<LLMQ_GGML_Q8_0>(ctx, a, grid, (int)T, cap);
}
