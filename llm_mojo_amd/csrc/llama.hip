// A TinyLlama-shaped decoder over GGUF weights: the benchmark's fifth
// configuration (22 layers, d_model 2048, 32 query / 4 key-value heads of 64,
// SwiGLU FFN 5632, RMSNorm, RoPE theta 10000, vocab 32000; Q4_K layers, Q6_K
// head, int8 KV cache), decoding one or several independent sequences.
//
// The reference's model code is GPT-2 only (gpt2t.mojo:74-81), so nothing
// here has a reference counterpart above the kernels it reuses: the GGUF
// GEMV / matmul (GGUFMatrix, gguf.mojo:344-511; matmul_rows,
// kernels.mojo:285-349), the int16 output head (head_i16, kernels.mojo:
// 693-736), the int8 cache (QuantKV[8], kvcache.mojo:248-385) and the float
// attention (attend_float_one, kvcache.mojo:113-150).  The rest follows the
// usual Llama definition:
//   h = x + Wo . attn(rope(Wq . n1), rope(Wk . n1), Wv . n1),  n1 = rmsnorm(x) * g1
//   y = h + Wdown . (silu(Wgate . n2) * (Wup . n2)),           n2 = rmsnorm(h) * g2
//   rmsnorm(x) = x / sqrt(mean(x^2) + eps);  rope rotates dims (2i, 2i+1) by
//   pos * theta^(-2i / head_dim);  silu(g) = g / (1 + exp(-g)).
//
// Device layout: Wq, Wk, Wv are one matrix of n_head + 2 n_kv heads' rows
// (one GEMV per layer); Wgate and Wup one of 2 ffn rows.  The cache is
// head-major: row ((sequence * n_layer + layer) * n_kv + head) * max_t + pos
// of HD int8 codes (and one scale), so a split's rows of one head are one
// contiguous run.  Decoding keeps the
// position and step on the device, so one captured graph replays every step.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "common.h"

namespace {

constexpr int HD = 64;  // head_dim

__device__ __forceinline__ float wave_sum(float v) { return llmq_wave_sum_all(v); }
__device__ __forceinline__ float wave_max(float v) { return llmq_wave_max_all(v); }
// Sum / max over a 256-thread workgroup, waves added in order.
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// out[r] = x[r] / sqrt(mean(x[r]^2) + eps) * g, one workgroup a row.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, int64_t ldx,
                                                      const float *__restrict__ g, float *__restrict__ out,
                                                      int64_t ldo, int C, float eps) {
    __shared__ float red[4];
    const float *xr = x + (int64_t)blockIdx.x * ldx;
    float *orow = out + (int64_t)blockIdx.x * ldo;
    float ss = 0.0f;
    // 8 loads a thread in flight at a time (zeros past C add nothing), in the loop's order
    for (int i0 = threadIdx.x; i0 < C; i0 += 256 * 8) {
        float t[8];
#pragma unroll
        for (int k = 0; k < 8; k++) t[k] = i0 + 256 * k < C ? xr[i0 + 256 * k] : 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) ss = fmaf(t[k], t[k], ss);
    }
    ss = block_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)C + eps);
#pragma unroll 8
    for (int i = threadIdx.x; i < C; i += 256) orow[i] = (xr[i] * r) * g[i];
}

// rmsnorm_kernel's row (x r) g written as the h16 record of the several-row
// Q4_K matmul (llmq_h16_store): one wave a (superblock blockIdx.x, row
// blockIdx.y), each wave forming the row's sum of squares itself
// (C = 256 NSB, a multiple of 256).
__global__ __launch_bounds__(64) void rmsnorm_rec_kernel(const float *__restrict__ x, int64_t ldx,
                                                         const float *__restrict__ g, int C, float eps,
                                                         uint8_t *__restrict__ planes, _Float16 *__restrict__ sums,
                                                         float *__restrict__ inv) {
    const float *xr = x + (int64_t)blockIdx.y * ldx;
    const int lane = threadIdx.x, sb = blockIdx.x;
    // the superblock's inputs and gains, then the row for its sum of squares,
    // 8 float4 a lane in flight at a time (zeros past C add nothing), all
    // before the first use
    float v[4], gv[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        v[q] = xr[sb * 256 + 64 * q + lane];
        gv[q] = g[sb * 256 + 64 * q + lane];
    }
    float ss = 0.0f;
    for (int i0 = 4 * lane; i0 < C; i0 += 256 * 8) {
        float4 t[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            t[k] = i0 + 256 * k < C ? *reinterpret_cast<const float4 *>(xr + i0 + 256 * k)
                                     : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            ss = fmaf(t[k].x, t[k].x, ss);
            ss = fmaf(t[k].y, t[k].y, ss);
            ss = fmaf(t[k].z, t[k].z, ss);
            ss = fmaf(t[k].w, t[k].w, ss);
        }
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)C + eps);
#pragma unroll
    for (int q = 0; q < 4; q++) v[q] = (v[q] * r) * gv[q];
    llmq_h16_store(planes, sums, inv, C / 32, C / 256, blockIdx.y, sb, v, true);
}

// RoPE and the cache store of a prompt: row `row` of qkv is token t = row % T
// of sequence seq0 + row / T, at position pos0 + t.
// query heads are rotated in place; key heads are rotated, then key and
// value heads quantized into the cache as QuantKV.store does
// (kvcache.mojo:320-342: s = max|x| / 127, 1 if zero; codes round(x / s)).
// One wave per (head, row); lane = dim.
__global__ __launch_bounds__(64) void rope_store_kernel(float *__restrict__ qkv, int64_t ld, int T, int seq0,
                                                        int pos0, int n_head,
                                                        int n_kv, int n_layer, int layer, int max_t,
                                                        const float2 *__restrict__ rope, int8_t *__restrict__ K8,
                                                        int8_t *__restrict__ V8, float *__restrict__ KS,
                                                        float *__restrict__ VS) {
    const int hh = blockIdx.x, row = blockIdx.y, d = threadIdx.x;
    const int seq = seq0 + row / T, t = row % T;
    const int pos = pos0 + t;
    float *r = qkv + (int64_t)row * ld;
    const bool is_q = hh < n_head;
    float *src = r + hh * HD;  // query heads, then key heads
    // rotation of pair (2i, 2i + 1), i = d / 2, by the table's angle
    const float2 cs = rope[pos * (HD / 2) + (d >> 1)];
    const float c = cs.x, s = cs.y;
    const float v = src[d], p = llmq_dppf<0xB1>(v);  // lane d ^ 1
    // (x0, x1) -> (x0 c - x1 s, x0 s + x1 c)
    const float rot = (d & 1) ? p * s + v * c : v * c - p * s;
    if (is_q) {
        src[d] = rot;
        return;
    }
    const int kvh = hh - n_head;
    const int64_t sl = (((int64_t)seq * n_layer + layer) * n_kv + kvh) * max_t + pos;
    for (int kv = 0; kv < 2; kv++) {
        const float x = kv == 0 ? rot : r[(n_head + n_kv + kvh) * HD + d];
        const float m = wave_max(fabsf(x));
        float sc = m / 127.0f;
        if (sc == 0.0f) sc = 1.0f;
        const float inv = 1.0f / sc;
        (kv == 0 ? K8 : V8)[sl * HD + d] = (int8_t)llmq_to_int(roundf(x * inv));
        if (d == 0) (kv == 0 ? KS : VS)[sl] = sc;
    }
}

// One decode position for query head h = blockIdx.x of sequence b =
// blockIdx.y at position pos = state[0]: RoPE of the query and of the new
// key, the new key and value quantized into the cache (rope_store_kernel's
// arithmetic), then attend_float_one (kvcache.mojo:113-150) over the int8
// cache (QuantKV.score / add_value, 344-370) of key / value head
// h / (n_head / n_kv), split over blocks of kSplit positions (blockIdx.z),
// a thread a position, so a head's positions are scored on several CUs.  A
// split writes its maximum score m, its sum of e = exp(score - m) and its
// partial sum_s (e * vs) * v (layout kPart: m, t, 2 unused, 64 sums); the
// splits are combined by attend_combine_kernel or by the Wo GEMV as it
// stages its input row (gguf1.hip): rescaled to the overall maximum, in split
// order, divided by the overall sum.  (The reference divides each e by the
// total before the value products; the float rounding differs, the sums are
// the same.)
//
// The split holding pos takes the new key and value from LDS: the cache row
// at pos is written by the first query head of each key / value group and
// read by no workgroup of this launch.  A score is q . (u - 128) over the
// key's codes u = k + 128 (one byte conversion each): q . u - 128 sum(q).
constexpr int kSplit = 256;
constexpr int kPart = kLlmqSplitRec;  // floats of one split's result (common.h's split record)
constexpr int kMaxSplits = kLlmqMaxSplits;
static_assert(HD == kLlmqSplitHD, "split records hold one head of HD dimensions");
constexpr int kSW = kSplit / 64;  // waves of a split

__global__ __launch_bounds__(kSplit) void attend_split_kernel(const float *__restrict__ qkv, int64_t ld,
                                                              const int *__restrict__ state, int n_head, int n_kv,
                                                              int n_layer, int layer, int max_t,
                                                              const float2 *__restrict__ rope,
                                                              int8_t *__restrict__ K8, int8_t *__restrict__ V8,
                                                              float *__restrict__ KS, float *__restrict__ VS,
                                                              float *__restrict__ part, int NS) {
    __shared__ __align__(16) float q[HD];
    __shared__ __align__(16) int8_t vrow[kSplit][HD];
    __shared__ __align__(16) int8_t knew[HD];
    __shared__ float wv[kSplit], red[kSW], vred[kSW][HD], snew[2], s_qsum;
    const int h = blockIdx.x, b = blockIdx.y, j = blockIdx.z, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int s0 = j * kSplit;
    const int grp = n_head / n_kv, kvh = h / grp;
    const int64_t row0 = (((int64_t)b * n_layer + layer) * n_kv + kvh) * max_t;  // the head's position 0
    const float *r = qkv + (int64_t)b * ld;
    // The query, new key and value and this split's cache rows go out
    // together with the position, which none of their addresses needs.
    float qv = 0.0f, kvx = 0.0f, vvx = 0.0f;
    if (w == 0) qv = r[h * HD + lane];
    if (w == 1) {
        kvx = r[(n_head + kvh) * HD + lane];
        vvx = r[(n_head + n_kv + kvh) * HD + lane];
    }
    const int64_t sl = row0 + min(s0 + tid, max_t - 1);
    int4 kr[HD / 16], vr[HD / 16];
#pragma unroll
    for (int i = 0; i < HD / 16; i++) {
        kr[i] = reinterpret_cast<const int4 *>(K8 + sl * HD)[i];
        vr[i] = reinterpret_cast<const int4 *>(V8 + sl * HD)[i];
    }
    float ks = KS[sl], vs = VS[sl];
    // The position's read goes out after these loads and before their first
    // use, and nothing branches on the position before that use (the
    // compiler would move the loads behind the position's round trip):
    // every row goes to LDS (the new position's written over its slot
    // below), and an empty split (s0 > pos) runs with cnt = 0, its result
    // never read.
    __builtin_amdgcn_sched_barrier(0);
    const int pos = state[0], npos = pos + 1;
    const float2 csn = rope[pos * (HD / 2) + (lane >> 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < HD / 16; i++) reinterpret_cast<int4 *>(vrow[tid])[i] = vr[i];
    const int cnt = max(0, min(kSplit, npos - s0));
    const bool valid = tid < cnt;
    const bool has_new = cnt > 0 && s0 + cnt == npos;  // the last split holds pos at tid cnt - 1
    const bool is_new = has_new && tid == cnt - 1;
    __syncthreads();  // the cached rows are in before the new one goes over its slot
    // RoPE of pair (2i, 2i + 1), i = d / 2, by the table's angle:
    // (x0, x1) -> (x0 c - x1 s, x0 s + x1 c); wave 0 the query, wave 1 the
    // new key, which it quantizes with the new value
    if (w == 0 || (w == 1 && has_new)) {
        const int d = lane;
        const float v = w == 0 ? qv : kvx, pv = llmq_dppf<0xB1>(v);  // lane d ^ 1
        const float rot = (d & 1) ? pv * csn.y + v * csn.x : v * csn.x - pv * csn.y;
        if (w == 0) {
            q[d] = rot;
            const float qs = wave_sum(rot);
            if (d == 0) s_qsum = qs;
        } else {
            const int64_t sn = row0 + pos;
            for (int kv = 0; kv < 2; kv++) {
                const float x = kv == 0 ? rot : vvx;
                const float m = wave_max(fabsf(x));
                float sc = m / 127.0f;
                if (sc == 0.0f) sc = 1.0f;
                const float inv = 1.0f / sc;
                const int8_t code = (int8_t)llmq_to_int(roundf(x * inv));
                if (kv == 0)
                    knew[d] = code;
                else
                    vrow[cnt - 1][d] = code;
                if (d == 0) snew[kv] = sc;
                if (h % grp == 0) {  // one writer per key / value head
                    (kv == 0 ? K8 : V8)[sn * HD + d] = code;
                    if (d == 0) (kv == 0 ? KS : VS)[sn] = sc;
                }
            }
        }
    }
    __syncthreads();
    if (is_new) {
        ks = snew[0];
        vs = snew[1];
    }
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < HD / 16; i++) {
        const int4 k4 = is_new ? reinterpret_cast<const int4 *>(knew)[i] : kr[i];
        const uint32_t kw[4] = {(uint32_t)k4.x ^ 0x80808080u, (uint32_t)k4.y ^ 0x80808080u,
                                (uint32_t)k4.z ^ 0x80808080u, (uint32_t)k4.w ^ 0x80808080u};
        const float4 *q4 = reinterpret_cast<const float4 *>(q + 16 * i);
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
            const float4 qq = q4[e4];
            d = fmaf(qq.x, (float)(kw[e4] & 255u), d);
            d = fmaf(qq.y, (float)((kw[e4] >> 8) & 255u), d);
            d = fmaf(qq.z, (float)((kw[e4] >> 16) & 255u), d);
            d = fmaf(qq.w, (float)(kw[e4] >> 24), d);
        }
    }
    const float score = valid ? (d - 128.0f * s_qsum) * ks * (1.0f / sqrtf((float)HD)) : -INFINITY;
    float m = wave_max(score);
    if (lane == 0) red[w] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int i = 1; i < kSW; i++) m = fmaxf(m, red[i]);
    const float e = valid ? expf(score - m) : 0.0f;
    wv[tid] = e * vs;
    float t = wave_sum(e);
    __syncthreads();  // every read of red done
    if (lane == 0) red[w] = t;
    __syncthreads();
    t = red[0];
#pragma unroll
    for (int i = 1; i < kSW; i++) t += red[i];
    // values: wave w takes positions w, w + kSW, ..; lane = dim
    float acc = 0.0f;
    int sp = w;
    for (; sp + 7 * kSW < cnt; sp += 8 * kSW) {
        float pw[8], vv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            pw[u] = wv[sp + kSW * u];
            vv[u] = (float)vrow[sp + kSW * u][lane];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) acc = fmaf(pw[u], vv[u], acc);
    }
    for (; sp < cnt; sp += kSW) acc = fmaf(wv[sp], (float)vrow[sp][lane], acc);
    vred[w][lane] = acc;
    __syncthreads();
    float *P = part + (((int64_t)b * n_head + h) * NS + j) * kPart;
    if (tid < HD) {
        float o = vred[0][tid];
#pragma unroll
        for (int i = 1; i < kSW; i++) o += vred[i][tid];
        P[4 + tid] = o;
    }
    if (tid == 0) {
        P[0] = m;
        P[1] = t;
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Maximum / sum over the 4 rows of 16 lanes (lanes l % 16 + 16 g).
__device__ __forceinline__ float rows4_max(float v) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}
__device__ __forceinline__ float rows4_sum(float v) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// 8 bytes (a, b) as fp16 1024 + byte, in order.
__device__ __forceinline__ v8h bytes8_f16(uint32_t a, uint32_t b, v2h sub) {
    const uint32_t d[4] = {__builtin_amdgcn_perm(0x64646464u, a, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)};
    v8h r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const v2h h = __builtin_bit_cast(v2h, d[i]) - sub;
        r[2 * i] = h[0];
        r[2 * i + 1] = h[1];
    }
    return r;
}

// x as two fp16 planes, hi = fp16(x), lo = fp16(x - hi).
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// Decode attention of the 8 query heads of key / value head blockIdx.x
// (sequence blockIdx.y, split blockIdx.z of 256 positions) on the fp16
// matrix cores, for batches: the same scores, softmax and value sums as
// attend_split_kernel, with its RoPE, cache store and partial layout, and
// the split's cache rows read once for the 8 heads.  Scores
// q . (u - 128) ks / 8 over the byte codes u = k + 128 (exact in fp16)
// against the query as hi / lo fp16 planes; values sum_p (e_p vs_p) v_p
// with e vs as hi / lo planes under a power-of-two scale of the split (the
// largest vs below 2^10) and v exact.  Wave w scores positions 64 w ..
// 64 w + 63 (lane l: head l % 16, positions 4 (l / 16) + i of each
// 16-position tile, heads 8..15 empty) and forms their value sums for all 64
// dimensions from the same registers; the waves' sums are added in order.
// Sums are in the matrix cores' order, so results agree with
// attend_split_kernel to float rounding, not bit for bit.
__global__ __launch_bounds__(kSplit) void attend_split_group_kernel(const float *__restrict__ qkv, int64_t ld,
                                                                    const int *__restrict__ state, int n_head,
                                                                    int n_kv, int n_layer, int layer, int max_t,
                                                                    const float2 *__restrict__ rope,
                                                                    int8_t *__restrict__ K8, int8_t *__restrict__ V8,
                                                                    float *__restrict__ KS, float *__restrict__ VS,
                                                                    float *__restrict__ part, int NS) {
    constexpr int G = 8, KR = HD + 8;  // heads; key row stride in LDS (bytes)
    static_assert(G * HD == 2 * kSplit, "two query values a thread");
    __shared__ __align__(16) uint8_t ku[kSplit][KR];
    __shared__ __align__(16) int8_t vrow[kSplit][HD];
    __shared__ __align__(16) _Float16 qh[2][G][HD];  // query hi / lo planes
    __shared__ float ksv[kSplit], vsv[kSplit], s_qsum[G], red[kSW][G], redt[kSW][G], vmx[kSW];
    __shared__ __align__(16) float vred[kSW][G][HD];
    const int kvh = blockIdx.x, b = blockIdx.y, j = blockIdx.z, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int s0 = j * kSplit, h0 = kvh * G;
    const int64_t row0 = (((int64_t)b * n_layer + layer) * n_kv + kvh) * max_t;  // the head's position 0
    const float *r = qkv + (int64_t)b * ld;
    // queries (head w and w + 4, dimension lane), new key and value, cache
    // rows, all before the position
    const float qa = r[h0 * HD + tid], qb = r[h0 * HD + kSplit + tid];
    float kvx = 0.0f, vvx = 0.0f;
    if (w == 1) {
        kvx = r[(n_head + kvh) * HD + lane];
        vvx = r[(n_head + n_kv + kvh) * HD + lane];
    }
    const int64_t sl = row0 + min(s0 + tid, max_t - 1);
    int4 kr[HD / 16], vr[HD / 16];
#pragma unroll
    for (int i = 0; i < HD / 16; i++) {
        kr[i] = reinterpret_cast<const int4 *>(K8 + sl * HD)[i];
        vr[i] = reinterpret_cast<const int4 *>(V8 + sl * HD)[i];
    }
    const float ks = KS[sl], vs = VS[sl];
    // the position's read between the loads and their first use, as in
    // attend_split_kernel; scales of positions past the split's end are not
    // used (scores are masked, the value weights selected to 0)
    __builtin_amdgcn_sched_barrier(0);
    const int pos = state[0], npos = pos + 1;
    const float2 csn = rope[pos * (HD / 2) + (lane >> 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < HD / 16; i++) {
        const int4 k4 = kr[i];
        reinterpret_cast<int4 *>(&ku[tid][16 * i])[0] =
            make_int4(k4.x ^ 0x80808080, k4.y ^ 0x80808080, k4.z ^ 0x80808080, k4.w ^ 0x80808080);
        reinterpret_cast<int4 *>(vrow[tid])[i] = vr[i];
    }
    ksv[tid] = ks;
    vsv[tid] = vs;
    const int cnt = max(0, min(kSplit, npos - s0));
    const bool valid = tid < cnt;
    const bool has_new = cnt > 0 && s0 + cnt == npos;  // the last split holds pos at tid cnt - 1
    const bool is_new = has_new && tid == cnt - 1;
    float vm = wave_max(valid && !is_new ? vs : 0.0f);
    __syncthreads();  // the cached rows are in before the new one goes over its slot
    // RoPE of pair (2i, 2i + 1), i = d / 2, as attend_split_kernel's; wave 1
    // also rotates the new key and quantizes it with the new value
    {
        const int d = lane;
        const float pa = llmq_dppf<0xB1>(qa), pb = llmq_dppf<0xB1>(qb);  // lane d ^ 1
        const float ra = (d & 1) ? pa * csn.y + qa * csn.x : qa * csn.x - pa * csn.y;
        const float rb = (d & 1) ? pb * csn.y + qb * csn.x : qb * csn.x - pb * csn.y;
        split_f16(ra, qh[0][w][d], qh[1][w][d]);
        split_f16(rb, qh[0][w + kSW][d], qh[1][w + kSW][d]);
        const float sa = wave_sum(ra), sb = wave_sum(rb);
        if (d == 0) {
            s_qsum[w] = sa;
            s_qsum[w + kSW] = sb;
        }
        if (w == 1 && has_new) {
            const float pk = llmq_dppf<0xB1>(kvx);
            const float rk = (d & 1) ? pk * csn.y + kvx * csn.x : kvx * csn.x - pk * csn.y;
            const int64_t sn = row0 + pos;
            for (int kv = 0; kv < 2; kv++) {
                const float x = kv == 0 ? rk : vvx;
                const float m = wave_max(fabsf(x));
                float sc = m / 127.0f;
                if (sc == 0.0f) sc = 1.0f;
                const float inv = 1.0f / sc;
                const int8_t code = (int8_t)llmq_to_int(roundf(x * inv));
                if (kv == 0)
                    ku[cnt - 1][d] = (uint8_t)(code ^ 0x80);
                else
                    vrow[cnt - 1][d] = code;
                if (d == 0) (kv == 0 ? ksv : vsv)[cnt - 1] = sc;
                vm = kv == 1 ? fmaxf(vm, sc) : vm;
                (kv == 0 ? K8 : V8)[sn * HD + d] = code;  // this workgroup is the head's only writer
                if (d == 0) (kv == 0 ? KS : VS)[sn] = sc;
            }
        }
    }
    if (lane == 0) vmx[w] = vm;
    __syncthreads();
    // the value weights' scale: vs_max sigma < 2^10, a power of two
    int ex = 0;
    frexpf(fmaxf(fmaxf(vmx[0], vmx[1]), fmaxf(vmx[2], vmx[3])), &ex);
    const int sig_e = min(126, max(-126, 10 - ex));
    const float sigma = ldexpf(1.0f, sig_e);
    const int hl = lane & 15, g = lane >> 4;
    const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f}, k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    // the query operand (dimensions 32 kb + 8 g .., hi and lo planes), heads 8..15 zero
    v8h bq[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int pl = 0; pl < 2; pl++) {
            const uint4 t = hl < G ? *reinterpret_cast<const uint4 *>(&qh[pl][hl & 7][32 * kb + 8 * g])
                                   : make_uint4(0u, 0u, 0u, 0u);
            bq[kb][pl] = __builtin_bit_cast(v8h, t);
        }
    const float qs = s_qsum[hl & 7];
    // scores of the wave's 4 tiles of 16 positions
    float sc[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int pt = 0; pt < 4; pt++) {
        const int pb = 64 * w + 16 * pt;
        v4f d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            const uint2 kk = *reinterpret_cast<const uint2 *>(&ku[pb + hl][32 * kb + 8 * g]);
            const v8h ak = bytes8_f16(kk.x, kk.y, k1024);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bq[kb][0], d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ak, bq[kb][1], d, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = pb + 4 * g + i;
            const float v = (d[i] - 128.0f * qs) * ksv[p] * (1.0f / sqrtf((float)HD));
            sc[pt][i] = p < cnt && hl < G ? v : -INFINITY;
            mx = fmaxf(mx, sc[pt][i]);
        }
    }
    mx = rows4_max(mx);
    if (g == 0 && hl < G) red[w][hl] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0][hl & 7], red[1][hl & 7]), fmaxf(red[2][hl & 7], red[3][hl & 7]));
    float te = 0.0f;
    // e vs sigma as hi / lo planes, in the value operand's position order:
    // element e of K-block c is position 64 w + 32 c + 16 (e / 4) + 4 g + e % 4
    v8h ph[2], plo[2];
#pragma unroll
    for (int pt = 0; pt < 4; pt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = 64 * w + 16 * pt + 4 * g + i;
            const float e = sc[pt][i] == -INFINITY ? 0.0f : expf(sc[pt][i] - M);
            te += e;
            _Float16 hi, lo;
            split_f16(e * (p < cnt ? vsv[p] : 0.0f) * sigma, hi, lo);
            ph[pt >> 1][4 * (pt & 1) + i] = hi;
            plo[pt >> 1][4 * (pt & 1) + i] = lo;
        }
    te = rows4_sum(te);
    if (g == 0 && hl < G) redt[w][hl] = te;
    // value sums of the wave's positions: dimension tile dt, lane (dim 16 dt
    // + l % 16, group g), D[head 4 g + i][dim]
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
        v4f o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < 2; c++) {
            uint32_t wv[2] = {0u, 0u};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int p = 64 * w + 32 * c + 16 * (e >> 2) + 4 * g + (e & 3);
                wv[e >> 2] |= (uint32_t)(uint8_t)(vrow[p][16 * dt + hl] ^ 0x80) << (8 * (e & 3));
            }
            const v8h bv = bytes8_f16(wv[0], wv[1], k1152);  // v = (v + 128) + 1024 - 1152
            o = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[c], bv, o, 0, 0, 0);
            o = __builtin_amdgcn_mfma_f32_16x16x32_f16(plo[c], bv, o, 0, 0, 0);
        }
        if (g < 2) {
#pragma unroll
            for (int i = 0; i < 4; i++) vred[w][4 * g + i][16 * dt + hl] = o[i];
        }
    }
    __syncthreads();
    const float isig = ldexpf(1.0f, -sig_e);
    for (int e = tid; e < G * HD; e += kSplit) {
        const int gg = e / HD, dd = e % HD;
        float o = vred[0][gg][dd];
#pragma unroll
        for (int i = 1; i < kSW; i++) o += vred[i][gg][dd];
        float *P = part + (((int64_t)b * n_head + h0 + gg) * NS + j) * kPart;
        P[4 + dd] = o * isig;
        if (dd == 0) {
            P[0] = fmaxf(fmaxf(red[0][gg], red[1][gg]), fmaxf(red[2][gg], red[3][gg]));
            float t = redt[0][gg];
#pragma unroll
            for (int i = 1; i < kSW; i++) t += redt[i][gg];
            P[1] = t;
        }
    }
}

// Dimension dd of a head's split results P (NS splits of kPart floats):
// sum_j acc_j exp(m_j - M) / sum_j t_j exp(m_j - M) over the splits j <
// min(NS, (pos + kSplit) / kSplit) that hold positions, in order (the same
// arithmetic as the Wo GEMV's staging of them, gguf1.hip).  Every split is
// loaded, used or not, ahead of the position, so the loads do not wait for
// it; unused ones are only selected away.
__device__ __forceinline__ float combine_splits(const float *__restrict__ P, int NS, const int *__restrict__ state,
                                                int dd) {
    float mj[kMaxSplits], tj[kMaxSplits], aj[kMaxSplits];
#pragma unroll
    for (int j = 0; j < kMaxSplits; j++) {
        const bool in = j < NS;
        mj[j] = in ? P[j * kPart] : -INFINITY;
        tj[j] = in ? P[j * kPart + 1] : 0.0f;
        aj[j] = in ? P[j * kPart + 4 + dd] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    const int ns = min(NS, (state[0] + kSplit) / kSplit);
    float M = mj[0];  // split 0 always holds positions
#pragma unroll
    for (int j = 1; j < kMaxSplits; j++) M = fmaxf(M, j < ns ? mj[j] : -INFINITY);
    float T = 0.0f, acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxSplits; j++) {
        if (j < ns) {
            const float f = expf(mj[j] - M);
            T = fmaf(tj[j], f, T);
            acc = fmaf(aj[j], f, acc);
        }
    }
    return acc / T;
}

// The splits of (head blockIdx.x, sequence blockIdx.y) into the output.
__global__ __launch_bounds__(64) void attend_combine_kernel(const float *__restrict__ part, int NS, int n_head,
                                                            const int *__restrict__ state, float *__restrict__ out,
                                                            int64_t ldo) {
    const int h = blockIdx.x, b = blockIdx.y, dd = threadIdx.x;
    out[(int64_t)b * ldo + h * HD + dd] = combine_splits(part + ((int64_t)b * n_head + h) * NS * kPart, NS, state, dd);
}

// attend_combine_kernel for the 4 heads of superblock blockIdx.x (wave w
// head 4 blockIdx.x + w), the outputs written as the h16 record of the
// several-row Q4_K matmul (llmq_h16_store, by wave 0 over the 4 heads).
__global__ __launch_bounds__(256) void attend_combine_rec_kernel(const float *__restrict__ part, int NS, int n_head,
                                                                 const int *__restrict__ state,
                                                                 uint8_t *__restrict__ planes,
                                                                 _Float16 *__restrict__ sums,
                                                                 float *__restrict__ inv) {
    __shared__ float o4[4][HD];
    const int w = threadIdx.x >> 6, dd = threadIdx.x & 63, h = blockIdx.x * 4 + w, b = blockIdx.y;
    o4[w][dd] = combine_splits(part + ((int64_t)b * n_head + h) * NS * kPart, NS, state, dd);
    __syncthreads();
    if (w == 0) {
        const float v[4] = {o4[0][dd], o4[1][dd], o4[2][dd], o4[3][dd]};
        llmq_h16_store(planes, sums, inv, n_head * HD / 32, n_head * HD / 256, b, blockIdx.x, v, true);
    }
}

// h[r][i] = silu(g) * u with g = gu[r][i], u = gu[r][F + i].
__global__ void swiglu_kernel(const float *__restrict__ gu, int64_t ldg, float *__restrict__ h, int64_t ldh, int F) {
    const int r = blockIdx.y;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < F; i += gridDim.x * blockDim.x) {
        const float g = gu[(int64_t)r * ldg + i], u = gu[(int64_t)r * ldg + F + i];
        h[(int64_t)r * ldh + i] = (g / (1.0f + expf(-g))) * u;
    }
}

// swiglu_kernel's superblock blockIdx.x of row blockIdx.y (F = 256 NSB)
// written as the h16 record of the several-row Q4_K matmul (by wave 0).
__global__ __launch_bounds__(256) void swiglu_rec_kernel(const float *__restrict__ gu, int64_t ldg, int F,
                                                         uint8_t *__restrict__ planes, _Float16 *__restrict__ sums,
                                                         float *__restrict__ inv) {
    __shared__ float hv[256];
    const int r = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    const float g = gu[(int64_t)r * ldg + i], u = gu[(int64_t)r * ldg + F + i];
    hv[threadIdx.x] = (g / (1.0f + expf(-g))) * u;
    __syncthreads();
    if (threadIdx.x < 64) {
        const int k = threadIdx.x;
        const float v[4] = {hv[k], hv[64 + k], hv[128 + k], hv[192 + k]};
        llmq_h16_store(planes, sums, inv, F / 32, F / 256, r, blockIdx.x, v, true);
    }
}

// Greedy pick (gpt2t.mojo:792-797: the first maximum) of logits row i =
// blockIdx.x for sequence b0 + i: the next token and gen[step * B + b0 + i],
// step = state[1] (0 without state).  With `advance`, the last workgroup to
// finish moves the decode state on (position and step + 1; state[2] counts
// the finished workgroups and is cleared again).
constexpr int kArgNT = 1024;
__global__ __launch_bounds__(kArgNT) void argmax_kernel(const float *__restrict__ logits, int64_t ld, int V, int B,
                                                        int b0, int *__restrict__ state, int advance,
                                                        int64_t *__restrict__ next, int64_t *__restrict__ gen) {
    constexpr int NW = kArgNT / 64;
    __shared__ float bv[NW];
    __shared__ int bi[NW];
    const float *l = logits + (int64_t)blockIdx.x * ld;
    const int tid = threadIdx.x;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    int i = tid;
    for (; i + 7 * kArgNT < V; i += 8 * kArgNT) {  // 8 loads in flight, compared in index order
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; u++) x[u] = l[i + u * kArgNT];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (x[u] > v) {
                v = x[u];
                idx = i + u * kArgNT;
            }
    }
    for (; i < V; i += kArgNT) {
        const float x = l[i];
        if (x > v) {
            v = x;
            idx = i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o);
        const int oi = __shfl_xor(idx, o);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    if ((tid & 63) == 0) {
        bv[tid >> 6] = v;
        bi[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        v = bv[0];
        idx = bi[0];
        for (int k = 1; k < NW; k++)
            if (bv[k] > v || (bv[k] == v && bi[k] < idx)) {
                v = bv[k];
                idx = bi[k];
            }
        const int b = b0 + blockIdx.x;
        const int step = state ? state[1] : 0;
        next[b] = idx;
        gen[(int64_t)step * B + b] = idx;
        if (advance) {
            __threadfence();
            if (atomicAdd(&state[2], 1) == (int)gridDim.x - 1) {  // every workgroup has read the step
                state[2] = 0;
                state[0] += 1;
                state[1] += 1;
            }
        }
    }
}

}  // namespace

struct llmq_llama {
    llmq_ctx *ctx = nullptr;
    llmq_llama_cfg cfg{};
    llmq_mat *embd = nullptr, *head = nullptr;
    std::vector<llmq_mat *> wqkv, wo, wgu, wdown;
    float *norms = nullptr;  // per layer attn / ffn gains, then the output gain
    int8_t *k8 = nullptr, *v8 = nullptr;
    float *ks = nullptr, *vs = nullptr;
    // activations for up to `rows` tokens
    int rows = 0;
    ArgmaxPart *hparts = nullptr;  // head argmax partials, batch x nhparts
    int nhparts = 0;               // the int16 head's partials a row, fixed at creation
    float *apart = nullptr;        // decode attention split results, batch x heads x splits x kPart
    float2 *rope = nullptr;        // (cos, sin) of position p, pair i at [p * head_dim / 2 + i]
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *gu = nullptr, *hh = nullptr,
          *logits = nullptr;
    void *h16 = nullptr;  // fp16 activation record of a several-row Q4_K matmul's input
    int64_t h16_cap = 0;
    void *hs[2] = {nullptr, nullptr};  // the batch-decode chain's h16s records (the matmul epilogues write them)
    int64_t *tokens = nullptr, *next = nullptr, *gen = nullptr;
    int64_t gen_cap = 0;
    int graph_B = 0;  // batch size of the captured decode step
    bool graph_fused = false;  // whether it was captured as the fused chain
    int *state = nullptr;
    // captured decode steps: [0] one step, [1] step_k steps
    hipGraphExec_t step_graph[2] = {};
    hipGraph_t step_graph_def[2] = {};
    int step_k = 0;
};

namespace {

int qkv_cols(const llmq_llama_cfg &c) { return (c.n_head + 2 * c.n_kv) * c.head_dim; }

void drop_graph(llmq_llama *m) {
    for (int i = 0; i < 2; i++) {
        if (m->step_graph[i]) hipGraphExecDestroy(m->step_graph[i]);
        if (m->step_graph_def[i]) hipGraphDestroy(m->step_graph_def[i]);
        m->step_graph[i] = nullptr;
        m->step_graph_def[i] = nullptr;
    }
    m->step_k = 0;
    m->graph_B = 0;
}

// Activation buffers for `rows` tokens; growing them drops the decode graph,
// which holds their addresses.
int ensure_rows(llmq_llama *m, int rows) {
    if (rows <= m->rows) return LLMQ_OK;
    const llmq_llama_cfg &c = m->cfg;
    hipStreamSynchronize(m->ctx->stream);
    drop_graph(m);
    hipFree(m->x);
    hipFree(m->xn);
    hipFree(m->qkv);
    hipFree(m->att);
    hipFree(m->gu);
    hipFree(m->hh);
    hipFree(m->tokens);
    hipFree(m->h16);
    hipFree(m->hs[0]);
    hipFree(m->hs[1]);
    m->x = m->xn = m->qkv = m->att = m->gu = m->hh = nullptr;
    m->tokens = nullptr;
    m->h16 = m->hs[0] = m->hs[1] = nullptr;
    m->h16_cap = 0;
    m->rows = 0;
    const size_t r = (size_t)rows;
    if (hipMalloc(&m->x, r * c.dim * 4) != hipSuccess || hipMalloc(&m->xn, r * c.dim * 4) != hipSuccess ||
        hipMalloc(&m->qkv, r * qkv_cols(c) * 4) != hipSuccess || hipMalloc(&m->att, r * c.dim * 4) != hipSuccess ||
        hipMalloc(&m->gu, r * 2 * c.ffn * 4) != hipSuccess || hipMalloc(&m->hh, r * c.ffn * 4) != hipSuccess ||
        hipMalloc(&m->tokens, r * 8) != hipSuccess)
        return llmq_set_error(LLMQ_ENOMEM, "llama: activations for %d tokens", rows);
    if (rows > 1) {
        const int64_t cap = h16_rec_bytes(rows, std::max(c.dim, c.ffn));
        const size_t scap = (size_t)h16s_rec_bytes(rows, std::max(c.dim, c.ffn));
        if (hipMalloc(&m->h16, (size_t)cap) != hipSuccess || hipMalloc(&m->hs[0], scap) != hipSuccess ||
            hipMalloc(&m->hs[1], scap) != hipSuccess)
            return llmq_set_error(LLMQ_ENOMEM, "llama: activation records for %d tokens", rows);
        m->h16_cap = cap;
    }
    m->rows = rows;
    return LLMQ_OK;
}

const float *gain(const llmq_llama *m, int layer, int which) {  // which: 0 attn, 1 ffn
    return m->norms + ((size_t)2 * layer + which) * m->cfg.dim;
}

// Whether the several-row matmul by w takes an h16 record its producer
// writes (Q4_K rows whose inputs are whole superblocks) and
// LLMQ_GEMM_H16=0 does not turn the fp16 matrix cores off.
bool rec_ok(const llmq_llama *m, const llmq_mat *w) {
    const char *he = getenv("LLMQ_GEMM_H16");
    return m->h16 && gguf_gemm_h16_ok(w) && !(he && he[0] == '0');
}

// A GGUF matmul of R rows: the one-token GEMV for R == 1, else the
// several-token matmul.
int linear(llmq_llama *m, const llmq_mat *w, const float *x, int64_t ldx, int R, float *out, int64_t ldo,
           int flags) {
    if (R == 1) return launch_gguf_gemv(m->ctx, w, x, out, nullptr, flags, nullptr, 0);
    return launch_gguf_gemm(m->ctx, w, x, ldx, R, out, ldo, nullptr, flags, m->h16, m->h16_cap);
}

// rmsnorm(x) * g then the matmul: for one row the GEMV normalizes the row it
// stages (no separate kernel), else the norm goes to m->xn first.
int norm_linear(llmq_llama *m, const float *g, const llmq_mat *w, int R, float *out, int64_t ldo, int flags) {
    const llmq_llama_cfg &c = m->cfg;
    if (R == 1) return launch_gguf_gemv(m->ctx, w, m->x, out, nullptr, flags, nullptr, 0, g, c.eps);
    if (rec_ok(m, w)) {  // the norm writes the Q4_K matmul's fp16 record directly
        uint8_t *pl;
        _Float16 *su;
        float *iv;
        h16_rec_parts(m->h16, R, c.dim, &pl, &su, &iv);
        hipLaunchKernelGGL(rmsnorm_rec_kernel, dim3(c.dim / 256, R), dim3(64), 0, m->ctx->stream, m->x,
                           (int64_t)c.dim, g, c.dim, c.eps, pl, su, iv);
        return launch_gguf_gemm_h16(m->ctx, w, m->h16, R, out, ldo, nullptr, flags);
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(R), dim3(256), 0, m->ctx->stream, m->x, (int64_t)c.dim, g, m->xn,
                       (int64_t)c.dim, c.dim, c.eps);
    return launch_gguf_gemm(m->ctx, w, m->xn, c.dim, R, out, ldo, nullptr, flags, m->h16, m->h16_cap);
}

// The layers for R = nseq * T rows in m->x: T tokens of sequences seq0 ..
// at positions pos0 + t (prefill: nseq = 1), or one token of every
// sequence at position state[0] (decode: T = 1, state given).
// Decode attention of layer l for R sequences (RoPE, the cache store and
// the attention over splits of kSplit positions in one launch); returns the
// split count.
int attend_splits(llmq_llama *m, int R, int l, const int *state) {
    const llmq_llama_cfg &c = m->cfg;
    const int NS = (c.max_t + kSplit - 1) / kSplit, QC = qkv_cols(c);
    // LLMQ_ATTN_GROUP=1 / 0 forces the grouped / per-head kernel
    static const char *ge = getenv("LLMQ_ATTN_GROUP");
    const bool grouped = c.n_head == 8 * c.n_kv && (ge ? ge[0] == '1' : R > 1);
    if (grouped)  // the 8 query heads of a key / value head in one workgroup
        hipLaunchKernelGGL(attend_split_group_kernel, dim3(c.n_kv, R, NS), dim3(kSplit), 0, m->ctx->stream, m->qkv,
                           (int64_t)QC, state, c.n_head, c.n_kv, c.n_layer, l, c.max_t, m->rope, m->k8, m->v8, m->ks,
                           m->vs, m->apart, NS);
    else
        hipLaunchKernelGGL(attend_split_kernel, dim3(c.n_head, R, NS), dim3(kSplit), 0, m->ctx->stream, m->qkv,
                           (int64_t)QC, state, c.n_head, c.n_kv, c.n_layer, l, c.max_t, m->rope, m->k8, m->v8, m->ks,
                           m->vs, m->apart, NS);
    return NS;
}

// Whether the batch-decode step of R sequences takes the fused chain: each
// Q4_K matmul's epilogue writes the next one's h16s record (RMSNorm as a
// factor on the reading matmul's outputs, SwiGLU in the gate / up
// epilogue), instead of the record kernels between them; LLMQ_FUSE_REC=0
// turns it off.
bool fused_chain(const llmq_llama *m, int R, const int *state) {
    const char *fe = getenv("LLMQ_FUSE_REC");
    if (!state || R < 2 || !m->hs[0] || (fe && fe[0] == '0')) return false;
    return rec_ok(m, m->wqkv[0]) && rec_ok(m, m->wo[0]) && rec_ok(m, m->wgu[0]) && rec_ok(m, m->wdown[0]) &&
           gguf_gemm_h16s_ok(m->wqkv[0], false, R) && gguf_gemm_h16s_ok(m->wo[0], false, R) &&
           gguf_gemm_h16s_ok(m->wgu[0], true, R) && gguf_gemm_h16s_ok(m->wdown[0], false, R) &&
           m->cfg.n_head % 4 == 0;
}

// Fused: layer 0's record (of m->x times the attention norm gain) is
// formed here, or, with rec_ready, is already in m->hs[0] (the previous
// step's pick wrote it).
int llama_layers(llmq_llama *m, int R, int T, int seq0, int pos0, const int *state, bool rec_ready = false) {
    llmq_ctx *ctx = m->ctx;
    const llmq_llama_cfg &c = m->cfg;
    const int QC = qkv_cols(c);
    const bool fused = fused_chain(m, R, state);
    int cur = 0;  // fused: m->hs[cur] holds the next qkv matmul's input record
    if (fused && !rec_ready) RC(launch_rec_h16s(ctx, m->x, c.dim, R, c.dim, gain(m, 0, 0), m->hs[cur]));
    for (int l = 0; l < c.n_layer; l++) {
        if (fused) {
            H16Fuse fq;
            fq.in_s = fq.norm = true;
            fq.eps = c.eps;
            RC(launch_gguf_gemm_h16(ctx, m->wqkv[l], m->hs[cur], R, m->qkv, QC, nullptr, 0, &fq));
            const int NS = attend_splits(m, R, l, state);
            uint8_t *pl;
            _Float16 *su;
            float *iv;
            h16_rec_parts(m->h16, R, c.dim, &pl, &su, &iv);
            hipLaunchKernelGGL(attend_combine_rec_kernel, dim3(c.n_head / 4, R), dim3(256), 0, ctx->stream, m->apart,
                               NS, c.n_head, state, pl, su, iv);
            // Wo + residual, writing the ffn norm's record of the new x
            H16Fuse fo;
            fo.out_rec = m->hs[cur ^ 1];
            fo.gain = gain(m, l, 1);
            RC(launch_gguf_gemm_h16(ctx, m->wo[l], m->h16, R, m->x, c.dim, nullptr, LLMQ_RESID, &fo));
            // gate / up (normalized), writing silu(gate) * up as down's record
            H16Fuse fg;
            fg.in_s = fg.norm = fg.swiglu = true;
            fg.eps = c.eps;
            fg.out_rec = m->hs[cur];
            RC(launch_gguf_gemm_h16(ctx, m->wgu[l], m->hs[cur ^ 1], R, nullptr, 0, nullptr, 0, &fg));
            // down + residual, writing the next layer's attention norm record
            H16Fuse fd;
            fd.in_s = true;
            if (l + 1 < c.n_layer) {
                fd.out_rec = m->hs[cur ^ 1];
                fd.gain = gain(m, l + 1, 0);
            }
            RC(launch_gguf_gemm_h16(ctx, m->wdown[l], m->hs[cur], R, m->x, c.dim, nullptr, LLMQ_RESID, &fd));
            cur ^= 1;
            continue;
        }
        RC(norm_linear(m, gain(m, l, 0), m->wqkv[l], R, m->qkv, QC, 0));
        if (state) {  // RoPE, the cache store and the attention splits in one launch
            const int NS = attend_splits(m, R, l, state);
            if (R == 1 && gguf_gemv_attn_ok(m->wo[l], NS, HD)) {  // Wo combines the splits as it stages its row
                RC(launch_gguf_gemv(ctx, m->wo[l], nullptr, m->x, nullptr, LLMQ_RESID, nullptr, 0, nullptr, 0.0f, 0,
                                    nullptr, nullptr, m->apart, state, kSplit, NS));
            } else if (rec_ok(m, m->wo[l]) && c.n_head % 4 == 0) {  // the combination writes Wo's record
                uint8_t *pl;
                _Float16 *su;
                float *iv;
                h16_rec_parts(m->h16, R, c.dim, &pl, &su, &iv);
                hipLaunchKernelGGL(attend_combine_rec_kernel, dim3(c.n_head / 4, R), dim3(256), 0, ctx->stream,
                                   m->apart, NS, c.n_head, state, pl, su, iv);
                RC(launch_gguf_gemm_h16(ctx, m->wo[l], m->h16, R, m->x, c.dim, nullptr, LLMQ_RESID));
            } else {
                hipLaunchKernelGGL(attend_combine_kernel, dim3(c.n_head, R), dim3(HD), 0, ctx->stream, m->apart, NS,
                                   c.n_head, state, m->att, (int64_t)c.dim);
                RC(linear(m, m->wo[l], m->att, c.dim, R, m->x, c.dim, LLMQ_RESID));
            }
        } else {
            hipLaunchKernelGGL(rope_store_kernel, dim3(c.n_head + c.n_kv, R), dim3(64), 0, ctx->stream, m->qkv,
                               (int64_t)QC, T, seq0, pos0, c.n_head, c.n_kv, c.n_layer, l, c.max_t, m->rope,
                               m->k8, m->v8, m->ks, m->vs);
            RC(launch_attend_prompt(ctx, m->k8, m->v8, m->ks, m->vs, seq0 * c.n_layer + l, c.max_t, c.n_head,
                                    c.n_kv, m->qkv, QC, pos0, T, m->att, c.dim, true));
            RC(linear(m, m->wo[l], m->att, c.dim, R, m->x, c.dim, LLMQ_RESID));
        }
        RC(norm_linear(m, gain(m, l, 1), m->wgu[l], R, m->gu, 2 * c.ffn, 0));
        if (R == 1) {  // the GEMV forms silu(gate) * up as it stages its row
            RC(launch_gguf_gemv(ctx, m->wdown[l], m->gu, m->x, nullptr, LLMQ_RESID, nullptr, 0, nullptr, 0.0f, 1));
        } else if (rec_ok(m, m->wdown[l])) {  // silu(gate) * up written as the down matmul's record
            uint8_t *pl;
            _Float16 *su;
            float *iv;
            h16_rec_parts(m->h16, R, c.ffn, &pl, &su, &iv);
            hipLaunchKernelGGL(swiglu_rec_kernel, dim3(c.ffn / 256, R), dim3(256), 0, ctx->stream, m->gu,
                               (int64_t)2 * c.ffn, c.ffn, pl, su, iv);
            RC(launch_gguf_gemm_h16(ctx, m->wdown[l], m->h16, R, m->x, c.dim, nullptr, LLMQ_RESID));
        } else {
            hipLaunchKernelGGL(swiglu_kernel, dim3((c.ffn + 255) / 256, R), dim3(256), 0, ctx->stream, m->gu,
                               (int64_t)2 * c.ffn, m->hh, (int64_t)c.ffn, c.ffn);
            RC(linear(m, m->wdown[l], m->hh, c.ffn, R, m->x, c.dim, LLMQ_RESID));
        }
    }
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

// The output norm and head for nrows consecutive rows of m->x from row r0,
// into m->logits; with parts, an int16 head also leaves its argmax partials
// there (false is returned through *has_parts for a float head).
int llama_head(llmq_llama *m, int r0, int nrows, ArgmaxPart *parts = nullptr, bool *has_parts = nullptr) {
    llmq_ctx *ctx = m->ctx;
    const llmq_llama_cfg &c = m->cfg;
    const float *g = m->norms + (size_t)2 * c.n_layer * c.dim;
    const float *x = m->x + (int64_t)r0 * c.dim;
    if (has_parts) *has_parts = false;
    // the int16 head normalizes the rows it quantizes
    if (gguf_has_i16(m->head)) {
        // the pick reads exactly nhparts partials a row
        LLMQ_REQUIRE(!parts || gguf_head16_parts(m->head) == m->nhparts,
                     "llama head: %d argmax partials a row, the model reads %d", gguf_head16_parts(m->head),
                     m->nhparts);
        if (has_parts) *has_parts = parts != nullptr;
        return launch_gguf_head16(ctx, m->head, x, m->logits, nrows, g, c.eps, parts,
                                  parts ? nrows * m->nhparts : 0);
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(nrows), dim3(256), 0, ctx->stream, x, (int64_t)c.dim, g, m->xn,
                       (int64_t)c.dim, c.dim, c.eps);
    return linear(m, m->head, m->xn, c.dim, nrows, m->logits, c.vocab, 0);
}

// The fused chain's first record, of the embedded picks in m->x (nothing
// outside the fused chain).
int decode_rec(llmq_llama *m, int B) {
    if (!fused_chain(m, B, m->state)) return LLMQ_OK;
    return launch_rec_h16s(m->ctx, m->x, m->cfg.dim, B, m->cfg.dim, gain(m, 0, 0), m->hs[0]);
}

// One decode step of every sequence from the embedded picks in m->x: the
// layers, the head, the picks with the position and step advance, and the
// picks' embeddings for the next step.
// In the fused chain the step starts from layer 0's record, which the
// previous step's pick (or, before the first step, decode_rec) wrote.
int llama_step(llmq_llama *m, int B) {
    llmq_ctx *ctx = m->ctx;
    const llmq_llama_cfg &c = m->cfg;
    const bool fused = fused_chain(m, B, m->state);
    RC(llama_layers(m, B, 1, 0, 0, m->state, fused));
    bool parts = false;
    RC(llama_head(m, 0, B, m->hparts, &parts));
    if (parts && fused)  // the picks, their embeddings and the next step's first record in one launch
        return launch_gguf_pick_embed_rec(ctx, m->embd, m->hparts, m->nhparts, B, m->state, m->next, m->gen, m->x,
                                          c.dim, m->hs[0], gain(m, 0, 0));
    if (parts)
        return launch_gguf_pick_embed(ctx, m->embd, m->hparts, m->nhparts, B, m->state, m->next,
                                      m->gen, m->x, c.dim);
    hipLaunchKernelGGL(argmax_kernel, dim3(B), dim3(kArgNT), 0, ctx->stream, m->logits, (int64_t)c.vocab, c.vocab, B,
                       0, m->state, 1, m->next, m->gen);
    LLMQ_HIP(hipGetLastError());
    RC(launch_gguf_dequant_rows(ctx, m->embd, m->next, B, m->x, c.dim));
    return decode_rec(m, B);
}

// Prefill of sequence seq: T tokens (host) at positions pos0.., then its
// last token's logits and greedy pick (gen row 0 when state is null).
int llama_prefill(llmq_llama *m, int seq, const int64_t *tokens, int T, int pos0, int B, bool pick) {
    llmq_ctx *ctx = m->ctx;
    const llmq_llama_cfg &c = m->cfg;
    RC(ensure_rows(m, T));
    LLMQ_HIP(hipMemcpyAsync(m->tokens, tokens, sizeof(int64_t) * T, hipMemcpyHostToDevice, ctx->stream));
    RC(launch_gguf_dequant_rows(ctx, m->embd, m->tokens, T, m->x, c.dim));
    RC(llama_layers(m, T, T, seq, pos0, nullptr));
    RC(llama_head(m, T - 1, 1));
    if (pick)
        hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgNT), 0, ctx->stream, m->logits, (int64_t)c.vocab, c.vocab,
                           B, seq, nullptr, 0, m->next, m->gen);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

}  // namespace

int llmq_llama_free(llmq_llama *m) {
    if (!m) return LLMQ_OK;
    if (m->ctx) hipStreamSynchronize(m->ctx->stream);
    drop_graph(m);
    llmq_mat_free(m->embd);
    llmq_mat_free(m->head);
    for (auto *w : m->wqkv) llmq_mat_free(w);
    for (auto *w : m->wo) llmq_mat_free(w);
    for (auto *w : m->wgu) llmq_mat_free(w);
    for (auto *w : m->wdown) llmq_mat_free(w);
    void *bufs[] = {m->hparts, m->apart, m->rope, m->norms, m->k8, m->v8, m->ks, m->vs, m->x, m->xn, m->qkv, m->att, m->gu, m->hh, m->logits,
                    m->h16, m->hs[0], m->hs[1], m->tokens, m->next, m->gen, m->state};
    for (void *p : bufs) hipFree(p);
    delete m;
    return LLMQ_OK;
}

int llmq_llama_create(llmq_ctx *ctx, const llmq_llama_cfg *cfg, const void *const *t, llmq_llama **out) {
    LLMQ_REQUIRE(ctx && cfg && t && out, "llama_create: bad arguments");
    const llmq_llama_cfg c = *cfg;
    LLMQ_REQUIRE(c.n_layer > 0 && c.dim > 0 && c.n_head > 0 && c.n_kv > 0 && c.n_head % c.n_kv == 0 &&
                     c.head_dim == HD && c.n_head * c.head_dim == c.dim && c.ffn > 0 && c.vocab > 0 &&
                     c.max_t > 0 && c.batch > 0,
                 "llama_create: unsupported shape (head_dim must be 64, n_head * head_dim == dim)");
    LLMQ_REQUIRE(c.max_t <= kSplit * kMaxSplits, "llama_create: max_t %d beyond %d", c.max_t, kSplit * kMaxSplits);
    for (int ty : {c.layer_type, c.head_type, c.embd_type})
        LLMQ_REQUIRE(gguf_is_supported(ty), "llama_create: ggml type %d is not a supported block format", ty);
    llmq_llama *m = new llmq_llama();
    m->ctx = ctx;
    m->cfg = c;
    int rc = LLMQ_OK;
#define GO(call)                   \
    do {                           \
        rc = (call);               \
        if (rc != LLMQ_OK) goto fail; \
    } while (0)
    {
        const int bs = gguf_block_size(c.layer_type), bb = gguf_block_bytes(c.layer_type);
        auto rb = [&](int64_t cols) { return (size_t)(cols / bs) * bb; };
        auto mat = [&](const void *blocks, int ty, int64_t rows, int64_t cols, llmq_mat **w) {
            return llmq_mat_from_gguf(ctx, ty, blocks, rows, cols, w);
        };
        // host tensors: token_embd; per layer attn_norm, q, k, v, o, ffn_norm, gate, up, down; output_norm, output
        GO(mat(t[0], c.embd_type, c.vocab, c.dim, &m->embd));
        const size_t nn = (size_t)(2 * c.n_layer + 1) * c.dim;
        GO(hipMalloc(&m->norms, nn * 4) == hipSuccess ? LLMQ_OK : llmq_set_error(LLMQ_ENOMEM, "llama: norms"));
        std::vector<float> norms(nn);
        const int kvd = c.n_kv * HD;
        for (int l = 0; l < c.n_layer; l++) {
            const void *const *L = t + 1 + 9 * l;
            memcpy(&norms[(size_t)2 * l * c.dim], L[0], (size_t)c.dim * 4);
            memcpy(&norms[(size_t)(2 * l + 1) * c.dim], L[5], (size_t)c.dim * 4);
            std::vector<uint8_t> cat;
            auto append = [&](const void *p, int64_t rows, int64_t cols) {
                const uint8_t *b = static_cast<const uint8_t *>(p);
                cat.insert(cat.end(), b, b + rows * rb(cols));
            };
            append(L[1], c.dim, c.dim);
            append(L[2], kvd, c.dim);
            append(L[3], kvd, c.dim);
            llmq_mat *w = nullptr;
            GO(mat(cat.data(), c.layer_type, c.dim + 2 * kvd, c.dim, &w));
            m->wqkv.push_back(w);
            GO(mat(L[4], c.layer_type, c.dim, c.dim, &w));
            m->wo.push_back(w);
            cat.clear();
            append(L[6], c.ffn, c.dim);
            append(L[7], c.ffn, c.dim);
            GO(mat(cat.data(), c.layer_type, 2 * c.ffn, c.dim, &w));
            m->wgu.push_back(w);
            GO(mat(L[8], c.layer_type, c.dim, c.ffn, &w));
            m->wdown.push_back(w);
        }
        memcpy(&norms[(size_t)2 * c.n_layer * c.dim], t[1 + 9 * c.n_layer], (size_t)c.dim * 4);
        GO(mat(t[2 + 9 * c.n_layer], c.head_type, c.vocab, c.dim, &m->head));
        GO(hipMemcpy(m->norms, norms.data(), nn * 4, hipMemcpyHostToDevice) == hipSuccess
               ? LLMQ_OK
               : llmq_set_error(LLMQ_EHIP, "llama: norms copy"));
        const size_t slots = (size_t)c.batch * c.n_layer * c.max_t * c.n_kv;
        if (hipMalloc(&m->k8, slots * HD) != hipSuccess || hipMalloc(&m->v8, slots * HD) != hipSuccess ||
            hipMalloc(&m->ks, slots * 4) != hipSuccess || hipMalloc(&m->vs, slots * 4) != hipSuccess ||
            hipMalloc(&m->logits, (size_t)c.batch * c.vocab * 4) != hipSuccess ||
            hipMalloc(&m->next, (size_t)c.batch * 8) != hipSuccess || hipMalloc(&m->state, 16) != hipSuccess)
            GO(llmq_set_error(LLMQ_ENOMEM, "llama: cache of %zu slots", slots));
        if (hipMemset(m->k8, 0, slots * HD) != hipSuccess || hipMemset(m->v8, 0, slots * HD) != hipSuccess ||
            hipMemset(m->ks, 0, slots * 4) != hipSuccess || hipMemset(m->vs, 0, slots * 4) != hipSuccess)
            GO(llmq_set_error(LLMQ_EHIP, "llama: cache clear"));
        GO(ensure_rows(m, c.batch));
        if (gguf_has_i16(m->head)) m->nhparts = gguf_head16_parts(m->head);
        if (gguf_has_i16(m->head) &&
            hipMalloc(&m->hparts, sizeof(ArgmaxPart) * c.batch * m->nhparts) != hipSuccess)
            GO(llmq_set_error(LLMQ_ENOMEM, "llama: head partials"));
        if (hipMalloc(&m->apart, sizeof(float) * c.batch * c.n_head * ((c.max_t + kSplit - 1) / kSplit) * kPart) !=
            hipSuccess)
            GO(llmq_set_error(LLMQ_ENOMEM, "llama: attention partials"));
        {   // RoPE: angle pos * theta^(-2i / head_dim) (both in float), cos and sin rounded from double
            std::vector<float> tab((size_t)c.max_t * HD);
            for (int p = 0; p < c.max_t; p++)
                for (int i = 0; i < HD / 2; i++) {
                    const float freq = powf(c.theta, -(float)(2 * i) / (float)HD);
                    const double ang = (double)((float)p * freq);
                    tab[((size_t)p * (HD / 2) + i) * 2] = (float)cos(ang);
                    tab[((size_t)p * (HD / 2) + i) * 2 + 1] = (float)sin(ang);
                }
            if (hipMalloc(&m->rope, tab.size() * 4) != hipSuccess)
                GO(llmq_set_error(LLMQ_ENOMEM, "llama: RoPE table"));
            if (hipMemcpy(m->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
                GO(llmq_set_error(LLMQ_EHIP, "llama: RoPE table copy"));
        }
    }
#undef GO
    *out = m;
    return LLMQ_OK;
fail:
    llmq_llama_free(m);
    return rc;
}

int64_t llmq_llama_weight_bytes(const llmq_llama *m) {
    if (!m) return 0;
    int64_t n = llmq_mat_nbytes(m->embd) + llmq_mat_nbytes(m->head);
    for (auto *w : m->wqkv) n += llmq_mat_nbytes(w);
    for (auto *w : m->wo) n += llmq_mat_nbytes(w);
    for (auto *w : m->wgu) n += llmq_mat_nbytes(w);
    for (auto *w : m->wdown) n += llmq_mat_nbytes(w);
    return n + (int64_t)(2 * m->cfg.n_layer + 1) * m->cfg.dim * 4;
}

int llmq_llama_forward(llmq_llama *m, int seq, const int64_t *tokens, int T, int pos0, float *logits) {
    LLMQ_REQUIRE(m && tokens && T >= 1, "llama_forward: bad arguments");
    const llmq_llama_cfg &c = m->cfg;
    LLMQ_REQUIRE(seq >= 0 && seq < c.batch, "llama_forward: sequence %d of %d", seq, c.batch);
    LLMQ_REQUIRE(pos0 >= 0 && pos0 + T <= c.max_t, "llama_forward: positions %d..%d beyond %d", pos0, pos0 + T - 1,
                 c.max_t);
    for (int t = 0; t < T; t++)
        LLMQ_REQUIRE(tokens[t] >= 0 && tokens[t] < c.vocab, "llama_forward: token %lld out of range",
                     (long long)tokens[t]);
    OwnStream os_(m->ctx);
    RC(llama_prefill(m, seq, tokens, T, pos0, 1, false));
    if (logits)
        LLMQ_HIP(hipMemcpyAsync(logits, m->logits, sizeof(float) * c.vocab, hipMemcpyDeviceToHost, m->ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(m->ctx->stream));
    return LLMQ_OK;
}

int llmq_llama_generate(llmq_llama *m, const int64_t *prompts, int B, int n_prompt, int steps, int64_t *out_tokens,
                        double *prefill_ms, double *decode_ms) {
    LLMQ_REQUIRE(m && prompts && n_prompt >= 1 && steps >= 1 && out_tokens, "llama_generate: bad arguments");
    const llmq_llama_cfg &c = m->cfg;
    LLMQ_REQUIRE(B >= 1 && B <= c.batch, "llama_generate: %d sequences, capacity %d", B, c.batch);
    LLMQ_REQUIRE(n_prompt + steps - 1 <= c.max_t, "llama_generate: %d + %d positions beyond %d", n_prompt, steps,
                 c.max_t);
    for (int64_t i = 0; i < (int64_t)B * n_prompt; i++)
        LLMQ_REQUIRE(prompts[i] >= 0 && prompts[i] < c.vocab, "llama_generate: token %lld out of range",
                     (long long)prompts[i]);
    OwnStream os_(m->ctx);
    llmq_ctx *ctx = m->ctx;
    if (B != m->graph_B) drop_graph(m);  // a captured step serves one batch size
    if ((int64_t)steps * B > m->gen_cap) {
        hipFree(m->gen);
        m->gen = nullptr;
        m->gen_cap = 0;
        if (hipMalloc(&m->gen, sizeof(int64_t) * steps * B) != hipSuccess)
            return llmq_set_error(LLMQ_ENOMEM, "llama_generate: %d steps", steps);
        m->gen_cap = (int64_t)steps * B;
        drop_graph(m);  // it holds the old buffer's address
    }
    RC(ensure_rows(m, n_prompt));
    // a captured step starts from the fused chain's record only if it was
    // captured with the chain
    const bool fz = fused_chain(m, B, m->state);
    if (fz != m->graph_fused) drop_graph(m);
    m->graph_fused = fz;
    const char *ge = getenv("LLMQ_GRAPH");
    const bool use_graph = !(ge && ge[0] == '0');  // LLMQ_GRAPH=0: steps launched one by one
    // Each step picks its tokens and positions on the device, so k steps
    // capture as one graph, replayed while k or more remain, then the
    // one-step graph (k = LLMQ_GRAPH_STEPS, default 4, as for GPT-2).
    int k = 4;
    if (const char *e = getenv("LLMQ_GRAPH_STEPS")) k = atoi(e);
    k = k < 1 ? 1 : k > 64 ? 64 : k;
    const int n_steps = steps - 1, n_multi = k > 1 ? n_steps / k : 0, n_one = n_steps - n_multi * k;
    if (use_graph && n_multi > 0 && m->step_k != k && m->step_graph[1]) {
        hipGraphExecDestroy(m->step_graph[1]);
        hipGraphDestroy(m->step_graph_def[1]);
        m->step_graph[1] = nullptr;
        m->step_graph_def[1] = nullptr;
    }
    if (use_graph && n_multi > 0 && !m->step_graph[1]) {
        RC(llmq_capture(
            ctx->stream,
            [&]() -> int {
                for (int i = 0; i < k; i++) RC(llama_step(m, B));
                return LLMQ_OK;
            },
            &m->step_graph_def[1], &m->step_graph[1]));
        m->step_k = k;
        m->graph_B = B;
    }
    if (use_graph && n_one > 0 && !m->step_graph[0]) {
        RC(llmq_capture(ctx->stream, [&] { return llama_step(m, B); }, &m->step_graph_def[0], &m->step_graph[0]));
        m->graph_B = B;
    }
    ScopedEvents ev;
    RC(ev.create());
    hipEvent_t e0 = ev.e[0], e1 = ev.e[1], e2 = ev.e[2];
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    LLMQ_HIP(hipEventRecord(e0, ctx->stream));
    for (int b = 0; b < B; b++) RC(llama_prefill(m, b, prompts + (int64_t)b * n_prompt, n_prompt, 0, B, true));
    LLMQ_HIP(hipEventRecord(e1, ctx->stream));
    const int init_state[4] = {n_prompt, 1, 0, 0};  // position of the first pick, gen row of the next
    LLMQ_HIP(hipMemcpyAsync(m->state, init_state, sizeof(init_state), hipMemcpyHostToDevice, ctx->stream));
    RC(launch_gguf_dequant_rows(ctx, m->embd, m->next, B, m->x, c.dim));  // the first picks, embedded
    RC(decode_rec(m, B));
    if (use_graph) {
        for (int i = 0; i < n_multi; i++) LLMQ_HIP(hipGraphLaunch(m->step_graph[1], ctx->stream));
        for (int i = 0; i < n_one; i++) LLMQ_HIP(hipGraphLaunch(m->step_graph[0], ctx->stream));
    } else {
        for (int i = 1; i < steps; i++) RC(llama_step(m, B));
    }
    LLMQ_HIP(hipEventRecord(e2, ctx->stream));
    LLMQ_HIP(hipEventSynchronize(e2));
    float a = 0, bm = 0;
    LLMQ_HIP(hipEventElapsedTime(&a, e0, e1));
    LLMQ_HIP(hipEventElapsedTime(&bm, e1, e2));
    if (prefill_ms) *prefill_ms = a;
    if (decode_ms) *decode_ms = bm;
    LLMQ_HIP(hipMemcpy(out_tokens, m->gen, sizeof(int64_t) * steps * B, hipMemcpyDeviceToHost));
    return LLMQ_OK;
}
