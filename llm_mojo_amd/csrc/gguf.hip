// GGUF block formats on the GPU: GGUFMatrix (gguf.mojo:344-511) storage and
// its row dequantizer (the block decoders of gguf.mojo:178-297); the GEMV
// over this layout is gguf1.hip.
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
//   Q8_0  chunk = half block     meta16[block] = d ([tile][block][16]: block = c / 2)
//   Q4_K  chunk = sub-block      sb16[sb] = d | dmin << 16 | 12 scale bytes
//   Q5_K  as Q4_K                + bits32[c]: the 5th bit of weight n in bit n
//   Q6_K  chunk = 2 sub-blocks   + bits64[c]: high 2 bits of weight n in bits 2n..2n+1;
//                                  sb16[sb] = the 16 int8 scales, meta16[sb] = d
//
// The device bytes per row equal the reference's row_bytes (gguf.mojo:371).
#include <string.h>

#include <vector>

#include "common.h"
#include "hs_rec.h"

namespace {

__device__ __forceinline__ float h2f(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)bits)); }

struct GgufArgs {
    const uint4 *codes;
    const uint16_t *meta16;
    const uint32_t *meta32;
    const uint32_t *bits32;
    const uint2 *bits64;
    const uint4 *sb16;
    int n, K, ntiles, CK, NSB;
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

// The fields input k of a row reads (its chunk's codes and the type's side
// data) and the input's value from them (GGUFMatrix.dequant_row,
// gguf.mojo:381-382).
template <int TYPE>
struct RowDeq {
    using F = Fmt<TYPE>;
    struct Fields {
        uint4 d, f;
        uint32_t m;
        uint2 hb;
    };
    const GgufArgs &a;
    int64_t tile, r;
    __device__ RowDeq(const GgufArgs &a_, int64_t row) : a(a_), tile(row / 16), r(row % 16) {}
    __device__ __forceinline__ Fields load(int k) const {
        Fields x{};
        const int c = k / F::WPC;
        const size_t mi = ((size_t)tile * a.CK + c) * 16 + r;
        const size_t sbi = ((size_t)tile * a.NSB + c / F::CPS) * 16 + r;
        x.d = a.codes[mi];
        if constexpr (TYPE == LLMQ_GGML_Q8_0) x.m = a.meta16[((size_t)tile * (a.CK / 2) + (c >> 1)) * 16 + r];
        if constexpr (TYPE == LLMQ_GGML_Q4_0) x.m = a.meta16[mi];
        if constexpr (TYPE == LLMQ_GGML_Q4_1) x.m = a.meta32[mi];
        if constexpr (TYPE == LLMQ_GGML_Q5_K) x.m = a.bits32[mi];
        if constexpr (TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K || TYPE == LLMQ_GGML_Q6_K) x.f = a.sb16[sbi];
        if constexpr (TYPE == LLMQ_GGML_Q6_K) {
            x.hb = a.bits64[mi];
            x.m = a.meta16[sbi];
        }
        return x;
    }
    __device__ __forceinline__ float value(int k, const Fields &x) const {
        const int c = k / F::WPC, e = k % F::WPC;
        // the fields as scalars, chosen by selects (an indexed array or struct would go to scratch)
        const uint32_t d0 = x.d.x, d1 = x.d.y, d2 = x.d.z, d3 = x.d.w;
        const uint32_t f0 = x.f.x, f1 = x.f.y, f2 = x.f.z, f3 = x.f.w, h0 = x.hb.x, h1 = x.hb.y, mm = x.m;
        auto dword = [&](int i) { return i == 0 ? d0 : i == 1 ? d1 : i == 2 ? d2 : d3; };
        if constexpr (TYPE == LLMQ_GGML_Q8_0) {
            const int q = (int)(int8_t)((dword(e >> 2) >> (8 * (e & 3))) & 255u);
            return h2f(mm) * (float)q;
        } else {
            int u = (int)((dword(e >> 3) >> (4 * (e & 7))) & 15u);
            if constexpr (TYPE == LLMQ_GGML_Q4_0) {
                return ((float)u - 8.0f) * h2f(mm);
            } else if constexpr (TYPE == LLMQ_GGML_Q4_1) {
                return h2f(mm) * (float)u + h2f(mm >> 16);
            } else if constexpr (TYPE == LLMQ_GGML_Q4_K || TYPE == LLMQ_GGML_Q5_K) {
                if constexpr (TYPE == LLMQ_GGML_Q5_K) u |= (int)((mm >> e) & 1u) << 4;
                int sc, mn;
                k_scale_min(f1, f2, f3, c & 7, sc, mn);
                return (h2f(f0) * (float)sc) * (float)u - h2f(f0 >> 16) * (float)mn;
            } else {
                const uint32_t hw = e < 16 ? h0 : h1;
                u |= (int)((hw >> (2 * (e & 15))) & 3u) << 4;
                const int si = 2 * (c & 7) + (e >= 16);
                const uint32_t sw = si < 4 ? f0 : (si < 8 ? f1 : (si < 12 ? f2 : f3));
                const float sc = (float)(int8_t)((sw >> (8 * (si & 3))) & 255u);
                return (h2f(mm) * sc) * ((float)u - 32.0f);
            }
        }
    }
};

// Dequantize one row into float32 (GGUFMatrix.dequant_row, gguf.mojo:381-382).
template <int TYPE>
__device__ __forceinline__ void dequant_row_body(const GgufArgs &a, int64_t row, float *dst) {
    const RowDeq<TYPE> rd(a, row);
    // NB inputs a thread at a time: every load of the batch is issued before the first value
    constexpr int NB = 8;
    for (int k0 = threadIdx.x; k0 < a.K; k0 += NB * blockDim.x) {
        typename RowDeq<TYPE>::Fields x[NB];
#pragma unroll
        for (int kk = 0; kk < NB; kk++) {
            const int k = k0 + kk * (int)blockDim.x;
            x[kk] = rd.load(k < a.K ? k : k0);  // past K: a repeat of k0's fields, not stored
        }
#pragma unroll
        for (int kk = 0; kk < NB; kk++) {
            const int k = k0 + kk * (int)blockDim.x;
            if (k < a.K) dst[k] = rd.value(k, x[kk]);
        }
    }
}

template <int TYPE>
__global__ void gguf_dequant_row_kernel(GgufArgs a, int64_t row, float *dst) {
    dequant_row_body<TYPE>(a, row, dst);
}

// Rows rows[i] (device indices, e.g. token ids) into dst + i * ldd, one
// workgroup a row; an index outside the matrix writes zeros.
template <int TYPE>
__global__ void gguf_dequant_rows_kernel(GgufArgs a, const int64_t *rows, float *dst, int64_t ldd) {
    const int64_t row = rows[blockIdx.x];
    float *d = dst + (int64_t)blockIdx.x * ldd;
    if (row < 0 || row >= a.n) {
        for (int k = threadIdx.x; k < a.K; k += blockDim.x) d[k] = 0.0f;
        return;
    }
    dequant_row_body<TYPE>(a, row, d);
}

// Greedy pick and embedding of sequence b = blockIdx.x after a head that
// left per-workgroup argmax partials: the largest value over parts[b * nparts
// ..] (the smallest index among equal ones: the first maximum,
// gpt2t.mojo:792-797) is the next token, written to next[b] and
// gen[state[1] * B + b]; its row of E goes to dst + b * ldd.  The last
// workgroup to finish moves the decode state on (position and step + 1;
// state[2] counts the finished workgroups and is cleared again; one
// workgroup advances it directly).
template <int TYPE>
__global__ __launch_bounds__(256) void gguf_pick_embed_kernel(GgufArgs a, const ArgmaxPart *__restrict__ parts,
                                                              int nparts, int B, int *__restrict__ state,
                                                              int64_t *__restrict__ next, int64_t *__restrict__ gen,
                                                              float *__restrict__ dst, int64_t ldd) {
    __shared__ ArgmaxPart s_b[4];
    __shared__ int s_pick;
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const ArgmaxPart *P = parts + (int64_t)b * nparts;
    const int pos = state[0], step = state[1];  // read with the partials (before any advance)
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    // 4 partials a thread in flight at a time (the first-maximum rule is order-free)
    for (int i0 = tid; i0 < nparts; i0 += 4 * 256) {
        ArgmaxPart c[4];
#pragma unroll
        for (int k = 0; k < 4; k++) c[k] = i0 + 256 * k < nparts ? P[i0 + 256 * k] : ArgmaxPart{-INFINITY, 0x7fffffff};
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (c[k].v > bv || (c[k].v == bv && c[k].idx < bi)) {
                bv = c[k].v;
                bi = c[k].idx;
            }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) s_b[tid >> 6] = ArgmaxPart{bv, bi};
    __syncthreads();
    if (tid == 0) {
        ArgmaxPart best = s_b[0];
        for (int w = 1; w < 4; w++)
            if (s_b[w].v > best.v || (s_b[w].v == best.v && s_b[w].idx < best.idx)) best = s_b[w];
        next[b] = best.idx;
        gen[(int64_t)step * B + b] = best.idx;
        s_pick = best.idx;
        if (gridDim.x == 1) {  // the only reader of the step
            state[0] = pos + 1;
            state[1] = step + 1;
        } else {
            __threadfence();
            if (atomicAdd(&state[2], 1) == (int)gridDim.x - 1) {  // every workgroup has read the step
                state[2] = 0;
                state[0] += 1;
                state[1] += 1;
            }
        }
    }
    __syncthreads();
    const int64_t row = s_pick;
    float *d = dst + (int64_t)b * ldd;
    if (row < 0 || row >= a.n) {
        for (int k = tid; k < a.K; k += 256) d[k] = 0.0f;
        return;
    }
    dequant_row_body<TYPE>(a, row, d);
}

// The batch decode chain's pick, embedding and first record in one launch:
// workgroup (j, b), b < B, picks sequence b's token from its argmax partials
// (every workgroup of the sequence by the same first-maximum rule,
// gpt2t.mojo:792-797), writes inputs 256 j .. 256 j + 255 of the token's row
// of E to dst + b * ldd and the same inputs times rgain to token b of the
// h16s record rec (the first matmul's input of the next step, with the sums
// of squares for its RMSNorm); workgroup (0, b) writes next[b] and
// gen[state[1] * B + b]; the last of the B * gridDim.x workgroups to finish
// moves the decode state on (state[2] counts them and is cleared again).
// Workgroups b >= B write zero record rows for the padded tokens.
template <int TYPE>
__global__ __launch_bounds__(256) void gguf_pick_embed_rec_kernel(GgufArgs a, const ArgmaxPart *__restrict__ parts,
                                                                  int nparts, int B, int *__restrict__ state,
                                                                  int64_t *__restrict__ next,
                                                                  int64_t *__restrict__ gen, float *__restrict__ dst,
                                                                  int64_t ldd, HSRec rec,
                                                                  const float *__restrict__ rgain) {
    __shared__ ArgmaxPart s_b[4];
    __shared__ int s_pick;
    const int j = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int k = j * 256 + tid;
    if (b >= B) {  // (uniform over the workgroup)
        hs_store_half(rec, b, k >> 4, 0.0f, 0.0f);
        return;
    }
    const ArgmaxPart *P = parts + (int64_t)b * nparts;
    const int step = state[1];  // read with the partials (before any advance)
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i0 = tid; i0 < nparts; i0 += 4 * 256) {
        ArgmaxPart c[4];
#pragma unroll
        for (int q = 0; q < 4; q++) c[q] = i0 + 256 * q < nparts ? P[i0 + 256 * q] : ArgmaxPart{-INFINITY, 0x7fffffff};
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (c[q].v > bv || (c[q].v == bv && c[q].idx < bi)) {
                bv = c[q].v;
                bi = c[q].idx;
            }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) s_b[tid >> 6] = ArgmaxPart{bv, bi};
    __syncthreads();
    if (tid == 0) {
        ArgmaxPart best = s_b[0];
        for (int w = 1; w < 4; w++)
            if (s_b[w].v > best.v || (s_b[w].v == best.v && s_b[w].idx < best.idx)) best = s_b[w];
        if (j == 0) {
            next[b] = best.idx;
            gen[(int64_t)step * B + b] = best.idx;
        }
        s_pick = best.idx;
        __threadfence();
        if (atomicAdd(&state[2], 1) == (int)gridDim.x * B - 1) {  // every workgroup has read the step
            state[2] = 0;
            state[0] += 1;
            state[1] += 1;
        }
    }
    __syncthreads();
    const int64_t row = s_pick;
    float v = 0.0f;
    if (row >= 0 && row < a.n) {
        const RowDeq<TYPE> rd(a, row);
        v = rd.value(k, rd.load(k));
    }
    dst[(int64_t)b * ldd + k] = v;
    hs_store_half(rec, b, k >> 4, v * rgain[k], v);
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

}  // namespace

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
    LLMQ_REQUIRE(ntc * 16 < (int64_t)kLlmqOOB, "from_gguf: %lld x %lld matrix: code array reaches the 2 GiB limit",
                 (long long)rows, (long long)cols);
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
                meta16[(size_t)((tile * (m->CK / 2) + b) * 16 + r)] = (uint16_t)u16(p);  // [tile][block][16]
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
        // kernels address each array with 32-bit buffer offsets (0x80000000 = a disabled load)
        if (bytes >= kLlmqOOB)
            return llmq_set_error(LLMQ_EINVAL, "from_gguf: an array of %zu bytes reaches the 2 GiB limit", bytes);
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

int launch_gguf_dequant_rows(llmq_ctx *ctx, const llmq_mat *w, const int64_t *rows, int n, float *dst, int64_t ldd) {
    LLMQ_REQUIRE(w && w->kind == MAT_GGUF && rows && dst && n > 0, "gguf dequant rows: bad arguments");
    GgufArgs a = make_args(w);
    switch (w->ggml_type) {
    case LLMQ_GGML_Q4_0: hipLaunchKernelGGL(gguf_dequant_rows_kernel<LLMQ_GGML_Q4_0>, dim3(n), dim3(256), 0, ctx->stream, a, rows, dst, ldd); break;
    case LLMQ_GGML_Q4_1: hipLaunchKernelGGL(gguf_dequant_rows_kernel<LLMQ_GGML_Q4_1>, dim3(n), dim3(256), 0, ctx->stream, a, rows, dst, ldd); break;
    case LLMQ_GGML_Q8_0: hipLaunchKernelGGL(gguf_dequant_rows_kernel<LLMQ_GGML_Q8_0>, dim3(n), dim3(256), 0, ctx->stream, a, rows, dst, ldd); break;
    case LLMQ_GGML_Q4_K: hipLaunchKernelGGL(gguf_dequant_rows_kernel<LLMQ_GGML_Q4_K>, dim3(n), dim3(256), 0, ctx->stream, a, rows, dst, ldd); break;
    case LLMQ_GGML_Q5_K: hipLaunchKernelGGL(gguf_dequant_rows_kernel<LLMQ_GGML_Q5_K>, dim3(n), dim3(256), 0, ctx->stream, a, rows, dst, ldd); break;
    case LLMQ_GGML_Q6_K: hipLaunchKernelGGL(gguf_dequant_rows_kernel<LLMQ_GGML_Q6_K>, dim3(n), dim3(256), 0, ctx->stream, a, rows, dst, ldd); break;
    default: return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf dequant: type %d", w->ggml_type);
    }
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_gguf_pick_embed_rec(llmq_ctx *ctx, const llmq_mat *E, const ArgmaxPart *parts, int nparts, int B,
                               int *state, int64_t *next, int64_t *gen, float *dst, int64_t ldd, void *rec,
                               const float *rgain) {
    LLMQ_REQUIRE(E && E->kind == MAT_GGUF && parts && nparts > 0 && B > 0 && state && next && gen && dst && rec &&
                     rgain && E->k % 256 == 0 && B <= 65535,
                 "gguf pick embed rec: bad arguments");
    GgufArgs a = make_args(E);
    const HSRec hr = hs_parts(rec, B, E->k);
    const dim3 grid((unsigned)(E->k / 256), (unsigned)((B + 15) / 16 * 16));
#define PR(T)                                                                                                     \
    hipLaunchKernelGGL(gguf_pick_embed_rec_kernel<T>, grid, dim3(256), 0, ctx->stream, a, parts, nparts, B, state, \
                       next, gen, dst, ldd, hr, rgain)
    switch (E->ggml_type) {
    case LLMQ_GGML_Q4_0: PR(LLMQ_GGML_Q4_0); break;
    case LLMQ_GGML_Q4_1: PR(LLMQ_GGML_Q4_1); break;
    case LLMQ_GGML_Q8_0: PR(LLMQ_GGML_Q8_0); break;
    case LLMQ_GGML_Q4_K: PR(LLMQ_GGML_Q4_K); break;
    case LLMQ_GGML_Q5_K: PR(LLMQ_GGML_Q5_K); break;
    case LLMQ_GGML_Q6_K: PR(LLMQ_GGML_Q6_K); break;
    default: return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf pick embed rec: type %d", E->ggml_type);
    }
#undef PR
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_gguf_pick_embed(llmq_ctx *ctx, const llmq_mat *E, const ArgmaxPart *parts, int nparts, int B, int *state,
                           int64_t *next, int64_t *gen, float *dst, int64_t ldd) {
    LLMQ_REQUIRE(E && E->kind == MAT_GGUF && parts && nparts > 0 && B > 0 && state && next && gen && dst,
                 "gguf pick embed: bad arguments");
    GgufArgs a = make_args(E);
#define PE(T)                                                                                                   \
    hipLaunchKernelGGL(gguf_pick_embed_kernel<T>, dim3(B), dim3(256), 0, ctx->stream, a, parts, nparts, B, state, \
                       next, gen, dst, ldd)
    switch (E->ggml_type) {
    case LLMQ_GGML_Q4_0: PE(LLMQ_GGML_Q4_0); break;
    case LLMQ_GGML_Q4_1: PE(LLMQ_GGML_Q4_1); break;
    case LLMQ_GGML_Q8_0: PE(LLMQ_GGML_Q8_0); break;
    case LLMQ_GGML_Q4_K: PE(LLMQ_GGML_Q4_K); break;
    case LLMQ_GGML_Q5_K: PE(LLMQ_GGML_Q5_K); break;
    case LLMQ_GGML_Q6_K: PE(LLMQ_GGML_Q6_K); break;
    default: return llmq_set_error(LLMQ_EUNSUPPORTED, "gguf pick embed: type %d", E->ggml_type);
    }
#undef PE
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
