// Internal declarations shared by libllmq's HIP sources (gfx950 only).
//
// Device layout of a QuantMatrix ("row tiles"): rows are grouped in tiles of
// 16; within a tile the codes are stored chunk-major, 16 bytes per (chunk,
// row), so one wave's 64 lanes (16 rows x 4 consecutive chunks) read 1 KiB
// of contiguous memory with one 128-bit load each:
//
//   codes  byte ((tile * CK + c) * 16 + r) * 16 + b   (CK = 16-byte chunks per row)
//   scales [tile][group][16] float16 bits
//   zps    [tile][group][16] uint8
//
// A chunk holds 32 int4 codes (dword i, nibble j = weight 32c + 8i + j) or 16
// int8 codes (byte b = weight 16c + b).  Rows past the matrix end (the last
// tile of a vocabulary of 50257) hold zero codes and zero scales.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdlib.h>

#include <string>

#include "llmq.h"

#define LLMQ_TILE_ROWS 16
// Chunks (of 16 rows x 16 bytes) of readable padding after a matrix's codes,
// and groups (of 16 rows) after its scales and zero points: covers the GEMV's
// look-ahead of up to 8 steps x 4 chunks past the last tile.
#define LLMQ_PAD_CHUNKS 64

struct llmq_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    hipDeviceProp_t prop{};
    // grow-only workspaces: slot 0 the prompt-side int16 activation codes
    // (and LayerNorm outputs), slot 1 the fp16 activation records of the
    // several-token Q4_K matmul
    void *ws[2] = {nullptr, nullptr};
    size_t ws_bytes[2] = {0, 0};
    void *scratch = nullptr;  // this device's no-allocation scratch (llmq_linear_noalloc), from llmq_init
};

// The context's workspace `slot` of at least `bytes` (api.hip); growing it
// waits for the context's stream first.  Not for use under graph capture.
int ctx_workspace(llmq_ctx *ctx, size_t bytes, void **p, int slot = 0);

enum { MAT_QUANT = 0, MAT_GGUF = 1 };

struct llmq_mat {
    llmq_ctx *ctx = nullptr;
    int kind = MAT_QUANT;
    // QuantMatrix
    int bits = 0, group_param = 0, sym = 0, a16 = 0;
    int64_t n = 0, k = 0, group = 0;  // rows (outputs), cols (reduction), weights per group
    int64_t ntiles = 0, CK = 0, NG = 0;
    uint8_t *codes = nullptr;
    uint16_t *scales = nullptr;
    uint8_t *zps = nullptr;
    // GGUFMatrix: codes above plus the per-chunk / per-superblock fields
    // (gguf.hip); NG counts superblocks per row for the K-quants.
    int ggml_type = -1;
    uint8_t *blocks = nullptr;
    int64_t row_bytes = 0;
    void *g_meta16 = nullptr, *g_meta32 = nullptr, *g_bits32 = nullptr, *g_bits64 = nullptr, *g_sb16 = nullptr;
};

struct llmq_kv {
    llmq_ctx *ctx = nullptr;
    int n_layer = 0, max_t = 0, n_head = 0, head_dim = 0;
    int integer = 0;  // 0: QuantKV[8] (float scales); 1: IntAttnKV (int32 scales * 2^24)
    int8_t *k = nullptr, *v = nullptr;
    float *ks = nullptr, *vs = nullptr;     // QuantKV
    int32_t *kq = nullptr, *vq = nullptr;   // IntAttnKV
};

// Error reporting (api.hip).
int llmq_set_error(int code, const char *fmt, ...);
#define LLMQ_HIP(call)                                                                         \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) return llmq_set_error(LLMQ_EHIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)
#define LLMQ_REQUIRE(cond, ...)                                    \
    do {                                                           \
        if (!(cond)) return llmq_set_error(LLMQ_EINVAL, __VA_ARGS__); \
    } while (0)

#define RC(call)                   \
    do {                           \
        int rc_ = (call);          \
        if (rc_ != LLMQ_OK) return rc_; \
    } while (0)

// Runs the enclosing model call on the context's own (non-null) stream, which
// a decode-step graph can be captured on, after the caller's stream's
// earlier work; the caller's stream is restored on exit.
struct OwnStream {
    llmq_ctx *ctx;
    hipStream_t saved;
    explicit OwnStream(llmq_ctx *c) : ctx(c), saved(c->stream) {
        if (saved != ctx->own_stream) {
            hipStreamSynchronize(saved);
            ctx->stream = ctx->own_stream;
        }
    }
    ~OwnStream() {
        if (saved != ctx->own_stream) {
            hipStreamSynchronize(ctx->own_stream);
            ctx->stream = saved;
        }
    }
};

// Timing events of one call, destroyed on every return path.
struct ScopedEvents {
    hipEvent_t e[3] = {nullptr, nullptr, nullptr};
    int create() {
        for (auto &x : e)
            if (hipEventCreate(&x) != hipSuccess) {
                x = nullptr;
                return llmq_set_error(LLMQ_EHIP, "hipEventCreate failed");
            }
        return LLMQ_OK;
    }
    ~ScopedEvents() {
        for (auto x : e)
            if (x) hipEventDestroy(x);
    }
};

// Captures what enqueue() launches on stream s into an instantiated graph.
// On success *def / *exec receive it; on any failure (a launch error during
// capture, the end of capture, instantiation) nothing is kept, both stay as
// they were and the stream has left capture mode.
template <class F>
int llmq_capture(hipStream_t s, F &&enqueue, hipGraph_t *def, hipGraphExec_t *exec) {
    hipError_t b = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (b != hipSuccess) return llmq_set_error(LLMQ_EHIP, "hipStreamBeginCapture: %s", hipGetErrorString(b));
    int rc = enqueue();
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc == LLMQ_OK && e != hipSuccess)
        rc = llmq_set_error(LLMQ_EHIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    hipGraphExec_t x = nullptr;
    if (rc == LLMQ_OK) {
        hipError_t i = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        if (i != hipSuccess) rc = llmq_set_error(LLMQ_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(i));
    }
    if (rc != LLMQ_OK) {
        if (g) hipGraphDestroy(g);
        return rc;
    }
    *def = g;
    *exec = x;
    return LLMQ_OK;
}

// Argmax partial of one workgroup: the largest value and its (smallest) index.
// Code of column k of row `row` in the QuantMatrix row-tile layout (16-byte
// chunks of 32 int4 codes, weight e at dword e >> 3, nibble e & 7; or of 16
// int8 codes, byte e).  Scalar: for the few rows the reference leaves out of
// its tiles and for parity entry points.
__device__ __forceinline__ int llmq_tile_code(const uint8_t *codes, int bits, int64_t CK, int64_t row, int64_t k) {
    const int64_t tile = row >> 4, r = row & 15;
    if (bits == 4) {
        const int64_t c = k >> 5, e = k & 31;
        const uint8_t b = codes[((tile * CK + c) * 16 + r) * 16 + 4 * (e >> 3) + ((e & 7) >> 1)];
        return (e & 1) ? b >> 4 : b & 15;
    }
    const int64_t c = k >> 4;
    return codes[((tile * CK + c) * 16 + r) * 16 + (k & 15)];
}

// Reference SIMD lane L (0..15) of dot1_i16 (kernels.mojo:617-629), which is
// also QuantMatrix.dot_row_i16's general loop (tensor.mojo:567-577): per
// group an int32 sum (wrapping, as VPDPWSSD) of the lane's pairs
// (2L, 2L + 1) of each 32-input piece of xq * (u - zp), then
// accf = fma(f32(sum), scale, accf) in group order.
__device__ inline float llmq_dot1_lane(const uint8_t *codes, const uint16_t *scales, const uint8_t *zps, int bits,
                                       int64_t K, int64_t G, int64_t CK, int64_t NG, int64_t row, const int16_t *xq,
                                       int L) {
    const int64_t tile = row >> 4, r = row & 15;
    float accf = 0.0f;
    for (int64_t g = 0; g < K / G; g++) {
        const int64_t gi = (tile * NG + g) * 16 + r;
        const int zp = zps[gi];
        uint32_t acc = 0;
        for (int64_t k0 = g * G; k0 < (g + 1) * G; k0 += 32) {
            const int64_t k = k0 + 2 * L;
            acc += (uint32_t)(xq[k] * (llmq_tile_code(codes, bits, CK, row, k) - zp));
            acc += (uint32_t)(xq[k + 1] * (llmq_tile_code(codes, bits, CK, row, k + 1) - zp));
        }
        accf = fmaf((float)(int)acc, __half2float(__ushort_as_half(scales[gi])), accf);
    }
    return accf;
}

// SIMD reduce_add over 16 consecutive lanes as the reference's halving tree:
// (L, L + 8), then + 4, + 2, + 1; every lane of the 16 gets the sum.
__device__ __forceinline__ float llmq_reduce16(float v) {
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    return v;
}

struct ArgmaxPart {
    float v;
    int idx;
};

// ---------------------------------------------------------------- launchers
// Each returns LLMQ_OK or an error code (with llmq_set_error).

int launch_quant_weights(llmq_ctx *ctx, llmq_mat *m, const float *dsrc, int64_t rows, int64_t cols, int reduce_rows);
int launch_quantize_rows(llmq_ctx *ctx, const float *x, int64_t T, int64_t K, int16_t *xq, float *sx);

// Decode's embed step (embed_kernel, attn.hip) done in the prologue of the
// first layer's qkv GEMV: every workgroup picks the token from the previous
// head's argmax partials and forms its embedding row plus position row;
// workgroup 0 also stores the row to x, the token to gen[step] and the
// advanced position and step to state[2], state[3] (state[0], state[1] are
// the ones read; the step's head copies the new pair back).
struct EmbedFold {
    const llmq_mat *E = nullptr;  // the embedding (int4 or int8 codes)
    const float *wpe = nullptr;   // [wpe_rows, E->k] position rows
    int64_t wpe_rows = 0;
    const ArgmaxPart *parts = nullptr;
    int nparts = 0;
    int64_t *gen = nullptr;
    int *state = nullptr;
    float *x = nullptr;
};

// A prompt's QuantKV.store (kv_store_kernel, attn.hip) done by the qkv
// GEMM's epilogue: the workgroups whose 64 rows are one head's keys or
// values quantize them for positions pos0 .. pos0 + T - 1 of `layer`.
struct KvFold {
    llmq_kv *cache = nullptr;  // QuantKV (float scales), head_dim 64
    int layer = 0, pos0 = 0;
};

struct GemvRequest {
    const llmq_mat *w = nullptr;
    const float *x = nullptr;  // [T, ldx]
    int64_t ldx = 0;
    const float *ln_w = nullptr, *ln_b = nullptr;  // LayerNorm on the input rows when set
    float *out = nullptr;                          // [T, ldo]
    int64_t ldo = 0;
    const float *bias = nullptr;
    int64_t T = 1;
    int flags = 0;                 // LLMQ_BIAS | LLMQ_GELU | LLMQ_RESID
    ArgmaxPart *amax = nullptr;    // per-workgroup argmax partials (T == 1)
    int amax_cap = 0;              // capacity of amax, in partials
    int *amax_count = nullptr;     // receives the number of partials written
    int32_t *dbg = nullptr;        // per-chunk exact integer sums (T == 1, no LN)
    int16_t *xq_out = nullptr;     // quantized activations of the first token block
    float *sx_out = nullptr;
    void *ws = nullptr;            // caller-given workspace in place of the context's (never grown)
    size_t ws_cap = 0;             // its size in bytes
    const EmbedFold *emb = nullptr;  // the embed step in the prologue (x unused; exact one-token kernel)
    int *state_copy = nullptr;       // the kernel copies state_copy[2..3] to [0..1] (exact one-token kernel)
    const KvFold *kv = nullptr;      // the cache store in the prompt GEMM's epilogue (gemm_kv_fold_ok)
};
int launch_gemv_a16(llmq_ctx *ctx, const GemvRequest &rq);
// Number of argmax partials launch_gemv_a16 writes for a T == 1 GEMV of w
// (ln: with the LayerNorm prologue).
int gemv_a16_num_parts(const llmq_mat *w, bool ln);
// The T == 1 kernel (gemv1.hip) behind launch_gemv_a16.
bool gemv1_supports(const llmq_mat *w, bool ln);
// The prompt-side int8-MFMA GEMM (gemm_mfma.hip): xq / sx are T x K int16
// codes and T scales of workspace; with `planes` (gemm_f16_planes_bytes of
// workspace, for matrices gemm_f16_supports takes: int4 in groups of 32)
// the codes also go there as fp16 planes and the fp16 matrix-core form runs.
bool gemm_mfma_supports(const llmq_mat *w, int64_t T);
bool gemm_f16_supports(const llmq_mat *w, int64_t T);
// Whether launch_gemv_a16 takes w's T-token product on the fp16 GEMM in the
// tile whose epilogue can store the key / value rows (GemvRequest::kv).
bool gemm_kv_fold_ok(const llmq_mat *w, int64_t T, const llmq_kv *cache);
size_t gemm_f16_planes_bytes(const llmq_mat *w, int64_t T);
int launch_gemm_mfma(llmq_ctx *ctx, const GemvRequest &rq, int16_t *xq, float *sx, uint8_t *planes);
int launch_gemv1(llmq_ctx *ctx, const GemvRequest &rq);
int gemv1_num_parts(const llmq_mat *w, bool ln);
// One-token kernels in the reference's float order (gemv_exact.hip) for
// BLOCKED int4-g32-a16 and int8 per-channel A16 matrices; used unless
// LLMQ_EXACT=0 (then gemv1, whose float sums run in another order).
bool gemv_exact_supports(const llmq_mat *w);
int gemv_exact_num_parts(const llmq_mat *w);
// Whether the exact kernel of w (with LayerNorm) can take the embed step of
// embedding E in its prologue (GemvRequest::emb).
bool gemv_exact_embed_ok(const llmq_mat *w, const llmq_mat *E);
int launch_gemv_exact(llmq_ctx *ctx, const GemvRequest &rq);
// QuantMatrix.dot_row_i16 for rows row0 .. row0 + nrows - 1 (gemv_exact.hip).
int launch_dot_row_i16(llmq_ctx *ctx, const llmq_mat *w, int64_t row0, int64_t nrows, const int16_t *xq, float *out);

// A prepared activation record (llmq_act_prepare): one token's row after
// quantize_rows, in the forms the one-token integer GEMVs read, at byte
// offsets of one device buffer:
//   planes [K / 32][16] u32  nibble planes of X = xq + 32768 per code dword
//   hsum   [K / 32][2]  i32  sum of xq over each half of a 32-chunk
//   xq     [K]          i16  the codes, natural order
//   xsl    [16]         i32  sum of the pairs (2L, 2L + 1) of every 32-piece
//   sx     float             the row's scale
struct ActLayout {
    int64_t planes, hsum, xq, xsl, sx, bytes;
};
__host__ __device__ inline ActLayout llmq_act_layout(int64_t K) {
    ActLayout L;
    const int64_t ck = K / 32;
    L.planes = 0;
    L.hsum = ck * 64;
    L.xq = ck * 72;
    L.xsl = (L.xq + 2 * K + 15) & ~(int64_t)15;
    L.sx = L.xsl + 64;
    L.bytes = L.sx + 16;
    return L;
}
int launch_act_prepare(llmq_ctx *ctx, const float *x, int64_t K, const float *ln_w, const float *ln_b, void *rec);
int launch_linear_act(llmq_ctx *ctx, float *out, const void *rec, const llmq_mat *w, const float *bias, int flags);
inline bool exact_order() {
    const char *e = getenv("LLMQ_EXACT");
    return !(e && e[0] == '0');
}

// GGUF formats (gguf.hip).
int gguf_is_supported(int ggml_type);
int gguf_block_size(int ggml_type);   // weights per block (gguf.mojo:72-83)
int gguf_block_bytes(int ggml_type);  // bytes per block (gguf.mojo:86-98)
int gguf_upload(llmq_ctx *ctx, llmq_mat *m, int ggml_type, const uint8_t *blocks, int64_t rows, int64_t cols);
int gguf_num_parts(const llmq_mat *w);
// One-token GGUF GEMV (gguf1.hip); with rms_g the row is RMS-normalized
// (times the gain rms_g) before the product; with swiglu, x holds 2K floats
// [gate | up] and the row is silu(gate) * up; with ln_w the row goes through
// LayerNorm (eps 1e-5, weight ln_w, bias ln_b) first.  With apart, x is
// not read: the row is the combination of decode attention splits (64-dim
// heads, ns_max splits of asplit positions a head, position astate[0]; the
// split record above), which gguf_gemv_attn_ok(w, ns_max, head_dim) says
// the kernel can take.
// The decode attention split record (written by llama.hip's split kernels,
// read by its combine kernel and by the Wo GEMV in gguf1.hip): per head of
// kLlmqSplitHD dimensions and split, the maximum score m, the sum t of
// exp(score - m), two unused floats, then the head's kLlmqSplitHD partial
// value sums; at most kLlmqMaxSplits splits a head.
constexpr int kLlmqSplitHD = 64;
constexpr int kLlmqSplitRec = 4 + kLlmqSplitHD;  // floats of one record
constexpr int kLlmqMaxSplits = 8;
int launch_gguf_gemv(llmq_ctx *ctx, const llmq_mat *w, const float *x, float *out, const float *bias, int flags,
                     ArgmaxPart *amax, int amax_cap, const float *rms_g = nullptr, float rms_eps = 0.0f,
                     int swiglu = 0, const float *ln_w = nullptr, const float *ln_b = nullptr,
                     const float *apart = nullptr, const int *astate = nullptr, int asplit = 0, int ans_max = 0);
bool gguf_gemv_attn_ok(const llmq_mat *w, int ns_max, int head_dim);
int launch_gguf_dequant_row(llmq_ctx *ctx, const llmq_mat *w, int64_t row, float *dst);
int launch_gguf_dequant_rows(llmq_ctx *ctx, const llmq_mat *w, const int64_t *rows, int n, float *dst, int64_t ldd);
// Greedy pick of each of B sequences from a head's argmax partials (nparts
// per sequence), the decode state advanced, and the picked rows of the GGUF
// embedding E into dst + b * ldd (gguf.hip).
int launch_gguf_pick_embed_rec(llmq_ctx *ctx, const llmq_mat *E, const ArgmaxPart *parts, int nparts, int B,
                               int *state, int64_t *next, int64_t *gen, float *dst, int64_t ldd, void *rec,
                               const float *rgain);
int launch_gguf_pick_embed(llmq_ctx *ctx, const llmq_mat *E, const ArgmaxPart *parts, int nparts, int B, int *state,
                           int64_t *next, int64_t *gen, float *dst, int64_t ldd);
// Prompt attention over an int8 cache of n_kv heads (attn.hip): query head h
// reads cached head h / (n_head / n_kv) of `layer` (a slot index), the rows
// position-major (slot * max_t + pos) * n_kv + head (the KVCache layout) or,
// with head_major, (slot * n_kv + head) * max_t + pos.
int launch_attend_prompt(llmq_ctx *ctx, const int8_t *K8, const int8_t *V8, const float *KS, const float *VS,
                         int layer, int max_t, int n_head, int n_kv, const float *qkv, int64_t ld, int pos0, int T,
                         float *out, int64_t ldo, bool head_major = false);
// QuantMatrix with float activations (A16 = False) runs on the two GGUF
// float-activation kernels (launch_gguf_gemv, launch_gguf_gemm) as two
// internal types past the ggml range, over its own device layout (codes
// [tile][chunk][16 rows][16 B] in natural order, f16 scales and u8 zero
// points [tile][group][16 rows]).
constexpr int kQmFloat4 = 1004, kQmFloat8 = 1008;
inline bool is_float_act(const llmq_mat *w) { return w->kind == MAT_GGUF || (w->kind == MAT_QUANT && !w->a16); }
inline int float_act_type(const llmq_mat *w) {
    return w->kind == MAT_GGUF ? w->ggml_type : (w->bits == 8 ? kQmFloat8 : kQmFloat4);
}
// log2 of the chunks per group of a QuantMatrix (31 for per-channel: every
// chunk of a row is group 0); groups are powers of two times 32 otherwise.
int qm_cpg_shift(const llmq_mat *w);
// Several-token GGUF matmul on the fp32 matrix cores (gguf_gemm.hip).
// Q4_K matrices with whole superblocks take the fp16 matrix cores over an
// h16 record of x (gguf_gemm16.hip): `rec` of `rec_cap` bytes when given,
// the context's workspace slot 1 when rec_cap < 0, and the fp32 kernel when
// rec_cap == 0 (callers that may not allocate); LLMQ_GEMM_H16=0 forces the
// fp32 kernel.
int launch_gguf_gemm(llmq_ctx *ctx, const llmq_mat *w, const float *x, int64_t ldx, int64_t T, float *out,
                     int64_t ldo, const float *bias, int flags, void *rec = nullptr, int64_t rec_cap = -1);
// The h16 record (gguf_gemm16.hip): its size for T tokens of K inputs, the
// record kernel, and the Q4_K matmul over a record.
int64_t h16_rec_bytes(int64_t T, int64_t K);
void h16_rec_parts(void *rec, int64_t T, int64_t K, uint8_t **planes, _Float16 **sums, float **inv);
bool gguf_gemm_h16_ok(const llmq_mat *w);
int launch_act_h16(llmq_ctx *ctx, const float *x, int64_t ldx, int64_t T, int64_t K, void *rec);
// The batch-decode chain's forms of that matmul (gguf_gemm16.hip): the
// input may be an "h16s" record (a scale per 16 inputs of a token, written
// by the previous matmul's epilogue), its outputs then times each token's
// 1 / rms from the record's sums of squares (norm); the epilogue may write
// the next matmul's h16s record: of (out + residual) * gain (LLMQ_RESID),
// or, swiglu (rows [gate; up]), of silu(gate) * up alone.
struct H16Fuse {
    bool in_s = false;
    bool norm = false;
    float eps = 0.0f;
    void *out_rec = nullptr;
    const float *gain = nullptr;
    bool swiglu = false;
};
int launch_gguf_gemm_h16(llmq_ctx *ctx, const llmq_mat *w, const void *rec, int64_t T, float *out, int64_t ldo,
                         const float *bias, int flags, const H16Fuse *fz = nullptr);
int64_t h16s_rec_bytes(int64_t T, int64_t K);
// the h16s record of x * gain (with the sums of squares of x)
int launch_rec_h16s(llmq_ctx *ctx, const float *x, int64_t ldx, int64_t T, int64_t K, const float *gain, void *rec);
// whether the fused forms take w at T tokens (swiglu: as the [gate; up] matrix)
bool gguf_gemm_h16s_ok(const llmq_mat *w, bool swiglu, int64_t T);
// int16 output head for Q6_K / Q8_0 (gguf_head.hip).
int gguf_has_i16(const llmq_mat *w);
// with rms_g, each row of h is RMS-normalized (times rms_g) first; with
// amax, each workgroup leaves each token's largest logit over its rows in
// amax[token * gguf_head16_parts(w) + workgroup]
int launch_gguf_head16(llmq_ctx *ctx, const llmq_mat *w, const float *h, float *logits, int64_t T,
                       const float *rms_g = nullptr, float rms_eps = 0.0f, ArgmaxPart *amax = nullptr,
                       int amax_cap = 0);
int gguf_head16_parts(const llmq_mat *w);

int launch_layernorm(llmq_ctx *ctx, float *out, const float *x, const float *w, const float *b, int64_t T, int64_t C);
int launch_kv_store(llmq_ctx *ctx, llmq_kv *kv, int layer, int pos0, const int *pos_dev, const float *qkv, int T,
                    int64_t ld);
// store: also quantize and store the token's key and value (T == 1).
int launch_kv_attend(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
                     const int *pos_dev, int64_t ld, bool store);
// One decode token's qkv GEMV (LayerNorm fused) + KV store + attention, one
// workgroup per head (qkv_attn.hip); LLMQ_EUNSUPPORTED (no error recorded)
// when the shapes do not fit it.
int launch_qkv_attn(llmq_ctx *ctx, const llmq_mat *w, const float *x, const float *ln_w, const float *ln_b,
                    const float *bias, llmq_kv *kv, int layer, int pos0, const int *pos_dev, float *qkv_out,
                    float *att);
// The same two steps for an IntAttnKV cache (kv->integer; int_attn.hip);
// launch_kv_store / launch_kv_attend route there by themselves.
int launch_ikv_store(llmq_ctx *ctx, llmq_kv *kv, int layer, int pos0, const int *pos_dev, const float *qkv, int T,
                     int64_t ld);
int launch_ikv_attend(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0,
                      const int *pos_dev, int64_t ld, bool store);

// Embedding: x[t] = E.dequant_row(token_t) + wpe[pos0 + t] (gpt2t.mojo:378-385,
// 495-502).  With parts != nullptr the single token is first chosen as the
// argmax of the previous head (gpt2t.mojo:792-797) from nparts partials,
// written to gen[state[1]], and state = {pos, step} is advanced.
int launch_embed(llmq_ctx *ctx, const llmq_mat *E, const float *wpe, const int64_t *tokens, int T, int pos0,
                 float *x, const ArgmaxPart *parts, int nparts, int64_t *gen, int *state, int do_embed);

// Device helpers.
__device__ __forceinline__ int llmq_to_int(float r) {
    // Int(round(v)) for a rounded float, saturating (NaN -> 0), so the code
    // clamp that follows is defined for every input.
    if (r != r) return 0;
    if (r > 1.0e9f) return 1000000000;
    if (r < -1.0e9f) return -1000000000;
    return (int)r;
}

// ------------------------------------------------------ exp, tanh and GELU
// The float path's exp (attend_float_one's softmax, kvcache.mojo:131-138)
// and tanh (store_out's GELU, kernels.mojo:43-45), written out so that every
// kernel computes them with the same operations:
//
//   exp(x): Cody and Waite's reduction x = n ln2 + r (n = rint(x log2 e), ln2
//   split into a 24-bit head and a tail, both products exact inside the
//   fma), then e^r = 1 + r + r^2 P(r) with P of degree 4 fitted by weighted
//   least squares at 4000 Chebyshev nodes on [-0.35, 0.35], evaluated by
//   Horner's rule in fma, then scaled by 2^n through the exponent bits.
//   Results stay normal: x < -87 returns 0 and x > 88.5 infinity.  Error
//   under 1 ulp of the float64 exp over [-87, 88].
//
//   tanh(y): below |y| = 0.625, y + y^3 Q(y^2) with Q of degree 5 fitted the
//   same way; above, 1 - 2 / (exp(2|y|) + 1) with the sign of y (no
//   cancellation there: the quotient is below 0.45); 1 from |y| = 10.  Error
//   under 1.3 ulp of the float64 tanh.
//
// Both are compiled with -ffp-contract=off: each operation rounds as
// written.
__device__ __forceinline__ float ref_expf(float x) {
    if (x > 88.5f) return __builtin_huge_valf();
    if (!(x >= -87.0f)) return x != x ? x : 0.0f;
    const float n = rintf(x * 1.44269502f);
    float r = fmaf(-n, 0.693145752f, x);
    r = fmaf(-n, 1.42860677e-06f, r);
    float p = 0.0013748823f;
    p = fmaf(p, r, 0.008369628f);
    p = fmaf(p, r, 0.041669644f);
    p = fmaf(p, r, 0.16666512f);
    p = fmaf(p, r, 0.49999988f);
    const float r2 = r * r;
    p = fmaf(p, r2, r);
    p = p + 1.0f;
    return p * __uint_as_float((uint32_t)((int)n + 127) << 23);
}
__device__ __forceinline__ float ref_tanhf(float y) {
    const float a = fabsf(y);
    if (a < 0.625f) {
        const float s = y * y;
        float p = 0.002148991f;
        p = fmaf(p, s, -0.00818467f);
        p = fmaf(p, s, 0.021704003f);
        p = fmaf(p, s, -0.053947456f);
        p = fmaf(p, s, 0.13333212f);
        p = fmaf(p, s, -0.3333333f);
        return fmaf(p * s, y, y);
    }
    const float t = a >= 10.0f ? 1.0f : 1.0f - 2.0f / (ref_expf(2.0f * a) + 1.0f);
    return copysignf(t, y);
}
// GELU of kernels.store_out / finish (kernels.mojo:43-45, 277-279),
// operation by operation: 0.5 r (1 + tanh(s (r + ((0.044715 r) r) r))).
__device__ __forceinline__ float gelu_ref(float r) {
    const float s = 0.7978845608028654f;
    float t = 0.044715f * r;
    t = t * r;
    t = t * r;
    const float u = r + t;
    const float th = ref_tanhf(s * u);
    const float h = 0.5f * r;
    return h * (1.0f + th);
}

// ------------------------------------------- buffer loads and LDS barriers
// Raw buffer loads from a uniform base: an offset at or past the extent
// reads zeros without touching memory (how lanes and steps that carry no
// data are switched off without branches).  Extents stay below 2 GiB.
constexpr uint32_t kLlmqOOB = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t llmq_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 llmq_bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t llmq_bload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t llmq_bload2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t llmq_bload1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}
// Workgroup barrier that orders LDS only (global loads stay in flight).
__device__ __forceinline__ void llmq_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------- the reference's float reductions
// SIMD[f32, 16].reduce_add as a halving tree, lanes (l, l + 8), then
// (l, l + 4), (l, l + 2), (l, l + 1): each aligned group of 16 lanes holds
// the 16 values, lane 0 of the group gets the sum (the other lanes hold
// partial sums).  Float addition is commutative, so which lane of a pair
// adds is immaterial; the pairing is what fixes the bits.
// DPP row_shl:n gives lane l the value of lane l + n of its row of 16.
template <int CTRL>
__device__ __forceinline__ float llmq_dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float llmq_red16(float v) {
    v = v + llmq_dppf<0x108>(v);
    v = v + llmq_dppf<0x104>(v);
    v = v + llmq_dppf<0x102>(v);
    return v + llmq_dppf<0x101>(v);
}

// layernorm's statistics (kernels.mojo:179-197) over x[0, C) in LDS, in
// the reference's order: 16 lane partials s_l = x[l] + x[16 + l] + ...
// (left to right), mean = reduce_add(s) / C; the same for (x - mean)^2
// (multiply, then add); rstd = 1 / sqrt(reduce_add / C + 1e-5).  Called by
// every thread of the workgroup (C a multiple of 16); wave 0 computes, bc
// (2 floats of LDS) broadcasts.  Ends with a barrier.
// Lane l's partial sum of x[l], x[l + 16], ... (or of their squared
// deviations from `mean` when SQ), left to right; the LDS reads of a batch
// of 16 values are issued before its adds, so the chain waits once a batch.
template <bool SQ>
__device__ __forceinline__ float llmq_lane_chain(const float *xs, int C, int l, float mean) {
    float s = 0.0f;
    int i = l;
    for (; i + 16 * 15 < C; i += 256) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = xs[i + 16 * k];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (SQ) {
                const float d = v[k] - mean;
                s += d * d;
            } else {
                s += v[k];
            }
        }
    }
    for (; i < C; i += 16) {
        if (SQ) {
            const float d = xs[i] - mean;
            s += d * d;
        } else {
            s += xs[i];
        }
    }
    return s;
}
__device__ __forceinline__ void llmq_ln_stats(const float *xs, int C, float *bc, float &mean, float &rstd) {
    if (threadIdx.x < 64) {
        const int l = threadIdx.x & 15;
        const float m = llmq_red16(llmq_lane_chain<false>(xs, C, l, 0.0f)) / (float)C;
        const float mb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
        const float r = 1.0f / sqrtf(llmq_red16(llmq_lane_chain<true>(xs, C, l, mb)) / (float)C + 1e-5f);
        if (threadIdx.x == 0) {
            bc[0] = mb;
            bc[1] = r;
        }
    }
    llmq_lds_barrier();
    mean = bc[0];
    rstd = bc[1];
}

// The same statistics from registers, for C = 16 NV: lane l (of wave 0,
// any of its rows of 16) holds v[i] = x[16 i + l]; returns (mean, rstd) in
// every lane of the wave.
template <int NV>
__device__ __forceinline__ float2 llmq_ln_stats_regs(const float (&v)[NV]) {
    constexpr float C = (float)(16 * NV);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) s += v[i];
    const float m = llmq_red16(s) / C;
    const float mb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const float d = v[i] - mb;
        q += d * d;
    }
    const float r = 1.0f / sqrtf(llmq_red16(q) / C + 1e-5f);
    return make_float2(mb, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0)));
}

// v of lane l + 32 (l < 32) / l + 16 (even rows of 16): gfx950's lane swaps.
__device__ __forceinline__ float llmq_from_lane_plus32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[1]);
}
__device__ __forceinline__ float llmq_from_lane_plus16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[1]);
}
__device__ __forceinline__ int llmq_from_lane_plus32(int v) {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (int)r[1];
}

// Sum / max over the wave in every lane, without LDS: DPP within rows of 16
// (quad swaps, half-row and row mirrors), then gfx950's row-pair and
// half-wave swaps.  Every lane forms the same pairs, so all lanes hold the
// same bits; the order is this butterfly's (for sums where the reference
// fixes no order).
__device__ __forceinline__ float llmq_wave_sum_all(float v) {
    v = v + llmq_dppf<0xB1>(v);   // quad_perm [1,0,3,2]
    v = v + llmq_dppf<0x4E>(v);   // quad_perm [2,3,0,1]
    v = v + llmq_dppf<0x141>(v);  // row_half_mirror
    v = v + llmq_dppf<0x140>(v);  // row_mirror
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}
__device__ __forceinline__ float llmq_wave_max_all(float v) {
    v = fmaxf(v, llmq_dppf<0xB1>(v));
    v = fmaxf(v, llmq_dppf<0x4E>(v));
    v = fmaxf(v, llmq_dppf<0x141>(v));
    v = fmaxf(v, llmq_dppf<0x140>(v));
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
}

// Sum and maximum over the 32 lanes of each half of the wave.
__device__ __forceinline__ float llmq_half_sum(float v) {
    v = v + llmq_dppf<0xB1>(v);
    v = v + llmq_dppf<0x4E>(v);
    v = v + llmq_dppf<0x141>(v);
    v = v + llmq_dppf<0x140>(v);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float llmq_half_max(float v) {
    v = fmaxf(v, llmq_dppf<0xB1>(v));
    v = fmaxf(v, llmq_dppf<0x4E>(v));
    v = fmaxf(v, llmq_dppf<0x141>(v));
    v = fmaxf(v, llmq_dppf<0x140>(v));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// One superblock (256 inputs) of one token of an h16 activation record (the
// fp16-plane form of a float row that gemm_h16_q4k_kernel reads; layout in
// gguf_gemm16.hip), written by one wave: lane k holds inputs k + 64 q,
// q = 0..3, of superblock sb of token t in v[q] (zeros for padding).  The
// superblock's scale is the power of two s with max |x| s < 2^10; the
// input planes get hi = fp16(x s) and lo = fp16(x s - hi), the sum planes
// the same split of s times each 32-input sub-block's sum, and inv 1 / s.
// Every lane of the wave calls it (the reductions span the wave); ok = false
// stores nothing.
__device__ __forceinline__ void llmq_h16_store(uint8_t *planes, _Float16 *sums, float *inv, int KB, int NSB, int t,
                                               int sb, const float (&v)[4], bool ok) {
    const int k = threadIdx.x & 63;
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    m = llmq_wave_max_all(m);
    int ex = 0;
    frexpf(m, &ex);  // m < 2^ex
    const int e = min(126, max(-126, 10 - ex));
    const float s = ldexpf(1.0f, e);
    const int kk = k & 31, g = kk >> 3, i = kk & 7, pos = (i & 1) ? 4 + (i >> 1) : (i >> 1);
    const int64_t tt = t >> 4, c = t & 15;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float sx = llmq_half_sum(v[q]) * s;  // sub-block 2q + k / 32
        const float xs = v[q] * s;
        const _Float16 hi = (_Float16)xs, lo = (_Float16)(xs - (float)hi);
        const _Float16 shi = (_Float16)sx, slo = (_Float16)(sx - (float)shi);
        if (ok) {
            const int j = 2 * q + (k >> 5);
            _Float16 *p = reinterpret_cast<_Float16 *>(planes) + ((tt * KB + sb * 8 + j) * 1024 + (g * 16 + c) * 8 + pos);
            p[0] = hi;
            p[512] = lo;
            if (kk == 0) {
                _Float16 *ps = sums + (tt * NSB + sb) * 256 + c * 8 + j;
                ps[0] = shi;
                ps[128] = slo;
            }
        }
    }
    if (ok && k == 0) inv[(tt * NSB + sb) * 16 + c] = ldexpf(1.0f, -e);
}

template <int CTRL>
__device__ __forceinline__ int llmq_dppi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int llmq_wave_max_all(int v) {
    v = max(v, llmq_dppi<0xB1>(v));
    v = max(v, llmq_dppi<0x4E>(v));
    v = max(v, llmq_dppi<0x141>(v));
    v = max(v, llmq_dppi<0x140>(v));
    const auto r16 = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    v = max((int)r16[0], (int)r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return max((int)r32[0], (int)r32[1]);
}

// max over the wave, in every lane (order-free): DPP within rows of 16, then
// the four rows' results.
__device__ __forceinline__ float llmq_wave_max(float v) {
    v = fmaxf(v, llmq_dppf<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, llmq_dppf<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, llmq_dppf<0x141>(v));  // row_half_mirror
    v = fmaxf(v, llmq_dppf<0x140>(v));  // row_mirror
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
