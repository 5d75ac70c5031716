/*
 * llmq.h -- C ABI of libllmq.so, the MI355X (gfx950) implementation of
 * llm_mojo's quantized-weight matmul path.
 *
 * The reference selects weight formats through the Mojo trait WeightMatrix
 * (tensor.mojo:49-147) and KV formats through KVCache (kvcache.mojo:31-87);
 * its kernels (kernels.mojo) call those per output row.  A GPU format cannot
 * be driven per row, so this library is driven per whole matmul (linear /
 * head), per KV store / attention, or per decode step.  Each declaration
 * below names the reference interface it stands in for.
 *
 * Conventions
 *   - Every function returns LLMQ_OK (0) or a negative LLMQ_E* code; on error
 *     llmq_last_error() describes it (thread-local).  Nothing throws across
 *     this boundary.
 *   - "host" pointers are CPU memory, "device" pointers are GPU memory.  All
 *     compute entry points take device pointers and are stream-ordered on the
 *     context's stream: they return before the GPU finishes; llmq_sync waits.
 *   - Handles (llmq_mat, llmq_kv, llmq_gpt2) own their device memory and are
 *     released exactly once with their *_free function (tensor.mojo:49-55).
 *   - A context is used from one host thread at a time (the reference's
 *     thread 0 of the decode team, kernels.mojo:802-806).
 */
#ifndef LLMQ_H
#define LLMQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define LLMQ_API __attribute__((visibility("default")))
#else
#define LLMQ_API
#endif

enum {
    LLMQ_OK = 0,
    LLMQ_EINVAL = -1,      /* bad argument (the reference abort()s or raises) */
    LLMQ_EHIP = -2,        /* a HIP runtime call failed */
    LLMQ_ENOMEM = -3,      /* device allocation failed */
    LLMQ_EUNSUPPORTED = -4 /* a format or shape this build does not cover */
};

/* Epilogue flags of linear: kernels.linear's RESID / GELU parameters and
 * matmul_rows_a16's BIAS (kernels.mojo:38-48, 419-421, 655-673). */
enum { LLMQ_BIAS = 1, LLMQ_GELU = 2, LLMQ_RESID = 4 };

/* ggml tensor types accepted by llmq_mat_from_gguf (gguf.mojo:41-49). */
enum {
    LLMQ_GGML_F32 = 0, LLMQ_GGML_F16 = 1, LLMQ_GGML_Q4_0 = 2, LLMQ_GGML_Q4_1 = 3,
    LLMQ_GGML_Q8_0 = 8, LLMQ_GGML_Q4_K = 12, LLMQ_GGML_Q5_K = 13, LLMQ_GGML_Q6_K = 14
};

typedef struct llmq_ctx llmq_ctx;
typedef struct llmq_mat llmq_mat;
typedef struct llmq_kv llmq_kv;
typedef struct llmq_gpt2 llmq_gpt2;

/* ---------------------------------------------------------------- context */

/* No reference counterpart (the reference is CPU-only): one GPU, one stream. */
LLMQ_API int llmq_init(int device, llmq_ctx **ctx);
LLMQ_API int llmq_destroy(llmq_ctx *ctx);
LLMQ_API const char *llmq_last_error(void);
/* Makes the context issue its work on an existing HIP stream (e.g. a
 * framework's current stream); NULL returns to the context's own stream. */
LLMQ_API int llmq_set_stream(llmq_ctx *ctx, void *hip_stream);
LLMQ_API int llmq_sync(llmq_ctx *ctx);
/* Device memory helpers for callers without an allocator of their own. */
LLMQ_API int llmq_malloc(llmq_ctx *ctx, size_t bytes, void **dptr);
LLMQ_API int llmq_free(llmq_ctx *ctx, void *dptr);
LLMQ_API int llmq_memcpy_h2d(llmq_ctx *ctx, void *dst, const void *src, size_t bytes);
LLMQ_API int llmq_memcpy_d2h(llmq_ctx *ctx, void *dst, const void *src, size_t bytes);

/* ------------------------------------------------ weight matrices (formats) */

/* QuantMatrix[bits, group, sym, a16].from_f32 (tensor.mojo:334-383):
 * quantizes a row-major float32 host matrix src[rows, cols] on the GPU,
 * bit-identical to the reference (float16 RNE scales, integer zero points,
 * round-half-away codes).  reduce_rows as in the trait (tensor.mojo:76-85):
 * 1 for layer matrices in Hugging Face [IN, OUT] layout (stored transposed,
 * one output per row), 0 for wte [V, C].  bits 4 or 8; group 32, 64, 128 or
 * 0 for per-channel.  a16 selects the int16-activation kernels (ACT16,
 * tensor.mojo:66-69); the device layout is the same either way. */
LLMQ_API int llmq_mat_from_f32(llmq_ctx *ctx, int bits, int group, int sym, int a16, const float *src,
                               int64_t rows, int64_t cols, int reduce_rows, llmq_mat **out);
/* Same, with src already in device memory. */
LLMQ_API int llmq_mat_from_f32_device(llmq_ctx *ctx, int bits, int group, int sym, int a16, const float *src,
                                      int64_t rows, int64_t cols, int reduce_rows, llmq_mat **out);
/* GGUFMatrix(data, kind, rows, cols) (gguf.mojo:344-371): blocks used as
 * stored, rows of cols // block_size blocks, copied from host memory. */
LLMQ_API int llmq_mat_from_gguf(llmq_ctx *ctx, int ggml_type, const void *blocks, int64_t rows, int64_t cols,
                                llmq_mat **out);
/* GGUFFile (gguf.mojo:519-636): a GGUF v2 / v3 file's tensor index over a
 * read-only mapping of the file (every read bounds-checked).  Tensors are
 * (name, ggml type, rows = product of dims[1..], cols = dims[0], offset in
 * the data section, which starts at the general.alignment boundary, 32 by
 * default).  llmq_gguf_find gives the index of a name or -1 (GGUFFile.has);
 * llmq_gguf_tensor_data a host pointer to its bytes in the mapping;
 * llmq_gguf_matrix is GGUFFile.matrix (gguf.mojo:622-633) on the device
 * (llmq_mat_from_gguf: block formats; F32 / F16 tensors are read with
 * llmq_gguf_tensor_data).  The handle must outlive the pointers it gave. */
typedef struct llmq_gguf llmq_gguf;
LLMQ_API int llmq_gguf_open(const char *path, llmq_gguf **out);
LLMQ_API int llmq_gguf_close(llmq_gguf *g);
LLMQ_API int64_t llmq_gguf_n_tensors(const llmq_gguf *g);
LLMQ_API int llmq_gguf_find(const llmq_gguf *g, const char *name, int64_t *index);
LLMQ_API int llmq_gguf_tensor_info(const llmq_gguf *g, int64_t index, const char **name, int *ggml_type,
                                   int64_t *rows, int64_t *cols, int64_t *offset);
LLMQ_API int llmq_gguf_tensor_data(const llmq_gguf *g, int64_t index, const void **data, int64_t *bytes);
LLMQ_API int llmq_gguf_matrix(llmq_ctx *ctx, const llmq_gguf *g, const char *name, llmq_mat **out);

/* WeightMatrix.free (tensor.mojo:145-147). */
LLMQ_API int llmq_mat_free(llmq_mat *mat);
/* WeightMatrix.nbytes (tensor.mojo:131-133; QuantMatrix 629-632,
 * GGUFMatrix 507-508): bytes of the format as the reference counts them. */
LLMQ_API int64_t llmq_mat_nbytes(const llmq_mat *mat);
/* WeightMatrix.group_size (tensor.mojo:127-129, gguf.mojo:459-460). */
LLMQ_API int64_t llmq_mat_group_size(const llmq_mat *mat);
/* WeightMatrix.has_i16 (tensor.mojo:102-104; GGUFMatrix 456-457 of
 * gguf.mojo): 1 when the matrix has an int16-activation kernel (A16
 * QuantMatrix; GGUF Q6_K and Q8_0, whose heads use it), else 0. */
LLMQ_API int llmq_mat_has_i16(const llmq_mat *mat);
/* Shape: rows (outputs) and cols (the reduction axis) as stored. */
LLMQ_API int llmq_mat_shape(const llmq_mat *mat, int64_t *rows, int64_t *cols);
/* The codes, float16 scale bits and zero points in the reference's own
 * QuantMatrix memory layout (tensor.mojo:302-307, nibble_at 385-404,
 * BLOCKED for int4-g32-a16), copied to host buffers of nbytes-matching
 * sizes: rows*cols*bits/8, rows*cols/group, rows*cols/group.  This is the
 * layout QuantMatrix.save writes (tensor.mojo:634-643). */
LLMQ_API int llmq_mat_export(llmq_ctx *ctx, const llmq_mat *mat, uint8_t *codes, uint16_t *scales, uint8_t *zps);
/* WeightMatrix.dequant_row (tensor.mojo:94-96): row `row` as float32 into a
 * host buffer of cols floats. */
/* QuantMatrix.restore (tensor.mojo:646-656): a matrix from its codes in the
 * reference's own layout (BLOCKED for int4-g32-a16, tensor.mojo:385-404;
 * rows x cols * bits / 8 bytes), float16 scales and uint8 zero points
 * (rows x cols / group each), as llmq_mat_export writes them; group 0 is
 * one group per row. */
LLMQ_API int llmq_mat_restore(llmq_ctx *ctx, int bits, int group, int sym, int a16, int64_t rows, int64_t cols,
                              const uint8_t *codes, const uint16_t *scales, const uint8_t *zps, llmq_mat **out);
LLMQ_API int llmq_mat_dequant_row(llmq_ctx *ctx, const llmq_mat *mat, int64_t row, float *dst);
/* QuantMatrix.dot_row_i16 (tensor.mojo:518-577), the trait's per-row int16
 * dot (WeightMatrix.dot_row_i16, tensor.mojo:122-125), for rows row ..
 * row + nrows - 1: out[i] = row (row + i) . xq in weight scale (the caller
 * multiplies by the activations' sx, as matmul_rows_a16 does,
 * kernels.mojo:444-452), bit for bit the reference's float result for each
 * of its three branches (BLOCKED int4-g32, int8 per channel, the general
 * per-group loop).  xq: K int16 activation codes in natural column order
 * (device memory, as llmq_quantize_rows writes them): for BLOCKED matrices
 * permute_x_i16 (tensor.mojo:498-516) is the layout's concern and happens
 * inside.  out: nrows floats of device memory; stream-ordered.  A16
 * matrices only (the others abort in the reference, tensor.mojo:120-125:
 * here LLMQ_EINVAL).  For parity checks; the GEMVs do not use it. */
LLMQ_API int llmq_dot_row_i16(llmq_ctx *ctx, const llmq_mat *mat, int64_t row, int64_t nrows, const int16_t *xq,
                              float *out);

/* --------------------------------------------------------- compute (device) */

/* kernels.quantize_rows (kernels.mojo:400-416): xq[T, K] = round(x / sx),
 * sx[t] = max|x[t]| / 32767 (1 for an all-zero row). */
LLMQ_API int llmq_quantize_rows(llmq_ctx *ctx, const float *x, int64_t T, int64_t K, int16_t *xq, float *sx);
/* kernels.linear (kernels.mojo:655-673; decode team form linear_team
 * 774-866): out[T, OUT] (+)= act(x[T, IN] @ W^T + bias).  For an a16
 * QuantMatrix the activations are quantized per row to int16 and the sums
 * run in integers (matmul_rows_a16, 419-509); for a GGUF matrix or a
 * QuantMatrix with a16 = 0 the float path (matmul_rows, 285-349, over
 * GGUFMatrix.dot_row / QuantMatrix.dot_row, tensor.mojo:431-482).
 * flags: LLMQ_BIAS | LLMQ_GELU | LLMQ_RESID. */
LLMQ_API int llmq_linear(llmq_ctx *ctx, float *out, const float *x, const llmq_mat *w, const float *bias, int64_t T,
                         int64_t IN, int64_t OUT, int flags);
/* No counterpart in the reference: llmq_linear for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results
 * (bit for bit) as llmq_linear; where llmq_linear grows the context's
 * workspace (the a16 prompt GEMM's int16 activation codes and row scales,
 * the Q4_K matmul's fp16 activation record), this form uses a fixed
 * per-GPU scratch array of LLMQ_NOALLOC_SCRATCH_BYTES that each GPU the
 * library runs on holds until the process ends.  It calls no hipMalloc /
 * hipFree.  Sizes needing more scratch than that (a16: T x IN x 2 bytes
 * and T x 4, each rounded up to 256; Q4_K: the record's ~4.4 x T x IN
 * bytes, T rounded up to 16) return LLMQ_EINVAL; other formats use no
 * scratch.  An int4-g32 a16 matrix also puts its prompt GEMM's fp16
 * activation planes there (T x IN x 4 bytes, T rounded up to 16) when they
 * fit, else runs the int8-MFMA form of the same GEMM (the same bits).
 * Every call on one GPU shares the array: calls that overlap in time on one
 * GPU (different streams or threads) race; calls ordered on one stream do
 * not.  Nothing in the scratch needs to start at zero (each call writes all
 * it reads). */
#define LLMQ_NOALLOC_SCRATCH_BYTES (8 << 20)
LLMQ_API int llmq_linear_noalloc(llmq_ctx *ctx, float *out, const float *x, const llmq_mat *w, const float *bias,
                                 int64_t T, int64_t IN, int64_t OUT, int flags);
/* The same with LayerNorm (kernels.layernorm, 179-197; eps 1e-5) applied to
 * each input row first: the LN -> linear pairs of Model.decode
 * (gpt2t.mojo:390-399, 419-428) in one call (one kernel for a16 matrices;
 * for a16 = 0 the LayerNorm goes through the context's workspace, so that
 * form is not for graph capture). */
LLMQ_API int llmq_ln_linear(llmq_ctx *ctx, float *out, const float *x, const float *ln_w, const float *ln_b,
                            const llmq_mat *w, const float *bias, int64_t T, int64_t IN, int64_t OUT, int flags);
/* kernels.head / head_team (kernels.mojo:676-690, 869-910): logits[T, V] =
 * h[T, C] @ W[V, C]^T, no bias.  GGUF Q6_K / Q8_0 heads take the int16 path
 * (head_i16, 693-736). */
LLMQ_API int llmq_head(llmq_ctx *ctx, float *logits, const float *h, const llmq_mat *w, int64_t T, int64_t V,
                       int64_t C);
/* linear_team's prepared activations (kernels.mojo:774-866: thread 0 runs
 * quantize_rows and permute_x_i16 once into the team's xq / xp / xs / sx,
 * then every thread's rows read them): one token's row x[K] (device, after
 * LayerNorm with ln_w / ln_b when given) quantized to int16 once, into the
 * caller's device buffer act of llmq_act_bytes(K) bytes, in the forms the
 * one-token integer GEMVs read (codes, nibble planes, per-half-group and
 * per-lane sums, the scale).  K a multiple of 32, at most 16384. */
LLMQ_API int64_t llmq_act_bytes(int64_t K);
LLMQ_API int llmq_act_prepare(llmq_ctx *ctx, const float *x, int64_t K, const float *ln_w, const float *ln_b,
                              void *act);
/* linear_team's rows over prepared activations (kernels.mojo:793-816,
 * dot_row_i16 * sx + bias, store_out): out[OUT] (+)= act(act @ W^T + bias)
 * for one token, bit-identical to llmq_linear on the same row.  Takes
 * int4-g32-a16 (BLOCKED) and int8 per-channel a16 matrices. */
LLMQ_API int llmq_linear_act(llmq_ctx *ctx, float *out, const void *act, const llmq_mat *w, const float *bias,
                             int64_t IN, int64_t OUT, int flags);
/* kernels.layernorm (kernels.mojo:179-197). */
LLMQ_API int llmq_layernorm(llmq_ctx *ctx, float *out, const float *x, const float *w, const float *b, int64_t T,
                            int64_t C);
/* Parity hook for the integer sums (tensor.mojo:262-275): runs the linear
 * kernel on xf[T=1, IN] and also writes, per output row and per 16-byte code
 * chunk of the device layout, the exact int32 partial
 * sum_k xq_k * (u_k - zp) (chunks of 32 int4 or 16 int8 weights, in column
 * order), plus the quantized activations xq[IN] and their scale sx[1].
 * chunk_sums has OUT * IN / (bits == 4 ? 32 : 16) int32 entries. */
LLMQ_API int llmq_debug_chunk_sums(llmq_ctx *ctx, const float *xf, const llmq_mat *w, float *out, int32_t *chunk_sums,
                                   int16_t *xq, float *sx);
/* Parity/debug: the float path's exp (op 0, attend_float_one's softmax,
 * kvcache.mojo:131-138), tanh (op 1) and GELU (op 2, store_out,
 * kernels.mojo:43-45) as every kernel computes them, elementwise over n
 * device floats x into y.  No reference counterpart (the reference calls
 * Mojo's exp / tanh); for bit-for-bit checks against the oracle. */
LLMQ_API int llmq_debug_refmath(llmq_ctx *ctx, int op, const float *x, float *y, int64_t n);
/* Measurement: reads `bytes` (a multiple of 16) of device memory at buf
 * with `grid` workgroups of 256 threads, eight 128-bit loads in flight per
 * thread, and writes one XOR of the words per workgroup to out[grid]: the
 * read rate a kernel with no arithmetic reaches (the GEMV's floor).  No
 * reference counterpart. */
LLMQ_API int llmq_debug_read(llmq_ctx *ctx, const void *buf, int64_t bytes, uint32_t *out, int grid);

/* ------------------------------------------------------ int8 KV cache */

/* QuantKV[8].create (kvcache.mojo:297-311): int8 keys and values
 * [layer, pos, head, head_dim] with float32 scales [layer, pos, head]. */
LLMQ_API int llmq_kv_create(llmq_ctx *ctx, int n_layer, int max_t, int n_head, int head_dim, llmq_kv **out);
LLMQ_API int llmq_kv_free(llmq_kv *kv);
/* KVCache.nbytes (kvcache.mojo:377-379). */
LLMQ_API int64_t llmq_kv_nbytes(const llmq_kv *kv);
/* QuantKV.store for T consecutive tokens (kvcache.mojo:333-342, called per
 * token at gpt2t.mojo:401-404, 526-530): keys and values are columns C.. and
 * 2C.. of each row of qkv[T, 3C]. */
LLMQ_API int llmq_kv_store(llmq_ctx *ctx, llmq_kv *kv, int layer, int pos0, const float *qkv, int T);
/* KVCache.attend (kvcache.mojo:62-79) with QuantKV's float attention
 * (attend_float_one, 113-150): causal attention of T tokens at positions
 * pos0.. over this layer's cache, which already holds them; out[T, C]. */
LLMQ_API int llmq_kv_attend(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T,
                            int pos0);
/* Copies the cache's codes and scales to host buffers (parity tests). */
LLMQ_API int llmq_kv_export(llmq_ctx *ctx, const llmq_kv *kv, int8_t *k, int8_t *v, float *ks, float *vs);

/* IntAttnKV.create (int_attention.mojo:99-113): the same int8 codes
 * [layer, pos, head, head_dim] with the scales as int32 = round(scale * 2^24)
 * [layer, pos, head].  Shape check of int_attention.mojo:100-101 (max_t % 16,
 * head_dim % 32: LLMQ_EINVAL); this build covers head_dim 64 and 128.
 * llmq_kv_store, llmq_kv_attend, llmq_kv_nbytes and llmq_kv_free take the
 * handle like any cache: store is IntAttnKV.store (132-168), attend runs
 * IntAttnKV.attend_one (170-269) for every token and head, in integers
 * (intmath.masked_exp, intmath.mojo:93-123). */
LLMQ_API int llmq_ikv_create(llmq_ctx *ctx, int n_layer, int max_t, int n_head, int head_dim, llmq_kv **out);
/* 1 for an IntAttnKV cache, 0 for QuantKV[8]. */
LLMQ_API int llmq_kv_is_integer(const llmq_kv *kv);
/* Copies an IntAttnKV cache's codes and int32 scales to host buffers. */
LLMQ_API int llmq_ikv_export(llmq_ctx *ctx, const llmq_kv *kv, int8_t *k, int8_t *v, int32_t *kq, int32_t *vq);

/* ------------------------------------------------ GPT-2 (the caller) */

/* load_model (gpt2t.mojo:579-609) from float32 host tensors in Hugging Face
 * layout, in this order: wte [V, C], wpe [MAX_T, C], ln_f.weight,
 * ln_f.bias, then per layer ln_1.weight, ln_1.bias, attn.c_attn.weight,
 * attn.c_attn.bias, attn.c_proj.weight, attn.c_proj.bias, ln_2.weight,
 * ln_2.bias, mlp.c_fc.weight, mlp.c_fc.bias, mlp.c_proj.weight,
 * mlp.c_proj.bias (4 + 12 * 12 pointers).  Layers become
 * QuantMatrix[bits, group, sym, A16=True] on the device, the tied head
 * HEAD8_A16 = QuantMatrix[8, 0, False, True] (gpt2t.mojo:1231-1235), the
 * cache QuantKV[8] (1238-1244). */
LLMQ_API int llmq_gpt2_create(llmq_ctx *ctx, const float *const *params, int bits, int group, int sym,
                              llmq_gpt2 **out);
/* The same with the attention chosen as gpt2t.mojo's --attention does
 * (gpt2t.mojo:856, 1251-1257): LLMQ_ATTN_FLOAT (QuantKV[8], float
 * attention) or LLMQ_ATTN_INT (IntAttnKV, integer attention). */
enum { LLMQ_ATTN_FLOAT = 0, LLMQ_ATTN_INT = 1 };
LLMQ_API int llmq_gpt2_create_ex(llmq_ctx *ctx, const float *const *params, int bits, int group, int sym,
                                 int attention, llmq_gpt2 **out);
/* The model gpt2t.mojo's main builds for --dtype / --head (1282-1348):
 * dtype a QuantMatrix name (int8-ch, int4-ch, int4-g128, int4-g64, int4-g32,
 * each optionally -sym, each optionally -a16), head "int8" (HEAD8, or
 * HEAD8_A16 for -a16 layers) or "same" (the layers' format). */
LLMQ_API int llmq_gpt2_create_fmt(llmq_ctx *ctx, const float *const *params, const char *dtype, const char *head,
                                  int attention, llmq_gpt2 **out);
LLMQ_API int llmq_gpt2_free(llmq_gpt2 *m);
/* Model.weight_bytes (gpt2t.mojo:312-319). */
LLMQ_API int64_t llmq_gpt2_weight_bytes(const llmq_gpt2 *m);
/* Model.forward (gpt2t.mojo:329-342): tokens (host) at positions pos0..;
 * the last token's logits [V] into a host buffer when logits != NULL. */
LLMQ_API int llmq_gpt2_forward(llmq_gpt2 *m, const int64_t *tokens, int T, int pos0, float *logits);
/* Parity/debug: with codes != NULL (device, 49 * 3072 int16), every later
 * one-token forward or decode step writes the int16 activation codes of
 * each linear's input (quantize_rows, kernels.mojo:400-416): slot 4 l + k
 * for layer l's qkv, proj, fc and fcproj (k = 0..3), slot 48 for the head,
 * 3072 entries a slot (the first IN used).  NULL stops it.  No reference
 * counterpart; it measures the int16 code-flip rate against the oracle. */
LLMQ_API int llmq_gpt2_debug_codes(llmq_gpt2 *m, int16_t *codes);
/* generate with -t 0 (gpt2t.mojo:929-1009): the prompt forward, then up to
 * `steps` greedy tokens (argmax, first maximum wins, gpt2t.mojo:792-797),
 * each fed back as the next input, entirely on the device.  Writes the
 * generated ids to out_tokens (host), stopping at the first EOT (50256) as
 * the reference does, and returns the count in *n_out.  prefill_ms and
 * decode_ms (either may be NULL) are the reference's timing spans: the
 * prompt forward, and the steps - 1 decode forwards plus the argmaxes. */
LLMQ_API int llmq_gpt2_generate(llmq_gpt2 *m, const int64_t *prompt, int n_prompt, int steps, int64_t *out_tokens,
                                int *n_out, double *prefill_ms, double *decode_ms);
/* Model.forward_all (gpt2t.mojo:448-459): the T tokens from position 0,
 * then LN_f and the head on every row: logits[T, V] (device memory), row t
 * predicting token t + 1. */
LLMQ_API int llmq_gpt2_forward_all(llmq_gpt2 *m, const int64_t *tokens, int T, float *logits);
/* score_rows (gpt2t.mojo:1040-1095) on the device for window rows r0..r1-1
 * of logits[*, V] (device): stats (device, float64) receives NLL at
 * stats[r]; with base != NULL (a baseline's logits, compare mode) also
 * NLL_BASE, AGREE, KL(base || model), DIFF_MAX, DIFF_SUM at stats[k * ld + r]
 * for k = 1..5.  targets (device, int64) holds each row's target token. */
LLMQ_API int llmq_score_rows(llmq_ctx *ctx, const float *logits, const float *base, const int64_t *targets, int r0,
                             int r1, int V, double *stats, int64_t ld);
/* Device pointer to the model's logits [V] (after forward / generate). */
LLMQ_API int llmq_gpt2_logits_device(llmq_gpt2 *m, float **dptr);

/* Saved models (--save / --weights, gpt2t.mojo:612-698), in serialize.mojo's
 * encoding and byte for byte the reference's file: save_model (630-650),
 * load_saved (668-698) with the cache chosen as in llmq_gpt2_create_ex, and
 * saved_formats (661-666), which copies the layer and head format names
 * (e.g. "int4-g32-a16", "int8-ch-a16") into buffers of cap bytes.  The
 * device model loads QuantMatrix layers with the int8 per-channel head
 * (HEAD8 / HEAD8_A16 as the layers) or the layers' own format as head
 * (main's --weights, 1298-1303); other files return LLMQ_EUNSUPPORTED. */
LLMQ_API int llmq_gpt2_save(llmq_gpt2 *m, const char *path);
LLMQ_API int llmq_gpt2_load(llmq_ctx *ctx, const char *path, int attention, llmq_gpt2 **out);
LLMQ_API int llmq_saved_formats(const char *path, char *layers, char *head, int cap);
/* load_gguf (gpt2t.mojo:728-760): GPT-2 124M from a llama.cpp GGUF file,
 * its matrices used as stored (GGUF names of gpt2t.mojo:702-718; the head is
 * output.weight, or token_embd.weight when absent; position_embd and the
 * norms / biases F32).  Layers run the GGUF kernels on float activations,
 * the head head_i16 for Q6_K / Q8_0; forward and generate as for
 * llmq_gpt2_create's model (generate's greedy pick is made on the host). */
LLMQ_API int llmq_gpt2_load_gguf(llmq_ctx *ctx, const char *path, int attention, llmq_gpt2 **out);

/* ---------------------------------------------------------------- config 4
 * A TinyLlama-shaped decoder over GGUF weights (the benchmark's fifth
 * configuration: RMSNorm, RoPE, grouped key / value heads, SwiGLU).  No counterpart in the reference,
 * whose model code is GPT-2 only (gpt2t.mojo:74-81); it composes the GGUF
 * kernels above (GGUFMatrix, gguf.mojo:344-511; matmul_rows and head_i16,
 * kernels.mojo:285-349, 693-736) with the int8 cache (QuantKV[8],
 * kvcache.mojo:248-385). */
typedef struct llmq_llama llmq_llama;
typedef struct {
    int n_layer, dim, n_head, n_kv, head_dim, ffn, vocab, max_t, batch;
    int layer_type, head_type, embd_type; /* ggml type ids of the layer, output and embedding matrices */
    float eps, theta;                     /* RMSNorm epsilon, RoPE base */
} llmq_llama_cfg;
/* tensors: 2 + 9 n_layer host pointers: token_embd [vocab][dim]; per layer
 * attn_norm (float32 [dim]), attn_q [dim][dim], attn_k [n_kv*64][dim],
 * attn_v [n_kv*64][dim], attn_output [dim][dim], ffn_norm (float32 [dim]),
 * ffn_gate [ffn][dim], ffn_up [ffn][dim], ffn_down [dim][ffn]; output_norm
 * (float32 [dim]); output [vocab][dim].  Matrices are GGUF blocks as stored,
 * [rows = outputs][row bytes]; batch sequences get their own cache. */
LLMQ_API int llmq_llama_create(llmq_ctx *ctx, const llmq_llama_cfg *cfg, const void *const *tensors,
                               llmq_llama **out);
LLMQ_API int llmq_llama_free(llmq_llama *m);
LLMQ_API int64_t llmq_llama_weight_bytes(const llmq_llama *m);
/* T tokens of sequence seq at positions pos0.. (cache written); logits of the
 * last token to a host buffer of vocab floats (may be null). */
LLMQ_API int llmq_llama_forward(llmq_llama *m, int seq, const int64_t *tokens, int T, int pos0, float *logits);
/* Prompts [batch][n_prompt] (batch <= cfg.batch) from position 0, then
 * `steps` greedy tokens per sequence (the first from the prompt, then
 * steps - 1 batched decode steps replayed from one captured graph);
 * out_tokens [steps][batch]. */
LLMQ_API int llmq_llama_generate(llmq_llama *m, const int64_t *prompts, int batch, int n_prompt, int steps,
                                 int64_t *out_tokens, double *prefill_ms, double *decode_ms);

#ifdef __cplusplus
}
#endif
#endif /* LLMQ_H */
