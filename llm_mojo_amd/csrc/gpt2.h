// GPT-2 124M model state shared by the model code (api.hip) and its saved
// files (model_io.hip).  Shapes are gpt2t.mojo's compile-time constants
// (74-81) and the small float tensors follow Model.small's order
// (gpt2t.mojo:108-119, 574-576).
#pragma once
#include <string>

#include "common.h"

namespace {
constexpr int kFuseFrom = 256;  // positions from which decode uses the fused qkv + attention kernel
constexpr int NL = 12, NH = 12, C = 768, HS = 64, MAXT = 1024, V = 50257, EOT = 50256;
enum { LN1_W, LN1_B, QKV_B, PROJ_B, LN2_W, LN2_B, FC_B, FCPROJ_B, N_VECS };
constexpr int VEC_LEN[N_VECS] = {C, C, 3 * C, C, C, C, 4 * C, C};
constexpr int VEC_PARAM[N_VECS] = {0, 1, 3, 5, 6, 7, 9, 11};  // index within a layer's 12 params
constexpr int64_t SMALL_FLOATS = (int64_t)NL * 13 * C + (int64_t)MAXT * C + 2 * C;  // gpt2t.mojo:576
}  // namespace

struct llmq_gpt2 {
    llmq_ctx *ctx = nullptr;
    llmq_mat *wte = nullptr;
    llmq_mat *mats[NL * 4] = {};
    float *small = nullptr;
    const float *vec[NL][N_VECS] = {};
    const float *wpe = nullptr, *lnf_w = nullptr, *lnf_b = nullptr;
    llmq_kv *kv = nullptr;
    float *x = nullptr, *qkv = nullptr, *att = nullptr, *fc = nullptr, *logits = nullptr;
    ArgmaxPart *parts = nullptr;
    int nparts = 0;
    int64_t *tokens = nullptr, *gen = nullptr;
    int *state = nullptr;  // {pos, step} of the device-driven decode loop
    // captured decode steps: [0] one step, [1] step_k steps
    hipGraphExec_t step_graph[2] = {};
    hipGraph_t step_graph_def[2] = {};
    int step_k = 0;
    // Model[GGUFMatrix, GGUFMatrix] (load_gguf, gpt2t.mojo:728-760): layers
    // and head as stored in a GGUF file, float activations, LayerNorm into xn
    // Decode tokens run qkv + attention as one kernel (qkv_attn.hip) past
    // kFuseFrom cached positions, where it is faster; LLMQ_DECODE_FUSION=0 / 1
    // forces two kernels / the fused one.
    int fuse_env = -1;
    int fuse_qkv_attn = 0;  // the mode the enqueued (and captured) step uses
    int gguf = 0;
    llmq_mat *lm = nullptr;  // the head when not tied to wte
    float *xn = nullptr;
    // llmq_gpt2_debug_codes: one-token forwards write each linear's int16
    // input codes here ([49][3072], slot 4 l + k, 48 the head)
    int16_t *dbg_codes = nullptr;
};

// A QuantMatrix format: QuantMatrix[bits, group (0: per channel), sym, A16].
struct QFormat {
    int bits = 0, group = 0, sym = 0, a16 = 0;
    bool operator==(const QFormat &o) const {
        return bits == o.bits && group == o.group && sym == o.sym && a16 == o.a16;
    }
};
// QuantMatrix.name() (tensor.mojo:326-331): int{4,8}-{ch,g<G>}[-sym][-a16].
std::string quant_name(const QFormat &f);
// The format a name denotes (the inverse of quant_name); false for any other
// name (model_io.hip).
bool parse_quant_name(const std::string &s, QFormat *f);
// Model[W, E] from the Hugging Face float32 tensors with layers in format w
// and the tied embedding / head in format e (run_quantized's W and E,
// gpt2t.mojo:1282-1292, 1231-1235); params as llmq_gpt2_create (api.hip).
int gpt2_create_formats(llmq_ctx *ctx, const float *const *params, const QFormat &w, const QFormat &e,
                        int attention, llmq_gpt2 **out);
// The GGUF model's forward (gpt2_gguf.hip): tokens already in m->tokens.
int gpt2g_enqueue(llmq_gpt2 *m, int T, int pos0, bool with_head = true);

// Uploads the small tensors (host, SMALL_FLOATS floats in Model.small's
// order) and allocates the cache (LLMQ_ATTN_FLOAT or LLMQ_ATTN_INT) and the
// activations of a model whose matrices are in place (api.hip).
int gpt2_finish(llmq_gpt2 *m, int attention, const float *small_host);
