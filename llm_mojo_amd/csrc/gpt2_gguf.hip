// GPT-2 124M from a llama.cpp GGUF file (load_gguf, gpt2t.mojo:728-760):
// Model[GGUFMatrix, GGUFMatrix] with the layers and head used as stored.
// GGUF layers take float activations (linear's OUT_MAJOR branch,
// kernels.mojo:817-826, and matmul_rows, 285-349), so LayerNorm writes xn
// and the GGUF GEMV (one token) or matmul (several) reads it; the head is
// head_i16 for Q6_K / Q8_0 (kernels.mojo:677-681, 693-736) and the float
// GEMV otherwise.  The embedding is GGUFMatrix.dequant_row of token_embd plus
// the position row (gpt2t.mojo:495-502).
#include <string.h>

#include <string>
#include <vector>

#include "gpt2.h"

namespace {

// GGUF names (gpt2t.mojo:702-718) in load_model's matrix order and in
// VEC_NAMES order.
const char *const kMatNames[4] = {"attn_qkv.weight", "attn_output.weight", "ffn_up.weight", "ffn_down.weight"};
const char *const kVecNames[N_VECS] = {"attn_norm.weight", "attn_norm.bias", "attn_qkv.bias", "attn_output.bias",
                                       "ffn_norm.weight",  "ffn_norm.bias",  "ffn_up.bias",   "ffn_down.bias"};

__global__ void add_rows_kernel(float *__restrict__ x, const float *__restrict__ add, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + add[i];
}

int linear(llmq_gpt2 *m, const llmq_mat *w, const float *x, int T, float *out, const float *bias, int flags) {
    if (T == 1) return launch_gguf_gemv(m->ctx, w, x, out, bias, flags, nullptr, 0);
    return launch_gguf_gemm(m->ctx, w, x, w->k, T, out, w->n, bias, flags);
}

// LayerNorm then linear: fused into the GEMV's prologue for one token,
// through xn for several.
int ln_linear(llmq_gpt2 *m, const llmq_mat *w, const float *x, const float *ln_w, const float *ln_b, int T,
              float *out, const float *bias, int flags) {
    if (T == 1)
        return launch_gguf_gemv(m->ctx, w, x, out, bias, flags, nullptr, 0, nullptr, 0.0f, 0, ln_w, ln_b);
    RC(launch_layernorm(m->ctx, m->xn, x, ln_w, ln_b, T, w->k));
    return linear(m, w, m->xn, T, out, bias, flags);
}

// A float32 tensor of the file (gguf_f32, gpt2t.mojo:721-726), n floats.
int gguf_f32(const llmq_gguf *g, const std::string &name, int64_t n, float *dst) {
    int64_t i;
    RC(llmq_gguf_find(g, name.c_str(), &i));
    LLMQ_REQUIRE(i >= 0, "tensor not in GGUF file: %s", name.c_str());
    int type;
    int64_t rows, cols;
    RC(llmq_gguf_tensor_info(g, i, nullptr, &type, &rows, &cols, nullptr));
    LLMQ_REQUIRE(type == LLMQ_GGML_F32, "%s is ggml type %d, expected F32", name.c_str(), type);
    LLMQ_REQUIRE(rows * cols == n, "%s has %lld values, expected %lld", name.c_str(), (long long)(rows * cols),
                 (long long)n);
    const void *p;
    RC(llmq_gguf_tensor_data(g, i, &p, nullptr));
    memcpy(dst, p, sizeof(float) * (size_t)n);
    return LLMQ_OK;
}

int gguf_mat(llmq_ctx *ctx, const llmq_gguf *g, const std::string &name, int64_t rows, int64_t cols,
             llmq_mat **out) {
    RC(llmq_gguf_matrix(ctx, g, name.c_str(), out));
    if ((*out)->n != rows || (*out)->k != cols)
        return llmq_set_error(LLMQ_EINVAL, "%s has an unexpected shape", name.c_str());
    return LLMQ_OK;
}

struct GgufCloser {
    llmq_gguf *g;
    ~GgufCloser() { llmq_gguf_close(g); }
};

}  // namespace

// Model.blocks and the head (gpt2t.mojo:329-342, 485-571) for the T tokens in
// m->tokens at positions pos0..
int gpt2g_enqueue(llmq_gpt2 *m, int T, int pos0, bool with_head) {
    llmq_ctx *ctx = m->ctx;
    RC(launch_gguf_dequant_rows(ctx, m->wte, m->tokens, T, m->x, C));
    const int64_t n = (int64_t)T * C;
    hipLaunchKernelGGL(add_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, m->x,
                       m->wpe + (int64_t)pos0 * C, n);
    LLMQ_HIP(hipGetLastError());
    for (int l = 0; l < NL; l++) {
        llmq_mat **w = &m->mats[l * 4];
        const float *const *v = m->vec[l];
        RC(ln_linear(m, w[0], m->x, v[LN1_W], v[LN1_B], T, m->qkv, v[QKV_B], LLMQ_BIAS));
        if (T > 1) RC(launch_kv_store(ctx, m->kv, l, pos0, nullptr, m->qkv, T, 3 * C));
        RC(launch_kv_attend(ctx, m->kv, m->att, m->qkv, l, T, pos0, nullptr, 3 * C, T == 1));
        RC(linear(m, w[1], m->att, T, m->x, v[PROJ_B], LLMQ_BIAS | LLMQ_RESID));
        RC(ln_linear(m, w[2], m->x, v[LN2_W], v[LN2_B], T, m->fc, v[FC_B], LLMQ_BIAS | LLMQ_GELU));
        RC(linear(m, w[3], m->fc, T, m->x, v[FCPROJ_B], LLMQ_BIAS | LLMQ_RESID));
    }
    if (!with_head) return LLMQ_OK;
    // LN_f on the last row, then the head (gpt2t.mojo:337-340)
    const float *last = m->x + (int64_t)(T - 1) * C;
    if (!gguf_has_i16(m->lm)) return ln_linear(m, m->lm, last, m->lnf_w, m->lnf_b, 1, m->logits, nullptr, 0);
    RC(launch_layernorm(ctx, m->xn, last, m->lnf_w, m->lnf_b, 1, C));
    return launch_gguf_head16(ctx, m->lm, m->xn, m->logits, 1);
}

extern "C" int llmq_gpt2_load_gguf(llmq_ctx *ctx, const char *path, int attention, llmq_gpt2 **out) {
    LLMQ_REQUIRE(ctx && path && out, "gpt2_load_gguf: bad arguments");
    LLMQ_REQUIRE(attention == LLMQ_ATTN_FLOAT || attention == LLMQ_ATTN_INT, "gpt2_load_gguf: attention %d",
                 attention);
    llmq_gguf *g = nullptr;
    RC(llmq_gguf_open(path, &g));
    GgufCloser gc{g};
    llmq_gpt2 *m = new llmq_gpt2();
    m->ctx = ctx;
    m->gguf = 1;
    int rc = gguf_mat(ctx, g, "token_embd.weight", V, C, &m->wte);
    int64_t out_idx = -1;
    if (rc == LLMQ_OK) rc = llmq_gguf_find(g, "output.weight", &out_idx);
    if (rc == LLMQ_OK) {
        if (out_idx < 0)
            m->lm = m->wte;  // tied (gpt2t.mojo:736-737)
        else
            rc = gguf_mat(ctx, g, "output.weight", V, C, &m->lm);
    }
    static const int64_t rows[4] = {3 * C, C, 4 * C, C}, cols[4] = {C, C, C, 4 * C};  // GGUF: [OUT, IN]
    std::vector<float> small((size_t)SMALL_FLOATS);
    int64_t off = 0;
    for (int l = 0; rc == LLMQ_OK && l < NL; l++) {
        const std::string prefix = "blk." + std::to_string(l) + ".";
        for (int j = 0; rc == LLMQ_OK && j < 4; j++)
            rc = gguf_mat(ctx, g, prefix + kMatNames[j], rows[j], cols[j], &m->mats[l * 4 + j]);
        for (int s = 0; rc == LLMQ_OK && s < N_VECS; s++) {
            rc = gguf_f32(g, prefix + kVecNames[s], VEC_LEN[s], small.data() + off);
            off += VEC_LEN[s];
        }
    }
    if (rc == LLMQ_OK) rc = gguf_f32(g, "position_embd.weight", (int64_t)MAXT * C, small.data() + off);
    off += (int64_t)MAXT * C;
    if (rc == LLMQ_OK) rc = gguf_f32(g, "output_norm.weight", C, small.data() + off);
    if (rc == LLMQ_OK) rc = gguf_f32(g, "output_norm.bias", C, small.data() + off + C);
    if (rc == LLMQ_OK) rc = gpt2_finish(m, attention, small.data());
    if (rc != LLMQ_OK) {
        llmq_gpt2_free(m);
        return rc;
    }
    *out = m;
    return LLMQ_OK;
}
