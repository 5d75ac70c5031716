// Weight quantization into the row-tile layout, and int16 activation
// quantization.
#include "common.h"

namespace {

__device__ __forceinline__ int clamp_code(int u, int levels) { return u < 0 ? 0 : (u > levels ? levels : u); }

// QuantMatrix.from_f32 (tensor.mojo:334-383), one thread per (row, group):
// the group's range widened to include 0, the float32 scale rounded to
// float16 (RNE) and back, then zero point and codes against that scale.
// Thread index runs over rows fastest, so with reduce_rows (Hugging Face
// [IN, OUT] source) neighbouring threads read neighbouring floats.
__global__ __launch_bounds__(256) void quant_weights_kernel(const float *__restrict__ src, int64_t cols,
                                                            int reduce_rows, int bits, int64_t G, int sym, int64_t n,
                                                            int64_t CK, int64_t NG, uint8_t *__restrict__ codes,
                                                            uint16_t *__restrict__ scales, uint8_t *__restrict__ zps) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n * NG) return;
    const int64_t o = idx % n, g = idx / n;
    auto at = [&](int64_t kk) -> float { return reduce_rows ? src[kk * cols + o] : src[o * cols + kk]; };
    float lo = 0.0f, hi = 0.0f;
    for (int64_t j = 0; j < G; j++) {
        float v = at(g * G + j);
        lo = v < lo ? v : lo;
        hi = v > hi ? v : hi;
    }
    const int levels = (1 << bits) - 1, half = 1 << (bits - 1);
    float s;
    if (sym) {
        float a = -lo > hi ? -lo : hi;
        s = a / (float)(half - 1);
    } else {
        s = (hi - lo) / (float)levels;
    }
    if (s == 0.0f) s = 1.0f;
    const __half s16 = __float2half_rn(s);
    const float sf = __half2float(s16);
    const int zp = sym ? half : clamp_code(llmq_to_int(roundf(-lo / sf)), levels);
    const int64_t tile = o / LLMQ_TILE_ROWS, r = o % LLMQ_TILE_ROWS;
    scales[(tile * NG + g) * LLMQ_TILE_ROWS + r] = __half_as_ushort(s16);
    zps[(tile * NG + g) * LLMQ_TILE_ROWS + r] = (uint8_t)zp;
    const int wpc = bits == 4 ? 32 : 16;  // weights per 16-byte chunk
    const int64_t cpg = G / wpc;
    for (int64_t cc = 0; cc < cpg; cc++) {
        const int64_t c = g * cpg + cc;
        uint32_t dw[4] = {0, 0, 0, 0};
        for (int w = 0; w < wpc; w++) {
            float v = at(c * wpc + w);
            int u = clamp_code(llmq_to_int(roundf(v / sf)) + zp, levels);
            if (bits == 4)
                dw[w >> 3] |= (uint32_t)u << (4 * (w & 7));
            else
                dw[w >> 2] |= (uint32_t)u << (8 * (w & 3));
        }
        reinterpret_cast<uint4 *>(codes)[(tile * CK + c) * LLMQ_TILE_ROWS + r] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    }
}

// kernels.quantize_rows (kernels.mojo:400-416): one workgroup per row.
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float *__restrict__ x, int64_t K,
                                                            int16_t *__restrict__ xq, float *__restrict__ sx) {
    __shared__ float red[4];
    const float *row = x + (int64_t)blockIdx.x * K;
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < K; i += blockDim.x) m = fmaxf(m, fabsf(row[i]));
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float s = m / 32767.0f;
    if (s == 0.0f) s = 1.0f;
    const float inv = 1.0f / s;
    if (threadIdx.x == 0) sx[blockIdx.x] = s;
    for (int64_t i = threadIdx.x; i < K; i += blockDim.x)
        xq[(int64_t)blockIdx.x * K + i] = (int16_t)llmq_to_int(roundf(row[i] * inv));
}

}  // namespace

int launch_quant_weights(llmq_ctx *ctx, llmq_mat *m, const float *dsrc, int64_t rows, int64_t cols,
                         int reduce_rows) {
    (void)rows;
    const int64_t total = m->n * m->NG;
    const int threads = 256;
    const int64_t blocks = (total + threads - 1) / threads;
    hipLaunchKernelGGL(quant_weights_kernel, dim3((unsigned)blocks), dim3(threads), 0, ctx->stream, dsrc, cols,
                       reduce_rows, m->bits, m->group, m->sym, m->n, m->CK, m->NG, m->codes, m->scales, m->zps);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int launch_quantize_rows(llmq_ctx *ctx, const float *x, int64_t T, int64_t K, int16_t *xq, float *sx) {
    LLMQ_REQUIRE(T > 0 && K > 0, "quantize_rows: bad shape T=%lld K=%lld", (long long)T, (long long)K);
    hipLaunchKernelGGL(quantize_rows_kernel, dim3((unsigned)T), dim3(256), 0, ctx->stream, x, K, xq, sx);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}
