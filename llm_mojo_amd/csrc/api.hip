// The C ABI of libllmq.so (include/llmq.h): contexts, weight-format handles,
// the int8 KV cache, the compute entry points and the GPT-2 caller.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <mutex>
#include <vector>

#include "common.h"
#include "gpt2.h"

static thread_local char g_err[512];

// The scratch of llmq_linear_noalloc: the prompt GEMM's int16 activation
// codes (256-byte aligned) and per-row scales, which llmq_linear keeps in the
// context's grow-only workspace.  Each GPU the library runs on holds its own
// copy for the life of the process.  The array's name is a host-side stand-in
// (never passed to a kernel): host code uses the device address that
// hipGetSymbolAddress returns, looked up once per device by llmq_init.
static __device__ __align__(256) uint8_t scratch[LLMQ_NOALLOC_SCRATCH_BYTES];

static int scratch_address(int device, void **p) {
    static std::mutex mu;
    static void *addr[64] = {};
    LLMQ_REQUIRE(device >= 0 && device < 64, "llmq_init: device %d beyond 64", device);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {  // with `device` current
        void *a = nullptr;
        const hipError_t e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !a)
            return llmq_set_error(LLMQ_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        addr[device] = a;
    }
    *p = addr[device];
    return LLMQ_OK;
}

int llmq_set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}


int ctx_workspace(llmq_ctx *ctx, size_t bytes, void **p, int slot) {
    if (bytes > ctx->ws_bytes[slot]) {
        LLMQ_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->ws[slot]) hipFree(ctx->ws[slot]);
        ctx->ws[slot] = nullptr;
        ctx->ws_bytes[slot] = 0;
        const size_t want = bytes + bytes / 4;
        if (hipMalloc(&ctx->ws[slot], want) != hipSuccess)
            return llmq_set_error(LLMQ_ENOMEM, "workspace of %zu bytes", want);
        ctx->ws_bytes[slot] = want;
    }
    *p = ctx->ws[slot];
    return LLMQ_OK;
}

extern "C" {

const char *llmq_last_error(void) { return g_err; }

int llmq_init(int device, llmq_ctx **out) {
    LLMQ_REQUIRE(out, "llmq_init: null output");
    int n = 0;
    LLMQ_HIP(hipGetDeviceCount(&n));
    LLMQ_REQUIRE(device >= 0 && device < n, "llmq_init: device %d of %d", device, n);
    LLMQ_HIP(hipSetDevice(device));
    llmq_ctx *c = new llmq_ctx();
    c->device = device;
    // A blocking stream: ordered with work on the null stream, which is where
    // frameworks without an explicit stream put their copies.
    hipError_t e = hipStreamCreateWithFlags(&c->own_stream, hipStreamDefault);
    if (e != hipSuccess) {
        delete c;
        return llmq_set_error(LLMQ_EHIP, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    c->stream = c->own_stream;
    int rc = LLMQ_OK;
    e = hipGetDeviceProperties(&c->prop, device);
    if (e != hipSuccess) rc = llmq_set_error(LLMQ_EHIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    if (rc == LLMQ_OK) rc = scratch_address(device, &c->scratch);
    if (rc != LLMQ_OK) {
        hipStreamDestroy(c->own_stream);
        delete c;
        return rc;
    }
    *out = c;
    return LLMQ_OK;
}

int llmq_destroy(llmq_ctx *ctx) {
    if (!ctx) return LLMQ_OK;
    hipStreamSynchronize(ctx->stream);
    for (void *p : ctx->ws)
        if (p) hipFree(p);
    if (ctx->own_stream) hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return LLMQ_OK;
}

int llmq_set_stream(llmq_ctx *ctx, void *s) {
    LLMQ_REQUIRE(ctx, "set_stream: null context");
    ctx->stream = s ? (hipStream_t)s : ctx->own_stream;
    return LLMQ_OK;
}

int llmq_sync(llmq_ctx *ctx) {
    LLMQ_REQUIRE(ctx, "sync: null context");
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

int llmq_malloc(llmq_ctx *ctx, size_t bytes, void **p) {
    LLMQ_REQUIRE(ctx && p, "malloc: bad arguments");
    if (hipMalloc(p, bytes ? bytes : 1) != hipSuccess) return llmq_set_error(LLMQ_ENOMEM, "hipMalloc(%zu) failed", bytes);
    return LLMQ_OK;
}

int llmq_free(llmq_ctx *ctx, void *p) {
    (void)ctx;
    if (p) LLMQ_HIP(hipFree(p));
    return LLMQ_OK;
}

int llmq_memcpy_h2d(llmq_ctx *ctx, void *dst, const void *src, size_t bytes) {
    LLMQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

int llmq_memcpy_d2h(llmq_ctx *ctx, void *dst, const void *src, size_t bytes) {
    LLMQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

// ------------------------------------------------------------ weight formats

// The shapes QuantMatrix storage accepts (n output rows, k inputs).
static int quant_shape_ok(int bits, int group, int a16, int64_t n, int64_t k) {
    LLMQ_REQUIRE(bits == 4 || bits == 8, "from_f32: BITS must be 4 or 8");
    LLMQ_REQUIRE(n > 0 && k > 0, "from_f32: empty matrix");
    const int64_t g = group == 0 ? k : group;
    // tensor.mojo:340-341
    LLMQ_REQUIRE(g > 0 && k % g == 0 && g % 32 == 0,
                 "group size must divide the reduction axis and be a multiple of 32");
    // The BLOCKED layout of int4-g32-a16 (tensor.mojo:296, 394-404) places
    // codes per 256-weight block; the reference has no layout for a partial
    // block (its nibble_at addresses past the row), so such matrices are
    // refused rather than exported wrongly.
    LLMQ_REQUIRE(!(a16 && bits == 4 && g == 32 && k % 256 != 0),
                 "int4-g32-a16 (BLOCKED layout) needs the reduction axis in whole 256-weight blocks, got %lld",
                 (long long)k);
    {   // every kernel addresses one array with 32-bit buffer offsets (0x80000000 = a disabled load)
        const int64_t nt = (n + LLMQ_TILE_ROWS - 1) / LLMQ_TILE_ROWS;
        const int64_t cb = (nt * (k * bits / 8 / 16) + LLMQ_PAD_CHUNKS) * 256,
                      sb = (nt * (k / g) + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS * 2;
        LLMQ_REQUIRE(cb < (int64_t)kLlmqOOB && sb < (int64_t)kLlmqOOB,
                     "from_f32: %lld x %lld matrix: code array of %lld bytes reaches the 2 GiB limit",
                     (long long)n, (long long)k, (long long)cb);
    }
    return LLMQ_OK;
}

static int mat_alloc_quant(llmq_ctx *ctx, int bits, int group, int sym, int a16, int64_t n, int64_t k,
                           llmq_mat **out) {
    RC(quant_shape_ok(bits, group, a16, n, k));
    const int64_t g = group == 0 ? k : group;
    llmq_mat *m = new llmq_mat();
    m->ctx = ctx;
    m->kind = MAT_QUANT;
    m->bits = bits;
    m->group_param = group;
    m->sym = sym ? 1 : 0;
    m->a16 = a16 ? 1 : 0;
    m->n = n;
    m->k = k;
    m->group = g;
    m->ntiles = (n + LLMQ_TILE_ROWS - 1) / LLMQ_TILE_ROWS;
    m->CK = k * bits / 8 / 16;
    m->NG = k / g;
    // Readable padding after codes, scales and zero points: the GEMV reads up
    // to LLMQ_PAD_CHUNKS chunks (and their groups) past a tile's end instead
    // of branching around the loads.
    const size_t cb = (size_t)(m->ntiles * m->CK + LLMQ_PAD_CHUNKS) * 256,
                 gb = (size_t)(m->ntiles * m->NG + LLMQ_PAD_CHUNKS) * LLMQ_TILE_ROWS;
    if (hipMalloc(&m->codes, cb) != hipSuccess || hipMalloc(&m->scales, gb * 2) != hipSuccess ||
        hipMalloc(&m->zps, gb) != hipSuccess) {
        hipFree(m->codes);
        hipFree(m->scales);
        hipFree(m->zps);
        delete m;
        return llmq_set_error(LLMQ_ENOMEM, "from_f32: device allocation of %zu bytes failed", cb + 3 * gb);
    }
    LLMQ_HIP(hipMemsetAsync(m->codes, 0, cb, ctx->stream));
    LLMQ_HIP(hipMemsetAsync(m->scales, 0, gb * 2, ctx->stream));
    LLMQ_HIP(hipMemsetAsync(m->zps, 0, gb, ctx->stream));
    *out = m;
    return LLMQ_OK;
}

int llmq_mat_from_f32_device(llmq_ctx *ctx, int bits, int group, int sym, int a16, const float *src, int64_t rows,
                             int64_t cols, int reduce_rows, llmq_mat **out) {
    LLMQ_REQUIRE(ctx && src && out, "from_f32: bad arguments");
    const int64_t n = reduce_rows ? cols : rows, k = reduce_rows ? rows : cols;
    llmq_mat *m = nullptr;
    RC(mat_alloc_quant(ctx, bits, group, sym, a16, n, k, &m));
    int rc = launch_quant_weights(ctx, m, src, rows, cols, reduce_rows);
    if (rc != LLMQ_OK) {
        llmq_mat_free(m);
        return rc;
    }
    *out = m;
    return LLMQ_OK;
}

int llmq_mat_from_f32(llmq_ctx *ctx, int bits, int group, int sym, int a16, const float *src, int64_t rows,
                      int64_t cols, int reduce_rows, llmq_mat **out) {
    LLMQ_REQUIRE(ctx && src && out, "from_f32: bad arguments");
    LLMQ_REQUIRE(rows > 0 && cols > 0, "from_f32: empty matrix");
    RC(quant_shape_ok(bits, group, a16, reduce_rows ? cols : rows, reduce_rows ? rows : cols));
    float *d = nullptr;
    const size_t bytes = sizeof(float) * (size_t)rows * cols;
    if (hipMalloc(&d, bytes) != hipSuccess) return llmq_set_error(LLMQ_ENOMEM, "from_f32: staging %zu bytes", bytes);
    int rc = LLMQ_OK;
    if (hipMemcpyAsync(d, src, bytes, hipMemcpyHostToDevice, ctx->stream) != hipSuccess)
        rc = llmq_set_error(LLMQ_EHIP, "from_f32: copy to device failed");
    if (rc == LLMQ_OK) rc = llmq_mat_from_f32_device(ctx, bits, group, sym, a16, d, rows, cols, reduce_rows, out);
    hipStreamSynchronize(ctx->stream);
    hipFree(d);
    return rc;
}

int llmq_mat_free(llmq_mat *m) {
    if (!m) return LLMQ_OK;
    if (m->ctx) hipStreamSynchronize(m->ctx->stream);
    hipFree(m->codes);
    hipFree(m->scales);
    hipFree(m->zps);
    hipFree(m->blocks);
    hipFree(m->g_meta16);
    hipFree(m->g_meta32);
    hipFree(m->g_bits32);
    hipFree(m->g_bits64);
    hipFree(m->g_sb16);
    delete m;
    return LLMQ_OK;
}

int64_t llmq_mat_nbytes(const llmq_mat *m) {
    if (!m) return 0;
    if (m->kind == MAT_GGUF) return m->n * m->row_bytes;  // gguf.mojo:507-508
    return m->n * m->k * m->bits / 8 + (m->n * m->k / m->group) * 3;  // tensor.mojo:629-632
}

int64_t llmq_mat_group_size(const llmq_mat *m) {
    if (!m) return 0;
    if (m->kind == MAT_GGUF) return m->ggml_type == LLMQ_GGML_Q6_K ? 256 : 32;  // gguf.mojo:459-460
    return m->group;
}

int llmq_mat_has_i16(const llmq_mat *m) {
    if (!m) return 0;
    if (m->kind == MAT_GGUF) return gguf_has_i16(m);  // gguf.mojo:456-457
    return m->a16 ? 1 : 0;                            // tensor.mojo:102-104 (ACT16)
}

int llmq_mat_shape(const llmq_mat *m, int64_t *rows, int64_t *cols) {
    LLMQ_REQUIRE(m, "shape: null matrix");
    if (rows) *rows = m->n;
    if (cols) *cols = m->k;
    return LLMQ_OK;
}

// nibble_at (tensor.mojo:385-404): byte and nibble of column col in the
// reference layout (BLOCKED or Q4_0-style).
static inline void ref_nibble_at(bool blocked, int64_t col, int64_t *byte, int *high) {
    int64_t j, chunk;
    if (blocked) {
        const int64_t w = col % 256, e = w % 32, p = e / 2;
        const int64_t lane = w / 32 + 8 * (p / 8);
        chunk = (col / 256) * 8 + p % 8;
        j = 2 * lane + e % 2;
    } else {
        chunk = col / 32;
        j = col % 32;
    }
    *byte = chunk * 16 + j % 16;
    *high = j >= 16;
}

int llmq_mat_export(llmq_ctx *ctx, const llmq_mat *m, uint8_t *codes, uint16_t *scales, uint8_t *zps) {
    LLMQ_REQUIRE(ctx && m && m->kind == MAT_QUANT, "export: not a QuantMatrix");
    const size_t cb = (size_t)m->ntiles * m->CK * 256, gb = (size_t)m->ntiles * m->NG * LLMQ_TILE_ROWS;
    std::vector<uint8_t> c(cb), z(gb);
    std::vector<uint16_t> s(gb);
    LLMQ_HIP(hipMemcpyAsync(c.data(), m->codes, cb, hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipMemcpyAsync(s.data(), m->scales, gb * 2, hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipMemcpyAsync(z.data(), m->zps, gb, hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    const bool blocked = m->a16 && m->bits == 4 && m->group_param == 32;  // tensor.mojo:296
    const int wpc = m->bits == 4 ? 32 : 16;
    const int64_t row_bytes = m->k * m->bits / 8;
    if (codes) memset(codes, 0, (size_t)(m->n * row_bytes));
    for (int64_t o = 0; o < m->n; o++) {
        const int64_t tile = o / LLMQ_TILE_ROWS, r = o % LLMQ_TILE_ROWS;
        for (int64_t g = 0; g < m->NG; g++) {
            const size_t gi = (size_t)(tile * m->NG + g) * LLMQ_TILE_ROWS + r;
            if (scales) scales[o * m->NG + g] = s[gi];
            if (zps) zps[o * m->NG + g] = z[gi];
        }
        if (!codes) continue;
        uint8_t *dst = codes + o * row_bytes;
        for (int64_t kk = 0; kk < m->k; kk++) {
            const int64_t ch = kk / wpc, e = kk % wpc;
            const uint8_t *chunk = c.data() + ((tile * m->CK + ch) * LLMQ_TILE_ROWS + r) * 16;
            if (m->bits == 8) {
                dst[kk] = chunk[e];
            } else {
                const int u = (chunk[e >> 1] >> (4 * (e & 1))) & 15;
                int64_t b;
                int hi;
                ref_nibble_at(blocked, kk, &b, &hi);
                dst[b] |= (uint8_t)(hi ? u << 4 : u);
            }
        }
    }
    return LLMQ_OK;
}

int llmq_mat_restore(llmq_ctx *ctx, int bits, int group, int sym, int a16, int64_t rows, int64_t cols,
                     const uint8_t *codes, const uint16_t *scales, const uint8_t *zps, llmq_mat **out) {
    LLMQ_REQUIRE(ctx && codes && scales && zps && out, "restore: bad arguments");
    llmq_mat *m = nullptr;
    RC(mat_alloc_quant(ctx, bits, group, sym, a16, rows, cols, &m));
    // The inverse of llmq_mat_export: reference layout -> row tiles.
    const size_t cb = (size_t)m->ntiles * m->CK * 256, gb = (size_t)m->ntiles * m->NG * LLMQ_TILE_ROWS;
    std::vector<uint8_t> c(cb, 0), z(gb, 0);
    std::vector<uint16_t> sc(gb, 0);
    const bool blocked = m->a16 && m->bits == 4 && m->group_param == 32;  // tensor.mojo:296
    const int wpc = m->bits == 4 ? 32 : 16;
    const int64_t row_bytes = m->k * m->bits / 8;
    for (int64_t o = 0; o < m->n; o++) {
        const int64_t tile = o / LLMQ_TILE_ROWS, r = o % LLMQ_TILE_ROWS;
        for (int64_t g = 0; g < m->NG; g++) {
            const size_t gi = (size_t)(tile * m->NG + g) * LLMQ_TILE_ROWS + r;
            sc[gi] = scales[o * m->NG + g];
            z[gi] = zps[o * m->NG + g];
        }
        const uint8_t *src = codes + o * row_bytes;
        for (int64_t kk = 0; kk < m->k; kk++) {
            const int64_t ch = kk / wpc, e = kk % wpc;
            uint8_t *chunk = c.data() + ((tile * m->CK + ch) * LLMQ_TILE_ROWS + r) * 16;
            if (m->bits == 8) {
                chunk[e] = src[kk];
            } else {
                int64_t b;
                int hi;
                ref_nibble_at(blocked, kk, &b, &hi);
                const int u = (src[b] >> (hi ? 4 : 0)) & 15;
                chunk[e >> 1] |= (uint8_t)(u << (4 * (e & 1)));
            }
        }
    }
    int rc = LLMQ_OK;
    if (hipMemcpyAsync(m->codes, c.data(), cb, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipMemcpyAsync(m->scales, sc.data(), gb * 2, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipMemcpyAsync(m->zps, z.data(), gb, hipMemcpyHostToDevice, ctx->stream) != hipSuccess ||
        hipStreamSynchronize(ctx->stream) != hipSuccess)
        rc = llmq_set_error(LLMQ_EHIP, "restore: copy to the device failed");
    if (rc != LLMQ_OK) {
        llmq_mat_free(m);
        return rc;
    }
    *out = m;
    return LLMQ_OK;
}

int llmq_dot_row_i16(llmq_ctx *ctx, const llmq_mat *m, int64_t row, int64_t nrows, const int16_t *xq, float *out) {
    LLMQ_REQUIRE(ctx && m, "dot_row_i16: bad arguments");
    return launch_dot_row_i16(ctx, m, row, nrows, xq, out);
}

int llmq_mat_dequant_row(llmq_ctx *ctx, const llmq_mat *m, int64_t row, float *dst) {
    LLMQ_REQUIRE(ctx && m && dst, "dequant_row: bad arguments");
    LLMQ_REQUIRE(row >= 0 && row < m->n, "dequant_row: row %lld out of range", (long long)row);
    if (m->kind == MAT_GGUF) {
        float *d = nullptr;
        if (hipMalloc(&d, sizeof(float) * m->k) != hipSuccess)
            return llmq_set_error(LLMQ_ENOMEM, "dequant_row: staging");
        int rc = launch_gguf_dequant_row(ctx, m, row, d);
        if (rc == LLMQ_OK &&
            hipMemcpyAsync(dst, d, sizeof(float) * m->k, hipMemcpyDeviceToHost, ctx->stream) != hipSuccess)
            rc = llmq_set_error(LLMQ_EHIP, "dequant_row: copy failed");
        hipStreamSynchronize(ctx->stream);
        hipFree(d);
        return rc;
    }
    const int64_t tile = row / LLMQ_TILE_ROWS, r = row % LLMQ_TILE_ROWS;
    std::vector<uint8_t> c(m->CK * 16), z(m->NG);
    std::vector<uint16_t> s(m->NG);
    LLMQ_HIP(hipMemcpy2DAsync(c.data(), 16, m->codes + ((tile * m->CK) * LLMQ_TILE_ROWS + r) * 16, 256, 16, m->CK,
                              hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipMemcpy2DAsync(s.data(), 2, m->scales + (tile * m->NG) * LLMQ_TILE_ROWS + r, 32, 2, m->NG,
                              hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipMemcpy2DAsync(z.data(), 1, m->zps + (tile * m->NG) * LLMQ_TILE_ROWS + r, 16, 1, m->NG,
                              hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    const int wpc = m->bits == 4 ? 32 : 16;
    for (int64_t kk = 0; kk < m->k; kk++) {
        const uint8_t *chunk = c.data() + (kk / wpc) * 16;
        const int64_t e = kk % wpc;
        const int u = m->bits == 8 ? chunk[e] : (chunk[e >> 1] >> (4 * (e & 1))) & 15;
        const int64_t g = kk / m->group;
        // row_op (tensor.mojo:463-473): (float(u) - float(zp)) * scale
        __half h = __ushort_as_half(s[g]);
        dst[kk] = ((float)u - (float)z[g]) * __half2float(h);
    }
    return LLMQ_OK;
}

int llmq_mat_from_gguf(llmq_ctx *ctx, int ggml_type, const void *blocks, int64_t rows, int64_t cols,
                       llmq_mat **out) {
    LLMQ_REQUIRE(ctx && blocks && out, "from_gguf: bad arguments");
    if (!gguf_is_supported(ggml_type))
        return llmq_set_error(LLMQ_EUNSUPPORTED, "from_gguf: ggml type %d is not a supported block format",
                              ggml_type);
    llmq_mat *m = new llmq_mat();
    m->ctx = ctx;
    int rc = gguf_upload(ctx, m, ggml_type, static_cast<const uint8_t *>(blocks), rows, cols);
    if (rc != LLMQ_OK) {
        llmq_mat_free(m);
        return rc;
    }
    *out = m;
    return LLMQ_OK;
}

// ------------------------------------------------------------------ compute

int llmq_quantize_rows(llmq_ctx *ctx, const float *x, int64_t T, int64_t K, int16_t *xq, float *sx) {
    LLMQ_REQUIRE(ctx && x && xq && sx, "quantize_rows: bad arguments");
    return launch_quantize_rows(ctx, x, T, K, xq, sx);
}

static int check_linear(const llmq_mat *w, int64_t IN, int64_t OUT) {
    LLMQ_REQUIRE(w, "linear: null matrix");
    LLMQ_REQUIRE(w->k == IN && w->n == OUT, "linear: matrix is %lldx%lld, call says IN=%lld OUT=%lld",
                 (long long)w->n, (long long)w->k, (long long)IN, (long long)OUT);
    return LLMQ_OK;
}

int llmq_linear(llmq_ctx *ctx, float *out, const float *x, const llmq_mat *w, const float *bias, int64_t T,
                int64_t IN, int64_t OUT, int flags) {
    LLMQ_REQUIRE(ctx, "linear: null context");
    RC(check_linear(w, IN, OUT));
    if (is_float_act(w)) {
        // matmul_rows (kernels.mojo:285-349) for GGUF and for QuantMatrix
        // with A16 = False: the one-token GEMV (dot_row, tensor.mojo:431-482;
        // gguf.mojo:389-417), or the dequantize-and-multiply matmul for
        // several tokens
        if (T == 1) return launch_gguf_gemv(ctx, w, x, out, bias, flags, nullptr, 0);
        return launch_gguf_gemm(ctx, w, x, IN, T, out, OUT, bias, flags);
    }
    GemvRequest rq;
    rq.w = w;
    rq.x = x;
    rq.out = out;
    rq.bias = bias;
    rq.T = T;
    rq.flags = flags;
    return launch_gemv_a16(ctx, rq);
}

int llmq_linear_noalloc(llmq_ctx *ctx, float *out, const float *x, const llmq_mat *w, const float *bias, int64_t T,
                        int64_t IN, int64_t OUT, int flags) {
    LLMQ_REQUIRE(ctx && ctx->scratch, "linear_noalloc: null context");
    RC(check_linear(w, IN, OUT));
    LLMQ_REQUIRE(T >= 1, "linear_noalloc: T must be >= 1");
    if (is_float_act(w)) {
        // the one-token GEMV uses no scratch; several tokens of Q4_K keep
        // their fp16 activation record there (the other types use none)
        if (T == 1) return launch_gguf_gemv(ctx, w, x, out, bias, flags, nullptr, 0);
        return launch_gguf_gemm(ctx, w, x, IN, T, out, OUT, bias, flags, ctx->scratch, LLMQ_NOALLOC_SCRATCH_BYTES);
    }
    // the least the prompt GEMM keeps there: T x IN int16 codes and T float
    // scales, each rounded up to 256 bytes (int4-g32 matrices also put their
    // fp16 planes there when they fit, else take the int8-MFMA form)
    const int64_t need = ((T * IN * 2 + 255) & ~(int64_t)255) + ((T * 4 + 255) & ~(int64_t)255);
    LLMQ_REQUIRE(need <= (int64_t)LLMQ_NOALLOC_SCRATCH_BYTES,
                 "linear_noalloc: %lld tokens x %lld inputs need %lld bytes of scratch, the maximum is %d",
                 (long long)T, (long long)IN, (long long)need, LLMQ_NOALLOC_SCRATCH_BYTES);
    GemvRequest rq;
    rq.w = w;
    rq.x = x;
    rq.out = out;
    rq.bias = bias;
    rq.T = T;
    rq.flags = flags;
    rq.ws = ctx->scratch;
    rq.ws_cap = LLMQ_NOALLOC_SCRATCH_BYTES;
    return launch_gemv_a16(ctx, rq);
}

int llmq_ln_linear(llmq_ctx *ctx, float *out, const float *x, const float *ln_w, const float *ln_b, const llmq_mat *w,
                   const float *bias, int64_t T, int64_t IN, int64_t OUT, int flags) {
    LLMQ_REQUIRE(ctx && ln_w && ln_b, "ln_linear: bad arguments");
    RC(check_linear(w, IN, OUT));
    LLMQ_REQUIRE(w->kind == MAT_QUANT, "ln_linear: GGUF matrices take llmq_layernorm then llmq_linear");
    if (!w->a16) {
        // float activations: one token with the LayerNorm fused into the
        // GEMV; several through the context's workspace, then matmul_rows
        // (not for use under graph capture, as the workspace)
        if (T == 1) return launch_gguf_gemv(ctx, w, x, out, bias, flags, nullptr, 0, nullptr, 0.0f, 0, ln_w, ln_b);
        void *ws = nullptr;
        RC(ctx_workspace(ctx, sizeof(float) * (size_t)(T * IN), &ws));
        float *xn = static_cast<float *>(ws);
        RC(launch_layernorm(ctx, xn, x, ln_w, ln_b, T, IN));
        return llmq_linear(ctx, out, xn, w, bias, T, IN, OUT, flags);
    }
    GemvRequest rq;
    rq.w = w;
    rq.x = x;
    rq.ln_w = ln_w;
    rq.ln_b = ln_b;
    rq.out = out;
    rq.bias = bias;
    rq.T = T;
    rq.flags = flags;
    return launch_gemv_a16(ctx, rq);
}

int llmq_head(llmq_ctx *ctx, float *logits, const float *h, const llmq_mat *w, int64_t T, int64_t V, int64_t C) {
    LLMQ_REQUIRE(ctx, "head: null context");
    if (gguf_has_i16(w)) {  // kernels.mojo:677-681: GGUF heads with an int16 kernel take head_i16
        RC(check_linear(w, C, V));
        return launch_gguf_head16(ctx, w, h, logits, T);
    }
    return llmq_linear(ctx, logits, h, w, nullptr, T, C, V, 0);
}

int64_t llmq_act_bytes(int64_t K) { return K >= 32 && K % 32 == 0 ? llmq_act_layout(K).bytes : -1; }

int llmq_act_prepare(llmq_ctx *ctx, const float *x, int64_t K, const float *ln_w, const float *ln_b, void *act) {
    LLMQ_REQUIRE(ctx, "act_prepare: null context");
    return launch_act_prepare(ctx, x, K, ln_w, ln_b, act);
}

int llmq_linear_act(llmq_ctx *ctx, float *out, const void *act, const llmq_mat *w, const float *bias, int64_t IN,
                    int64_t OUT, int flags) {
    LLMQ_REQUIRE(ctx && w, "linear_act: null argument");
    LLMQ_REQUIRE(w->k == IN && w->n == OUT, "linear_act: IN=%lld OUT=%lld but the matrix is %lldx%lld",
                 (long long)IN, (long long)OUT, (long long)w->k, (long long)w->n);
    return launch_linear_act(ctx, out, act, w, bias, flags);
}

int llmq_layernorm(llmq_ctx *ctx, float *out, const float *x, const float *w, const float *b, int64_t T, int64_t C) {
    LLMQ_REQUIRE(ctx, "layernorm: null context");
    return launch_layernorm(ctx, out, x, w, b, T, C);
}

}  // extern "C"

namespace {
// Streams `n16` 16-byte words with eight 128-bit loads in flight per thread
// and folds them with XOR into one word per workgroup: the memory system's
// read rate with no arithmetic to hide (bench.py's read floor).
__global__ __launch_bounds__(256) void read_kernel(const uint4 *__restrict__ p, int64_t n16,
                                                   uint32_t *__restrict__ out) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t lo = (int64_t)blockIdx.x * per, hi = lo + per < n16 ? lo + per : n16;
    uint32_t acc = 0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256 * 8) {
        uint4 v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = i + 256 * k < hi ? p[i + 256 * k] : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < 8; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

__global__ void refmath_kernel(int op, const float *__restrict__ x, float *__restrict__ y, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    y[i] = op == 0 ? ref_expf(v) : (op == 1 ? ref_tanhf(v) : gelu_ref(v));
}
}  // namespace

extern "C" {

int llmq_debug_read(llmq_ctx *ctx, const void *buf, int64_t bytes, uint32_t *out, int grid) {
    LLMQ_REQUIRE(ctx && buf && out && bytes > 0 && bytes % 16 == 0 && grid >= 1 && grid <= (1 << 20),
                 "debug_read: bad arguments");
    hipLaunchKernelGGL(read_kernel, dim3((unsigned)grid), dim3(256), 0, ctx->stream,
                       static_cast<const uint4 *>(buf), bytes / 16, out);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int llmq_debug_refmath(llmq_ctx *ctx, int op, const float *x, float *y, int64_t n) {
    LLMQ_REQUIRE(ctx && x && y && n >= 0 && op >= 0 && op <= 2, "debug_refmath: bad arguments");
    if (n == 0) return LLMQ_OK;
    hipLaunchKernelGGL(refmath_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, op, x, y, n);
    LLMQ_HIP(hipGetLastError());
    return LLMQ_OK;
}

int llmq_debug_chunk_sums(llmq_ctx *ctx, const float *xf, const llmq_mat *w, float *out, int32_t *chunk_sums,
                          int16_t *xq, float *sx) {
    LLMQ_REQUIRE(ctx && w, "debug_chunk_sums: bad arguments");
    RC(check_linear(w, w->k, w->n));
    LLMQ_REQUIRE(w->kind == MAT_QUANT && w->a16, "debug_chunk_sums: integer-activation QuantMatrix (A16) only");
    GemvRequest rq;
    rq.w = w;
    rq.x = xf;
    rq.out = out;
    rq.T = 1;
    rq.flags = 0;
    rq.dbg = chunk_sums;
    rq.xq_out = xq;
    rq.sx_out = sx;
    return launch_gemv_a16(ctx, rq);
}

// ------------------------------------------------------------- int8 KV cache

static int kv_alloc(llmq_ctx *ctx, int n_layer, int max_t, int n_head, int head_dim, int integer, llmq_kv **out) {
    llmq_kv *kv = new llmq_kv();
    kv->ctx = ctx;
    kv->n_layer = n_layer;
    kv->max_t = max_t;
    kv->n_head = n_head;
    kv->head_dim = head_dim;
    kv->integer = integer;
    const size_t n = (size_t)n_layer * max_t * n_head * head_dim, ns = (size_t)n_layer * max_t * n_head;
    void **ks = integer ? reinterpret_cast<void **>(&kv->kq) : reinterpret_cast<void **>(&kv->ks);
    void **vs = integer ? reinterpret_cast<void **>(&kv->vq) : reinterpret_cast<void **>(&kv->vs);
    if (hipMalloc(&kv->k, n) != hipSuccess || hipMalloc(&kv->v, n) != hipSuccess ||
        hipMalloc(ks, ns * 4) != hipSuccess || hipMalloc(vs, ns * 4) != hipSuccess) {
        llmq_kv_free(kv);
        return llmq_set_error(LLMQ_ENOMEM, "kv_create: allocation failed");
    }
    LLMQ_HIP(hipMemsetAsync(kv->k, 0, n, ctx->stream));
    LLMQ_HIP(hipMemsetAsync(kv->v, 0, n, ctx->stream));
    LLMQ_HIP(hipMemsetAsync(*ks, 0, ns * 4, ctx->stream));
    LLMQ_HIP(hipMemsetAsync(*vs, 0, ns * 4, ctx->stream));
    *out = kv;
    return LLMQ_OK;
}

int llmq_kv_create(llmq_ctx *ctx, int n_layer, int max_t, int n_head, int head_dim, llmq_kv **out) {
    LLMQ_REQUIRE(ctx && out && n_layer > 0 && max_t > 0 && n_head > 0 && head_dim > 0, "kv_create: bad arguments");
    LLMQ_REQUIRE(head_dim % 64 == 0 || head_dim == 16 || head_dim == 32, "kv_create: head_dim %d unsupported",
                 head_dim);
    return kv_alloc(ctx, n_layer, max_t, n_head, head_dim, 0, out);
}

int llmq_ikv_create(llmq_ctx *ctx, int n_layer, int max_t, int n_head, int head_dim, llmq_kv **out) {
    LLMQ_REQUIRE(ctx && out && n_layer > 0 && max_t > 0 && n_head > 0 && head_dim > 0, "ikv_create: bad arguments");
    // IntAttnKV.create's shape check (int_attention.mojo:100-101, 283-284)
    LLMQ_REQUIRE(max_t % 16 == 0 && head_dim % 32 == 0, "IntAttnKV needs max_t %% 16 == 0 and head_dim %% 32 == 0");
    if (head_dim != 64 && head_dim != 128)
        return llmq_set_error(LLMQ_EUNSUPPORTED, "ikv_create: head_dim %d (64 or 128)", head_dim);
    return kv_alloc(ctx, n_layer, max_t, n_head, head_dim, 1, out);
}

int llmq_kv_is_integer(const llmq_kv *kv) { return kv ? kv->integer : 0; }

int llmq_kv_free(llmq_kv *kv) {
    if (!kv) return LLMQ_OK;
    if (kv->ctx) hipStreamSynchronize(kv->ctx->stream);
    hipFree(kv->k);
    hipFree(kv->v);
    hipFree(kv->ks);
    hipFree(kv->vs);
    hipFree(kv->kq);
    hipFree(kv->vq);
    delete kv;
    return LLMQ_OK;
}

int64_t llmq_kv_nbytes(const llmq_kv *kv) {
    if (!kv) return 0;
    const int64_t n = (int64_t)kv->n_layer * kv->max_t * kv->n_head;
    return 2 * n * (kv->head_dim + 4);  // kvcache.mojo:377-379 with BITS = 8
}

int llmq_kv_store(llmq_ctx *ctx, llmq_kv *kv, int layer, int pos0, const float *qkv, int T) {
    LLMQ_REQUIRE(ctx, "kv_store: null context");
    return launch_kv_store(ctx, kv, layer, pos0, nullptr, qkv, T, 0);
}

int llmq_kv_attend(llmq_ctx *ctx, const llmq_kv *kv, float *out, const float *qkv, int layer, int T, int pos0) {
    LLMQ_REQUIRE(ctx, "kv_attend: null context");
    return launch_kv_attend(ctx, kv, out, qkv, layer, T, pos0, nullptr, 0, false);
}

int llmq_kv_export(llmq_ctx *ctx, const llmq_kv *kv, int8_t *k, int8_t *v, float *ks, float *vs) {
    LLMQ_REQUIRE(ctx && kv, "kv_export: bad arguments");
    LLMQ_REQUIRE(!kv->integer, "kv_export: an IntAttnKV cache holds integer scales (llmq_ikv_export)");
    const size_t n = (size_t)kv->n_layer * kv->max_t * kv->n_head * kv->head_dim,
                 ns = (size_t)kv->n_layer * kv->max_t * kv->n_head;
    if (k) LLMQ_HIP(hipMemcpyAsync(k, kv->k, n, hipMemcpyDeviceToHost, ctx->stream));
    if (v) LLMQ_HIP(hipMemcpyAsync(v, kv->v, n, hipMemcpyDeviceToHost, ctx->stream));
    if (ks) LLMQ_HIP(hipMemcpyAsync(ks, kv->ks, ns * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (vs) LLMQ_HIP(hipMemcpyAsync(vs, kv->vs, ns * 4, hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

int llmq_ikv_export(llmq_ctx *ctx, const llmq_kv *kv, int8_t *k, int8_t *v, int32_t *kq, int32_t *vq) {
    LLMQ_REQUIRE(ctx && kv, "ikv_export: bad arguments");
    LLMQ_REQUIRE(kv->integer, "ikv_export: not an IntAttnKV cache (llmq_kv_export)");
    const size_t n = (size_t)kv->n_layer * kv->max_t * kv->n_head * kv->head_dim,
                 ns = (size_t)kv->n_layer * kv->max_t * kv->n_head;
    if (k) LLMQ_HIP(hipMemcpyAsync(k, kv->k, n, hipMemcpyDeviceToHost, ctx->stream));
    if (v) LLMQ_HIP(hipMemcpyAsync(v, kv->v, n, hipMemcpyDeviceToHost, ctx->stream));
    if (kq) LLMQ_HIP(hipMemcpyAsync(kq, kv->kq, ns * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (vq) LLMQ_HIP(hipMemcpyAsync(vq, kv->vq, ns * 4, hipMemcpyDeviceToHost, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

}  // extern "C"

// ------------------------------------------------------------------- GPT-2

// One linear of Model.blocks / the head (kernels.linear, kernels.mojo:655-673):
// A16 layers take the integer kernels with the LayerNorm fused; float
// activations (A16 = False) take LayerNorm into xn, then matmul_rows.
static int gpt2_linear(llmq_gpt2 *m, const GemvRequest &rq) {
    if (rq.w->a16) return launch_gemv_a16(m->ctx, rq);
    if (rq.T == 1)  // LayerNorm fused into the GEMV's prologue
        return launch_gguf_gemv(m->ctx, rq.w, rq.x, rq.out, rq.bias, rq.flags, rq.amax, rq.amax_cap, nullptr, 0.0f,
                                0, rq.ln_w, rq.ln_b);
    const float *x = rq.x;
    if (rq.ln_w) {
        RC(launch_layernorm(m->ctx, m->xn, rq.x, rq.ln_w, rq.ln_b, rq.T, rq.w->k));
        x = m->xn;
    }
    return launch_gguf_gemm(m->ctx, rq.w, x, rq.w->k, rq.T, rq.out, rq.w->n, rq.bias, rq.flags);
}

// The slot of llmq_gpt2_debug_codes for one linear's input codes.
static int16_t *dbg_slot(llmq_gpt2 *m, int T, int slot) {
    return m->dbg_codes && T == 1 ? m->dbg_codes + (int64_t)slot * 4 * C : nullptr;
}

// Whether a decode step takes its embed step in the first layer's qkv GEMV
// (the exact one-token kernels for that matrix and the head, which copies
// the advanced state back; LLMQ_EMBED_FOLD=0 keeps embed_kernel).
static bool embed_fold_ok(const llmq_gpt2 *m) {
    const char *e = getenv("LLMQ_EMBED_FOLD");
    if (e && e[0] == '0') return false;
    return !m->gguf && !m->fuse_qkv_attn && exact_order() && m->mats[0]->a16 &&
           gemv_exact_embed_ok(m->mats[0], m->wte) && m->wte->a16 && gemv_exact_supports(m->wte);
}

// Model.blocks (gpt2t.mojo:485-571) for T tokens: tokens in m->tokens when
// state == nullptr, else one token picked on the device from the previous
// head's argmax partials (decode), with the position in state[0].  A decode
// step with the embed step folded into the first qkv GEMV finds the advanced
// position in state[2] (the head moves it to state[0]).
static int gpt2_enqueue(llmq_gpt2 *m, int T, int pos0, bool device_step, bool with_head = true) {
    llmq_ctx *ctx = m->ctx;
    const bool fold = device_step && T == 1 && with_head && embed_fold_ok(m);
    EmbedFold ef;
    if (fold) {
        ef.E = m->wte;
        ef.wpe = m->wpe;
        ef.wpe_rows = MAXT;
        ef.parts = m->parts;
        ef.nparts = m->nparts;
        ef.gen = m->gen;
        ef.state = m->state;
        ef.x = m->x;
    } else if (device_step) {
        RC(launch_embed(ctx, m->wte, m->wpe, nullptr, 1, 0, m->x, m->parts, m->nparts, m->gen, m->state, 1));
    } else {
        RC(launch_embed(ctx, m->wte, m->wpe, m->tokens, T, pos0, m->x, nullptr, 0, nullptr, nullptr, 1));
    }
    const int *pos_dev = device_step ? m->state + (fold ? 2 : 0) : nullptr;
    for (int l = 0; l < NL; l++) {
        llmq_mat **w = &m->mats[l * 4];
        const float *const *v = m->vec[l];
        int fused = LLMQ_EUNSUPPORTED;
        if (T == 1 && m->fuse_qkv_attn)  // qkv, the cache store and attention in one kernel
            fused = launch_qkv_attn(ctx, w[0], m->x, v[LN1_W], v[LN1_B], v[QKV_B], m->kv, l, pos0, pos_dev,
                                    m->qkv, m->att);
        if (fused != LLMQ_OK && fused != LLMQ_EUNSUPPORTED) return fused;
        if (fused == LLMQ_EUNSUPPORTED) {
            GemvRequest q;
            q.w = w[0];
            q.x = m->x;
            q.ln_w = v[LN1_W];
            q.ln_b = v[LN1_B];
            q.out = m->qkv;
            q.bias = v[QKV_B];
            q.T = T;
            q.flags = LLMQ_BIAS;
            q.xq_out = dbg_slot(m, T, 4 * l);
            if (fold && l == 0) q.emb = &ef;
            // prompts: the GEMM's epilogue stores the keys and values (else kv_store_kernel)
            KvFold kf;
            kf.cache = m->kv;
            kf.layer = l;
            kf.pos0 = pos0;
            const bool kv_fold = T > 1 && w[0]->a16 && gemm_kv_fold_ok(w[0], T, m->kv);
            if (kv_fold) q.kv = &kf;
            RC(gpt2_linear(m, q));
            if (T > 1 && !kv_fold) RC(launch_kv_store(ctx, m->kv, l, pos0, pos_dev, m->qkv, T, 3 * C));
            RC(launch_kv_attend(ctx, m->kv, m->att, m->qkv, l, T, pos0, pos_dev, 3 * C, T == 1));
        }
        GemvRequest p;
        p.w = w[1];
        p.x = m->att;
        p.out = m->x;
        p.bias = v[PROJ_B];
        p.T = T;
        p.flags = LLMQ_BIAS | LLMQ_RESID;
        p.xq_out = dbg_slot(m, T, 4 * l + 1);
        RC(gpt2_linear(m, p));
        GemvRequest f;
        f.w = w[2];
        f.x = m->x;
        f.ln_w = v[LN2_W];
        f.ln_b = v[LN2_B];
        f.out = m->fc;
        f.bias = v[FC_B];
        f.T = T;
        f.flags = LLMQ_BIAS | LLMQ_GELU;
        f.xq_out = dbg_slot(m, T, 4 * l + 2);
        RC(gpt2_linear(m, f));
        GemvRequest g;
        g.w = w[3];
        g.x = m->fc;
        g.out = m->x;
        g.bias = v[FCPROJ_B];
        g.T = T;
        g.flags = LLMQ_BIAS | LLMQ_RESID;
        g.xq_out = dbg_slot(m, T, 4 * l + 3);
        RC(gpt2_linear(m, g));
    }
    if (!with_head) return LLMQ_OK;
    // Model.forward's tail (gpt2t.mojo:337-340): LN_f on the last row, head.
    GemvRequest h;
    h.w = m->wte;
    h.x = m->x + (int64_t)(T - 1) * C;
    h.ln_w = m->lnf_w;
    h.ln_b = m->lnf_b;
    h.out = m->logits;
    h.T = 1;
    h.flags = 0;
    h.amax = m->parts;
    h.amax_cap = m->nparts;
    h.xq_out = dbg_slot(m, 1, 4 * NL);
    int written = -1;
    h.amax_count = &written;
    if (fold) h.state_copy = m->state;
    RC(gpt2_linear(m, h));
    // the embed step's argmax reads exactly m->nparts partials
    LLMQ_REQUIRE(written < 0 || written == m->nparts, "head: %d argmax partials, the model reads %d", written,
                 m->nparts);
    return LLMQ_OK;
}

static void set_fuse_mode(llmq_gpt2 *m, int max_pos);

// The model's small tensors (host, SMALL_FLOATS in Model.small's order),
// its KV cache and activation buffers; the matrices are already in place.
int gpt2_finish(llmq_gpt2 *m, int attention, const float *small_host) {
    llmq_ctx *ctx = m->ctx;
    auto alloc = [&](auto *&ptr, size_t bytes) -> int {
        if (hipMalloc(&ptr, bytes) != hipSuccess)
            return llmq_set_error(LLMQ_ENOMEM, "gpt2: allocation of %zu bytes", bytes);
        return LLMQ_OK;
    };
    RC(alloc(m->small, sizeof(float) * SMALL_FLOATS));
    int64_t off = 0;
    for (int l = 0; l < NL; l++)
        for (int s = 0; s < N_VECS; s++) {
            m->vec[l][s] = m->small + off;
            off += VEC_LEN[s];
        }
    m->wpe = m->small + off;
    off += (int64_t)MAXT * C;
    m->lnf_w = m->small + off;
    m->lnf_b = m->small + off + C;
    LLMQ_HIP(hipMemcpy(m->small, small_host, sizeof(float) * SMALL_FLOATS, hipMemcpyHostToDevice));
    const char *fe = getenv("LLMQ_DECODE_FUSION");
    m->fuse_env = fe && fe[0] == '0' ? 0 : (fe && fe[0] == '1' ? 1 : -1);
    // run_with[W, E, QuantKV[8] or IntAttnKV] (gpt2t.mojo:1238-1257)
    if (attention == LLMQ_ATTN_INT)
        RC(llmq_ikv_create(ctx, NL, MAXT, NH, HS, &m->kv));
    else
        RC(llmq_kv_create(ctx, NL, MAXT, NH, HS, &m->kv));
    RC(alloc(m->x, sizeof(float) * MAXT * C));
    RC(alloc(m->qkv, sizeof(float) * MAXT * 3 * C));
    RC(alloc(m->att, sizeof(float) * MAXT * C));
    RC(alloc(m->fc, sizeof(float) * MAXT * 4 * C));
    RC(alloc(m->logits, sizeof(float) * V));
    bool float_act = m->gguf != 0;  // LayerNorm output buffer for float-activation matrices
    for (auto *w : m->mats) float_act = float_act || is_float_act(w);
    if (float_act || is_float_act(m->wte)) RC(alloc(m->xn, sizeof(float) * MAXT * C));
    if (!m->gguf) {  // the head's argmax partials for the device-driven decode loop
        m->nparts = m->wte->a16 ? gemv_a16_num_parts(m->wte, true) : gguf_num_parts(m->wte);
        LLMQ_REQUIRE(m->nparts > 0, "gpt2: the head kernel leaves no argmax partials");
        RC(alloc(m->parts, sizeof(ArgmaxPart) * m->nparts));
        // no stale partial can win an argmax before the first head runs
        const std::vector<ArgmaxPart> none((size_t)m->nparts, ArgmaxPart{-INFINITY, 0x7fffffff});
        LLMQ_HIP(hipMemcpy(m->parts, none.data(), sizeof(ArgmaxPart) * m->nparts, hipMemcpyHostToDevice));
    }
    RC(alloc(m->tokens, sizeof(int64_t) * MAXT));
    RC(alloc(m->gen, sizeof(int64_t) * MAXT));
    RC(alloc(m->state, sizeof(int) * 4));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

// Drops the captured decode steps of graph slot i (they hold the pointers
// and the mode they were captured with).
static void drop_step_graph(llmq_gpt2 *m, int i) {
    if (!m->step_graph[i] && !m->step_graph_def[i]) return;
    if (m->ctx) hipStreamSynchronize(m->ctx->stream);
    if (m->step_graph[i]) hipGraphExecDestroy(m->step_graph[i]);
    if (m->step_graph_def[i]) hipGraphDestroy(m->step_graph_def[i]);
    m->step_graph[i] = nullptr;
    m->step_graph_def[i] = nullptr;
}

static void drop_step_graphs(llmq_gpt2 *m) {
    drop_step_graph(m, 0);
    drop_step_graph(m, 1);
}

extern "C" {

int llmq_gpt2_free(llmq_gpt2 *m) {
    if (!m) return LLMQ_OK;
    if (m->ctx) hipStreamSynchronize(m->ctx->stream);
    drop_step_graphs(m);
    llmq_mat_free(m->wte);
    if (m->lm != m->wte) llmq_mat_free(m->lm);
    for (auto *w : m->mats) llmq_mat_free(w);
    hipFree(m->xn);
    llmq_kv_free(m->kv);
    hipFree(m->small);
    hipFree(m->x);
    hipFree(m->qkv);
    hipFree(m->att);
    hipFree(m->fc);
    hipFree(m->logits);
    hipFree(m->parts);
    hipFree(m->tokens);
    hipFree(m->gen);
    hipFree(m->state);
    delete m;
    return LLMQ_OK;
}

int llmq_gpt2_create(llmq_ctx *ctx, const float *const *params, int bits, int group, int sym, llmq_gpt2 **out) {
    return llmq_gpt2_create_ex(ctx, params, bits, group, sym, LLMQ_ATTN_FLOAT, out);
}

int llmq_gpt2_create_ex(llmq_ctx *ctx, const float *const *params, int bits, int group, int sym, int attention,
                        llmq_gpt2 **out) {
    // E = HEAD8_A16 = QuantMatrix[8, 0, False, True] (gpt2t.mojo:1234).
    return gpt2_create_formats(ctx, params, QFormat{bits, group, sym ? 1 : 0, 1}, QFormat{8, 0, 0, 1}, attention, out);
}

int llmq_gpt2_create_fmt(llmq_ctx *ctx, const float *const *params, const char *dtype, const char *head,
                         int attention, llmq_gpt2 **out) {
    LLMQ_REQUIRE(dtype && head, "gpt2_create: bad arguments");
    QFormat w;
    if (!parse_quant_name(dtype, &w))
        return llmq_set_error(LLMQ_EUNSUPPORTED, "unknown --dtype %s (a QuantMatrix format: int8-ch, int4-ch, "
                              "int4-g128, int4-g64, int4-g32, -sym, -a16)", dtype);
    // run_quantized (gpt2t.mojo:1282-1292): int8 per channel, A16 as the layers, or the layers' own format
    QFormat e;
    if (strcmp(head, "int8") == 0)
        e = QFormat{8, 0, 0, w.a16};
    else if (strcmp(head, "same") == 0)
        e = w;
    else
        return llmq_set_error(LLMQ_EINVAL, "unknown --head %s (int8 or same)", head);
    return gpt2_create_formats(ctx, params, w, e, attention, out);
}

}  // extern "C"

int gpt2_create_formats(llmq_ctx *ctx, const float *const *params, const QFormat &fw, const QFormat &fe,
                        int attention, llmq_gpt2 **out) {
    LLMQ_REQUIRE(ctx && params && out, "gpt2_create: bad arguments");
    LLMQ_REQUIRE(attention == LLMQ_ATTN_FLOAT || attention == LLMQ_ATTN_INT, "gpt2_create: attention %d", attention);
    llmq_gpt2 *m = new llmq_gpt2();
    m->ctx = ctx;
    int rc = LLMQ_OK;
#define GO(call)                   \
    do {                           \
        rc = (call);               \
        if (rc != LLMQ_OK) goto fail; \
    } while (0)
    {
        GO(llmq_mat_from_f32(ctx, fe.bits, fe.group, fe.sym, fe.a16, params[0], V, C, 0, &m->wte));
        static const int64_t rows[4] = {C, C, C, 4 * C}, cols[4] = {3 * C, C, 4 * C, C};
        static const int mat_param[4] = {2, 4, 8, 10};
        for (int l = 0; l < NL; l++)
            for (int j = 0; j < 4; j++)
                GO(llmq_mat_from_f32(ctx, fw.bits, fw.group, fw.sym, fw.a16, params[4 + 12 * l + mat_param[j]], rows[j],
                                     cols[j], 1, &m->mats[l * 4 + j]));
        std::vector<float> host((size_t)SMALL_FLOATS);
        int64_t off = 0;
        for (int l = 0; l < NL; l++)
            for (int s = 0; s < N_VECS; s++) {
                memcpy(host.data() + off, params[4 + 12 * l + VEC_PARAM[s]], sizeof(float) * VEC_LEN[s]);
                off += VEC_LEN[s];
            }
        memcpy(host.data() + off, params[1], sizeof(float) * MAXT * C);
        off += (int64_t)MAXT * C;
        memcpy(host.data() + off, params[2], sizeof(float) * C);
        off += C;
        memcpy(host.data() + off, params[3], sizeof(float) * C);
        GO(gpt2_finish(m, attention, host.data()));
    }
    *out = m;
    return LLMQ_OK;
fail:
    llmq_gpt2_free(m);
    return rc;
#undef GO
}

extern "C" {

int64_t llmq_gpt2_weight_bytes(const llmq_gpt2 *m) {
    if (!m) return 0;
    int64_t n = llmq_mat_nbytes(m->wte);
    if (m->lm && m->lm != m->wte) n += llmq_mat_nbytes(m->lm);
    for (auto *w : m->mats) n += llmq_mat_nbytes(w);
    return n + SMALL_FLOATS * 4;  // gpt2t.mojo:312-319
}

int llmq_gpt2_debug_codes(llmq_gpt2 *m, int16_t *codes) {
    LLMQ_REQUIRE(m && !m->gguf, "gpt2_debug_codes: needs a QuantMatrix model");
    if (m->dbg_codes != codes) drop_step_graphs(m);  // the captured steps hold the old pointers
    m->dbg_codes = codes;
    return LLMQ_OK;
}

int llmq_gpt2_forward(llmq_gpt2 *m, const int64_t *tokens, int T, int pos0, float *logits) {
    LLMQ_REQUIRE(m && tokens && T >= 1, "gpt2_forward: bad arguments");
    LLMQ_REQUIRE(pos0 >= 0 && pos0 + T <= MAXT, "gpt2_forward: positions %d..%d beyond %d", pos0, pos0 + T - 1, MAXT);
    for (int t = 0; t < T; t++)
        LLMQ_REQUIRE(tokens[t] >= 0 && tokens[t] < V, "gpt2_forward: token %lld out of range", (long long)tokens[t]);
    OwnStream os_(m->ctx);
    llmq_ctx *ctx = m->ctx;
    LLMQ_HIP(hipMemcpyAsync(m->tokens, tokens, sizeof(int64_t) * T, hipMemcpyHostToDevice, ctx->stream));
    set_fuse_mode(m, pos0 + T);
    RC(m->gguf ? gpt2g_enqueue(m, T, pos0) : gpt2_enqueue(m, T, pos0, false));
    if (logits) {
        LLMQ_HIP(hipMemcpyAsync(logits, m->logits, sizeof(float) * V, hipMemcpyDeviceToHost, ctx->stream));
    }
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

int llmq_gpt2_forward_all(llmq_gpt2 *m, const int64_t *tokens, int T, float *logits) {
    LLMQ_REQUIRE(m && tokens && logits && T >= 1, "gpt2_forward_all: bad arguments");
    LLMQ_REQUIRE(T <= MAXT, "gpt2_forward_all: %d tokens beyond %d", T, MAXT);
    for (int t = 0; t < T; t++)
        LLMQ_REQUIRE(tokens[t] >= 0 && tokens[t] < V, "gpt2_forward_all: token %lld out of range",
                     (long long)tokens[t]);
    OwnStream os_(m->ctx);
    llmq_ctx *ctx = m->ctx;
    LLMQ_HIP(hipMemcpyAsync(m->tokens, tokens, sizeof(int64_t) * T, hipMemcpyHostToDevice, ctx->stream));
    RC(m->gguf ? gpt2g_enqueue(m, T, 0, false) : gpt2_enqueue(m, T, 0, false, false));
    // Model.forward_all's tail (gpt2t.mojo:448-459): LN_f on every row (into
    // att, free after the blocks), then the head for all T rows.
    RC(launch_layernorm(ctx, m->att, m->x, m->lnf_w, m->lnf_b, T, C));
    RC(llmq_head(ctx, logits, m->att, m->gguf ? m->lm : m->wte, T, V, C));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    return LLMQ_OK;
}

int llmq_gpt2_logits_device(llmq_gpt2 *m, float **dptr) {
    LLMQ_REQUIRE(m && dptr, "gpt2_logits_device: bad arguments");
    *dptr = m->logits;
    return LLMQ_OK;
}

// generate -t 0 for the GGUF model (gpt2t.mojo:949-1005): the argmax of each
// step's logits on the host (first maximum, 792-797), fed back as the next
// token; spans timed on the host around synchronized work.
static int gpt2g_generate(llmq_gpt2 *m, const int64_t *prompt, int n_prompt, int steps, int64_t *out_tokens,
                          int *n_out, double *prefill_ms, double *decode_ms) {
    OwnStream os_(m->ctx);
    llmq_ctx *ctx = m->ctx;
    std::vector<float> logits((size_t)V);
    auto now = [] { return std::chrono::steady_clock::now(); };
    auto argmax = [&](int64_t *tok) -> int {
        LLMQ_HIP(hipMemcpyAsync(logits.data(), m->logits, sizeof(float) * V, hipMemcpyDeviceToHost, ctx->stream));
        LLMQ_HIP(hipStreamSynchronize(ctx->stream));
        int64_t best = 0;
        for (int64_t i = 1; i < V; i++)
            if (logits[(size_t)i] > logits[(size_t)best]) best = i;
        *tok = best;
        return LLMQ_OK;
    };
    LLMQ_HIP(hipMemcpyAsync(m->tokens, prompt, sizeof(int64_t) * n_prompt, hipMemcpyHostToDevice, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    const auto t0 = now();
    RC(gpt2g_enqueue(m, n_prompt, 0));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    const auto t1 = now();
    int n = 0, pos = n_prompt;
    bool stopped = false;
    for (int i = 0; i < steps; i++) {
        int64_t tok;
        RC(argmax(&tok));
        if (!stopped && tok == EOT) stopped = true;  // gpt2t.mojo:971-972
        if (!stopped) out_tokens[n++] = tok;
        if (stopped || i + 1 == steps) break;
        LLMQ_HIP(hipMemcpyAsync(m->tokens, &tok, sizeof(int64_t), hipMemcpyHostToDevice, ctx->stream));
        RC(gpt2g_enqueue(m, 1, pos++));
    }
    const auto t2 = now();
    if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    if (decode_ms) *decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
    *n_out = n;
    return LLMQ_OK;
}

// The decode mode for contexts up to max_pos positions; a change drops the
// captured step graph.
static void set_fuse_mode(llmq_gpt2 *m, int max_pos) {
    // The fused kernel's float sums run in another order than the
    // reference's, so it is the default only with LLMQ_EXACT=0.
    const int want = m->fuse_env >= 0 ? m->fuse_env : (!exact_order() && max_pos > kFuseFrom ? 1 : 0);
    if (want == m->fuse_qkv_attn) return;
    m->fuse_qkv_attn = want;
    drop_step_graphs(m);
}

// n device-driven decode steps.  Each step reads its token and position
// from the device, so k steps capture as one graph: it is replayed while k
// or more remain, then the one-step graph.  k = 4 (LLMQ_GRAPH_STEPS): on
// config 0, 1 / 2 / 4 / 8 / 16 / 33 steps a graph measured 3667 / 3685 /
// 3697 / 3696 / 3671 / 3631 tok/s (larger graphs launch more slowly).
static int decode_steps(llmq_gpt2 *m, bool use_graph, int n) {
    llmq_ctx *ctx = m->ctx;
    if (!use_graph) {
        for (int i = 0; i < n; i++) RC(gpt2_enqueue(m, 1, 0, true));
        return LLMQ_OK;
    }
    int k = 4;
    if (const char *e = getenv("LLMQ_GRAPH_STEPS")) k = atoi(e);
    k = k < 1 ? 1 : k > 64 ? 64 : k;
    if (k > 1 && n >= k) {
        if (m->step_k != k) drop_step_graph(m, 1);
        if (!m->step_graph[1]) {
            RC(llmq_capture(
                ctx->stream,
                [&]() -> int {
                    for (int i = 0; i < k; i++) RC(gpt2_enqueue(m, 1, 0, true));
                    return LLMQ_OK;
                },
                &m->step_graph_def[1], &m->step_graph[1]));
            m->step_k = k;
        }
        for (; n >= k; n -= k) LLMQ_HIP(hipGraphLaunch(m->step_graph[1], ctx->stream));
    }
    if (n > 0 && !m->step_graph[0])
        RC(llmq_capture(ctx->stream, [&] { return gpt2_enqueue(m, 1, 0, true); }, &m->step_graph_def[0],
                        &m->step_graph[0]));
    for (; n > 0; n--) LLMQ_HIP(hipGraphLaunch(m->step_graph[0], ctx->stream));
    return LLMQ_OK;
}

int llmq_gpt2_generate(llmq_gpt2 *m, const int64_t *prompt, int n_prompt, int steps, int64_t *out_tokens, int *n_out,
                       double *prefill_ms, double *decode_ms) {
    LLMQ_REQUIRE(m && prompt && n_prompt >= 1 && steps >= 0 && out_tokens && n_out, "gpt2_generate: bad arguments");
    LLMQ_REQUIRE(n_prompt <= MAXT, "gpt2_generate: prompt longer than %d", MAXT);
    for (int t = 0; t < n_prompt; t++)
        LLMQ_REQUIRE(prompt[t] >= 0 && prompt[t] < V, "gpt2_generate: token %lld out of range", (long long)prompt[t]);
    steps = steps < MAXT - n_prompt ? steps : MAXT - n_prompt;  // gpt2t.mojo:945
    if (m->gguf) return gpt2g_generate(m, prompt, n_prompt, steps, out_tokens, n_out, prefill_ms, decode_ms);
    set_fuse_mode(m, n_prompt + steps);
    OwnStream os_(m->ctx);
    llmq_ctx *ctx = m->ctx;
    const char *ge = getenv("LLMQ_GRAPH");
    const bool use_graph = !(ge && ge[0] == '0');
    ScopedEvents ev;
    RC(ev.create());
    hipEvent_t e0 = ev.e[0], e1 = ev.e[1], e2 = ev.e[2];
    LLMQ_HIP(hipMemcpyAsync(m->tokens, prompt, sizeof(int64_t) * n_prompt, hipMemcpyHostToDevice, ctx->stream));
    const int init_state[4] = {n_prompt - 1, -1, 0, 0};
    LLMQ_HIP(hipMemcpyAsync(m->state, init_state, sizeof(init_state), hipMemcpyHostToDevice, ctx->stream));
    LLMQ_HIP(hipStreamSynchronize(ctx->stream));
    LLMQ_HIP(hipEventRecord(e0, ctx->stream));
    RC(gpt2_enqueue(m, n_prompt, 0, false));
    LLMQ_HIP(hipEventRecord(e1, ctx->stream));
    if (steps > 0) {
        RC(decode_steps(m, use_graph, steps - 1));
        // the last token: argmax only (gpt2t.mojo:975-976)
        RC(launch_embed(ctx, m->wte, m->wpe, nullptr, 1, 0, m->x, m->parts, m->nparts, m->gen, m->state, 0));
    }
    LLMQ_HIP(hipEventRecord(e2, ctx->stream));
    LLMQ_HIP(hipEventSynchronize(e2));
    float a = 0, b = 0;
    LLMQ_HIP(hipEventElapsedTime(&a, e0, e1));
    LLMQ_HIP(hipEventElapsedTime(&b, e1, e2));
    if (prefill_ms) *prefill_ms = a;
    if (decode_ms) *decode_ms = b;
    std::vector<int64_t> g(steps > 0 ? steps : 1);
    if (steps > 0) LLMQ_HIP(hipMemcpy(g.data(), m->gen, sizeof(int64_t) * steps, hipMemcpyDeviceToHost));
    int n = 0;
    for (; n < steps; n++) {
        if (g[n] == EOT) break;  // gpt2t.mojo:971-972
        out_tokens[n] = g[n];
    }
    *n_out = n;
    return LLMQ_OK;
}

}  // extern "C"
