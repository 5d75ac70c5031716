/*
 * llmq_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of llm_mojo's CPU arithmetic for its quantized-weight
 * matmul path: the QuantMatrix quantizer and code layouts, int16 activation
 * quantization, the VPDPWSSD-based integer GEMV / GEMM kernels, the GGUF
 * block decoders, the int8 KV cache with float attention, and the GPT-2 model
 * step that calls them.  It is the parity checker for the HIP product and the
 * CPU baseline timed next to it.  Nothing in llm_mojo_amd/ links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg do.
 *
 * Every function cites the reference file:line it follows (paths relative to
 * the llm_mojo tree).  Floating-point operations follow the reference's order
 * (16-lane SIMD accumulators are emulated lane by lane; fused multiply-adds
 * only where the reference calls .fma), so the file must be compiled with
 * -ffp-contract=off and without fast-math.
 *
 * Pinning status (what each function is checked against lives in tests/):
 *   - tie rule of Mojo's round(): parity unpinned (Mojo 1.1 stdlib absent);
 *     default half-away-from-zero, switchable with orc_set_round_half_even.
 *     Exact ties are counted per rounding site (orc_ties): config 0 meets
 *     136 in its weights and ~30 per forward in its int16 activation codes;
 *     the two rules give the same greedy tokens there (tests/).
 *   - order of SIMD.reduce_add / reduce_max: parity unpinned; emulated as a
 *     halving tree (lanes 0-7 + 8-15, ...).  Moves fp32 bits only.
 *   - last-ulp results of Mojo's exp / tanh: parity unpinned (Mojo 1.1
 *     stdlib absent).  The float path's exp and tanh are this build's own
 *     (orc_exp / orc_tanh below, the same method as the HIP product), so the
 *     oracle and the GPU round alike; tests pin them against float64 exp and
 *     tanh (under 1 and 1.3 ulp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define L16 16

/* ------------------------------------------------------------------------ */
/* Scalar helpers                                                            */
/* ------------------------------------------------------------------------ */

static int g_half_even = 0;

/* Mojo std.math.round (tensor.mojo:377,381; kernels.mojo:415;
 * kvcache.mojo:330).  Tie rule unpinned: half away from zero by default. */
void orc_set_round_half_even(int on) { g_half_even = on; }
static inline double orc_round_d(double v) { return g_half_even ? nearbyint(v) : round(v); }

/* Exact .5 ties met by each rounding site (where the tie rule decides the
 * result): 0 weight codes and zero points (from_f32), 1 int16 activation
 * codes (quantize_rows), 2 int8 KV codes (QuantKV.store), 3 the rest. */
static int64_t g_ties[4];
void orc_ties(int64_t *out) {
    for (int i = 0; i < 4; i++) out[i] = __atomic_load_n(&g_ties[i], __ATOMIC_RELAXED);
}
void orc_reset_ties(void) {
    for (int i = 0; i < 4; i++) __atomic_store_n(&g_ties[i], 0, __ATOMIC_RELAXED);
}
static inline float orc_round_at(float v, int site) {
    if (fabsf(v - truncf(v)) == 0.5f) __atomic_fetch_add(&g_ties[site], 1, __ATOMIC_RELAXED);
    return g_half_even ? nearbyintf(v) : roundf(v);
}
static inline float orc_round(float v) { return orc_round_at(v, 3); }

/* Int(float) for a value already rounded to an integer.  NaN (a scale that
 * rounded to zero in float16: outside the reference's defined inputs) maps
 * to 0, and out-of-range values saturate, so the clamp that follows is
 * well defined. */
static inline int64_t orc_to_int(float r) {
    if (r != r) return 0;
    if (r > 9.0e18f) return INT64_MAX / 2;
    if (r < -9.0e18f) return INT64_MIN / 2;
    return (int64_t)r;
}

/* float32 -> IEEE binary16 bits, round to nearest even (Mojo's
 * .cast[DType.float16](), tensor.mojo:371). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf, nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0));
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u); /* >= 65536 */
    uint32_t e = ax >> 23;
    if (e < 102) return (uint16_t)sign; /* < 2^-25: rounds to zero */
    if (e < 113) {                      /* f16 subnormal: n * 2^-24 */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* 14..24 */
        uint32_t n = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (n & 1))) n++;
        return (uint16_t)(sign | n);
    }
    uint32_t h = ((e - 112) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++; /* carry may reach inf: correct */
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24, exact in float */
            float v = (float)m * (1.0f / 16777216.0f);
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* SIMD[f32,16].reduce_add: order unpinned, emulated as a halving tree. */
static inline float red16(const float *v) {
    float a[8], b[4], c[2];
    for (int i = 0; i < 8; i++) a[i] = v[i] + v[i + 8];
    for (int i = 0; i < 4; i++) b[i] = a[i] + a[i + 4];
    for (int i = 0; i < 2; i++) c[i] = b[i] + b[i + 2];
    return c[0] + c[1];
}

/* dot_pairs (tensor.mojo:34-46): acc[i] + a[2i]*b[2i] + a[2i+1]*b[2i+1],
 * int32 lanes with wraparound (VPDPWSSD). */
static inline void dot_pairs(int32_t *acc, const int16_t *a, const int16_t *b) {
    for (int i = 0; i < L16; i++) {
        int64_t s = (int64_t)a[2 * i] * b[2 * i] + (int64_t)a[2 * i + 1] * b[2 * i + 1];
        acc[i] = (int32_t)(uint32_t)((uint32_t)acc[i] + (uint32_t)(int32_t)s);
    }
}

/* exp and tanh for the float path (attend_float_one's softmax,
 * kvcache.mojo:131-138; store_out's GELU, kernels.mojo:43-45).  Method:
 * exp by Cody and Waite's reduction x = n ln2 + r (n = rint(x log2 e), ln2 as
 * a 24-bit head plus a tail, each product exact inside fmaf), e^r = 1 + r +
 * r^2 P(r), P of degree 4 from a weighted least-squares fit at 4000
 * Chebyshev nodes on [-0.35, 0.35], Horner's rule in fmaf, times 2^n through
 * the exponent bits; x < -87 gives 0 (no subnormals), x > 88.5 infinity.
 * tanh: y + y^3 Q(y^2) below |y| = 0.625 (Q of degree 5, fitted the same
 * way), else 1 - 2 / (exp(2|y|) + 1) with y's sign, and 1 from |y| = 10. */
static inline float f32_from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
float orc_exp(float x) {
    if (x > 88.5f) return INFINITY;
    if (!(x >= -87.0f)) return x != x ? x : 0.0f;
    float n = rintf(x * 1.44269502f);
    float r = fmaf(-n, 0.693145752f, x);
    r = fmaf(-n, 1.42860677e-06f, r);
    float p = 0.0013748823f;
    p = fmaf(p, r, 0.008369628f);
    p = fmaf(p, r, 0.041669644f);
    p = fmaf(p, r, 0.16666512f);
    p = fmaf(p, r, 0.49999988f);
    float r2 = r * r;
    p = fmaf(p, r2, r);
    p = p + 1.0f;
    return p * f32_from_bits((uint32_t)((int)n + 127) << 23);
}
float orc_tanh(float y) {
    float a = fabsf(y);
    if (a < 0.625f) {
        float s = y * y;
        float p = 0.002148991f;
        p = fmaf(p, s, -0.00818467f);
        p = fmaf(p, s, 0.021704003f);
        p = fmaf(p, s, -0.053947456f);
        p = fmaf(p, s, 0.13333212f);
        p = fmaf(p, s, -0.3333333f);
        return fmaf(p * s, y, y);
    }
    float t = a >= 10.0f ? 1.0f : 1.0f - 2.0f / (orc_exp(2.0f * a) + 1.0f);
    return copysignf(t, y);
}

void orc_exp_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_exp(x[i]);
}
void orc_tanh_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_tanh(x[i]);
}

/* kernels.finish (274-282) / store_out (38-48): GELU, residual, store. */
#define EPI_BIAS 1
#define EPI_GELU 2
#define EPI_RESID 4
static inline float gelu_f(float r) {
    const float s = 0.7978845608028654f;
    float t = 0.044715f * r;
    t = t * r;
    t = t * r;
    float u = r + t;
    float th = orc_tanh(s * u);
    float a = 0.5f * r;
    return a * (1.0f + th);
}
void orc_gelu_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = gelu_f(x[i]);
}
static inline void finish(float *o, int64_t i, float r, int flags) {
    if (flags & EPI_GELU) r = gelu_f(r);
    if (flags & EPI_RESID) r += o[i];
    o[i] = r;
}

/* ------------------------------------------------------------------------ */
/* QuantMatrix (tensor.mojo:230-661)                                        */
/* ------------------------------------------------------------------------ */

typedef struct {
    int32_t bits;     /* 4 or 8 */
    int32_t sym;      /* SYMMETRIC */
    int32_t a16;      /* A16 */
    int32_t blocked;  /* BLOCKED = a16 && bits == 4 && GROUP == 32 (tensor.mojo:296) */
    int32_t perch;    /* GROUP == 0: one group per row ("per-channel") */
    int64_t n;        /* rows: outputs */
    int64_t k;        /* cols: the reduction axis */
    int64_t group;    /* weights per group (GROUP, or k for per-channel) */
    uint8_t *data;    /* codes, n * k * bits / 8 */
    uint16_t *scale;  /* float16 bits, n * k / group */
    uint8_t *zp;      /* n * k / group */
} orc_qm;

/* nibble_at (tensor.mojo:385-404): byte within the row holding column col's
 * code, and whether it is the high nibble. */
static inline void nibble_at(int blocked, int64_t col, int64_t *byte, int *high) {
    int64_t j, chunk;
    if (blocked) {
        int64_t w = col % 256, e = w % 32, p = e / 2;
        int64_t lane = w / 32 + 8 * (p / 8);
        chunk = (col / 256) * 8 + p % 8;
        j = 2 * lane + e % 2;
    } else {
        chunk = col / 32;
        j = col % 32;
    }
    *byte = chunk * 16 + j % 16;
    *high = j >= 16;
}
void orc_nibble_at(int blocked, int64_t col, int64_t *byte, int *high) { nibble_at(blocked, col, byte, high); }

/* set_code / code (tensor.mojo:406-429) */
static inline void set_code(const orc_qm *m, int64_t row, int64_t col, int u) {
    uint8_t *p = m->data + row * m->k * m->bits / 8;
    if (m->bits == 8) {
        p[col] = (uint8_t)u;
        return;
    }
    int64_t b;
    int hi;
    nibble_at(m->blocked, col, &b, &hi);
    if (hi)
        p[b] = (uint8_t)((p[b] & 0x0f) | (u << 4));
    else
        p[b] = (uint8_t)((p[b] & 0xf0) | u);
}
static inline int get_code(const orc_qm *m, int64_t row, int64_t col) {
    const uint8_t *p = m->data + row * m->k * m->bits / 8;
    if (m->bits == 8) return p[col];
    int64_t b;
    int hi;
    nibble_at(m->blocked, col, &b, &hi);
    return hi ? (p[b] >> 4) : (p[b] & 0xf);
}
int orc_qm_code(const orc_qm *m, int64_t row, int64_t col) { return get_code(m, row, col); }

static inline int clamp_code(int64_t u, int levels) { /* tensor.mojo:664-667 */
    return (int)(u < 0 ? 0 : (u > levels ? levels : u));
}

/* QuantMatrix.from_f32 (tensor.mojo:334-383).  m->bits/sym/a16 and m->group
 * (0 = per-channel) are inputs; m->data/scale/zp are caller-allocated with
 * the sizes orc_qm_sizes reports.  Returns 0, or -1 for a bad group. */
int orc_qm_from_f32(orc_qm *m, const float *src, int64_t rows, int64_t cols, int reduce_rows) {
    int64_t n = reduce_rows ? cols : rows;
    int64_t k = reduce_rows ? rows : cols;
    int64_t group = m->group == 0 ? k : m->group;
    if (k % group != 0 || group % 32 != 0) return -1;
    m->blocked = m->a16 && m->bits == 4 && m->group == 32;
    m->perch = m->group == 0;
    m->n = n;
    m->k = k;
    m->group = group;
    int levels = (1 << m->bits) - 1, half = 1 << (m->bits - 1);
    int64_t gpr = k / group;
    memset(m->data, 0, (size_t)(n * k * m->bits / 8));
    float *vals = (float *)malloc(sizeof(float) * (size_t)group);
    for (int64_t r = 0; r < n; r++) {
        for (int64_t g = 0; g < gpr; g++) {
            float lo = 0.0f, hi = 0.0f;
            for (int64_t j = 0; j < group; j++) {
                int64_t c = g * group + j;
                float v = reduce_rows ? src[c * cols + r] : src[r * cols + c];
                vals[j] = v;
                lo = v < lo ? v : lo;
                hi = v > hi ? v : hi;
            }
            float s;
            if (m->sym) {
                float a = -lo > hi ? -lo : hi;
                s = a / (float)(half - 1);
            } else {
                s = (hi - lo) / (float)levels;
            }
            if (s == 0.0f) s = 1.0f;
            uint16_t s16 = orc_f32_to_f16(s);
            float sf = orc_f16_to_f32(s16);
            int zp = m->sym ? half : clamp_code(orc_to_int(orc_round_at(-lo / sf, 0)), levels);
            m->scale[r * gpr + g] = s16;
            m->zp[r * gpr + g] = (uint8_t)zp;
            for (int64_t j = 0; j < group; j++) {
                int64_t u = orc_to_int(orc_round_at(vals[j] / sf, 0)) + zp;
                set_code(m, r, g * group + j, clamp_code(u, levels));
            }
        }
    }
    free(vals);
    return 0;
}

/* nbytes (tensor.mojo:629-632) */
int64_t orc_qm_nbytes(const orc_qm *m) { return m->n * m->k * m->bits / 8 + (m->n * m->k / m->group) * 3; }

/* row_op (tensor.mojo:431-476): dequantize a row (DOT=0) or the partial sums
 * of its dot product with x (DOT=1), returned as the 16 lanes' reduce_add. */
static float row_op(const orc_qm *m, int64_t row, float *dst, const float *x, int dot) {
    const uint8_t *p = m->data + row * m->k * m->bits / 8;
    int64_t gpr = m->k / m->group;
    if (m->blocked) { /* scalar path (tensor.mojo:438-452) */
        float d = 0.0f;
        for (int64_t k = 0; k < m->k; k++) {
            int64_t g = row * gpr + k / m->group;
            float v = (float)(get_code(m, row, k) - (int)m->zp[g]) * orc_f16_to_f32(m->scale[g]);
            if (dot)
                d += v * x[k];
            else
                dst[k] = v;
        }
        return d; /* acc[0] = d; reduce_add of (d, 0, ...) is d */
    }
    float acc[L16] = {0};
    for (int64_t g = 0; g < gpr; g++) {
        float s = orc_f16_to_f32(m->scale[row * gpr + g]);
        float zp = (float)m->zp[row * gpr + g];
        float accg[L16] = {0};
        for (int64_t c = 0; c < m->group / 32; c++) {
            int64_t k0 = g * m->group + 32 * c;
            float v0[L16], v1[L16];
            for (int i = 0; i < L16; i++) {
                if (m->bits == 4) {
                    uint8_t b = p[k0 / 2 + i];
                    v0[i] = (float)(b & 0xf) - zp;
                    v1[i] = (float)(b >> 4) - zp;
                } else {
                    v0[i] = (float)p[k0 + i] - zp;
                    v1[i] = (float)p[k0 + 16 + i] - zp;
                }
            }
            for (int i = 0; i < L16; i++) {
                if (dot) {
                    accg[i] = fmaf(v0[i], x[k0 + i], accg[i]);
                    accg[i] = fmaf(v1[i], x[k0 + 16 + i], accg[i]);
                } else {
                    dst[k0 + i] = v0[i] * s;
                    dst[k0 + 16 + i] = v1[i] * s;
                }
            }
        }
        if (dot)
            for (int i = 0; i < L16; i++) acc[i] = fmaf(accg[i], s, acc[i]);
    }
    return red16(acc);
}
void orc_qm_dequant_row(const orc_qm *m, int64_t row, float *dst) { (void)row_op(m, row, dst, dst, 0); }
float orc_qm_dot_row(const orc_qm *m, int64_t row, const float *x) { return row_op(m, row, NULL, x, 1); }

/* codes_i16 (tensor.mojo:484-496): 32 codes from column k0, minus zp. */
static inline void codes_i16(const orc_qm *m, const uint8_t *p, int64_t k0, int16_t zp, int16_t *out) {
    for (int i = 0; i < 16; i++) {
        if (m->bits == 4) {
            uint8_t b = p[k0 / 2 + i];
            out[i] = (int16_t)((b & 0xf) - zp);
            out[16 + i] = (int16_t)((b >> 4) - zp);
        } else {
            out[i] = (int16_t)(p[k0 + i] - zp);
            out[16 + i] = (int16_t)(p[k0 + 16 + i] - zp);
        }
    }
}

/* permute_x_i16 (tensor.mojo:498-516).  Returns 1 (and fills dst, sums) for
 * the BLOCKED layout, 0 otherwise. */
int orc_qm_permute_x_i16(const orc_qm *m, const int16_t *xq, int64_t n, int16_t *dst, float *sums) {
    if (!m->blocked) return 0;
    for (int64_t blk = 0; blk < n / 256; blk++) {
        for (int lane = 0; lane < 16; lane++) sums[blk * 16 + lane] = 0.0f;
        for (int64_t w = 0; w < 256; w++) {
            int64_t col = blk * 256 + w, e = w % 32, p = e / 2;
            int64_t lane = w / 32 + 8 * (p / 8);
            int16_t v = xq[col];
            dst[blk * 256 + (p % 8) * 32 + 2 * lane + e % 2] = v;
            sums[blk * 16 + lane] += (float)v;
        }
    }
    return 1;
}

/* dot_row_i16 (tensor.mojo:518-577), all three branches. */
float orc_qm_dot_row_i16(const orc_qm *m, int64_t row, const int16_t *xq, const float *xsums) {
    const uint8_t *p = m->data + row * m->k * m->bits / 8;
    int64_t gpr = m->k / m->group;
    float accf[L16] = {0};
    if (m->blocked) { /* 522-540 */
        for (int64_t blk = 0; blk < m->k / 256; blk++) {
            int32_t acc[L16] = {0};
            for (int step = 0; step < 8; step++) {
                const uint8_t *b = p + blk * 128 + step * 16;
                int16_t u[32];
                for (int i = 0; i < 16; i++) {
                    u[i] = (int16_t)(b[i] & 0xf);
                    u[16 + i] = (int16_t)(b[i] >> 4);
                }
                dot_pairs(acc, xq + blk * 256 + step * 32, u);
            }
            int64_t g0 = row * gpr + blk * 8;
            for (int i = 0; i < L16; i++) {
                float zp = (float)m->zp[g0 + i % 8];
                float sc = orc_f16_to_f32(m->scale[g0 + i % 8]);
                float xs = xsums[blk * 16 + i];
                float t = (float)acc[i] - zp * xs;
                accf[i] = fmaf(t, sc, accf[i]);
            }
        }
        return red16(accf);
    }
    if (m->perch && m->bits == 8) { /* int8 per-channel, 541-566 */
        int16_t zp = (int16_t)m->zp[row];
        int32_t acc[L16] = {0};
        int16_t w[32];
        for (int64_t k = 0; k < m->k; k += 32) {
            codes_i16(m, p, k, zp, w);
            dot_pairs(acc, xq + k, w);
        }
        float s = orc_f16_to_f32(m->scale[row]);
        for (int i = 0; i < L16; i++) accf[i] = fmaf((float)acc[i], s, 0.0f);
        return red16(accf);
    }
    for (int64_t g = 0; g < gpr; g++) { /* generic, 567-577 */
        int16_t zp = (int16_t)m->zp[row * gpr + g];
        int32_t acc[L16] = {0};
        int16_t w[32];
        for (int64_t c = 0; c < m->group / 32; c++) {
            int64_t k0 = g * m->group + 32 * c;
            codes_i16(m, p, k0, zp, w);
            dot_pairs(acc, xq + k0, w);
        }
        float s = orc_f16_to_f32(m->scale[row * gpr + g]);
        for (int i = 0; i < L16; i++) accf[i] = fmaf((float)acc[i], s, accf[i]);
    }
    return red16(accf);
}

/* unpack_row_i16 (tensor.mojo:579-615) */
void orc_qm_unpack_row_i16(const orc_qm *m, int64_t row, int16_t *dst, float *scales) {
    const uint8_t *p = m->data + row * m->k * m->bits / 8;
    int64_t gpr = m->k / m->group;
    for (int64_t g = 0; g < gpr; g++) scales[g] = orc_f16_to_f32(m->scale[row * gpr + g]);
    if (m->blocked) {
        for (int64_t blk = 0; blk < m->k / 256; blk++) {
            const uint8_t *zp8 = m->zp + row * gpr + blk * 8;
            for (int step = 0; step < 8; step++) {
                const uint8_t *b = p + blk * 128 + step * 16;
                int16_t u[32];
                for (int i = 0; i < 16; i++) {
                    u[i] = (int16_t)(b[i] & 0xf);
                    u[16 + i] = (int16_t)(b[i] >> 4);
                }
                for (int L = 0; L < 16; L++) {
                    int16_t z = (int16_t)zp8[L % 8];
                    int64_t at = blk * 128 + (L % 8) * 16 + (L / 8) * 8 + step;
                    dst[2 * at] = (int16_t)(u[2 * L] - z);
                    dst[2 * at + 1] = (int16_t)(u[2 * L + 1] - z);
                }
            }
        }
        return;
    }
    for (int64_t g = 0; g < gpr; g++) {
        int16_t zp = (int16_t)m->zp[row * gpr + g];
        for (int64_t c = 0; c < m->group / 32; c++) {
            int64_t k0 = g * m->group + 32 * c;
            codes_i16(m, p, k0, zp, dst + k0);
        }
    }
}

/* Exact per-group integer sums G[o, g] = sum_{k in g} xq_k * (u_{o,k} - zp_{o,g})
 * (the invariant the integer kernels compute; tensor.mojo:262-275). */
void orc_qm_group_sums(const orc_qm *m, const int16_t *xq, int64_t *G) {
    int64_t gpr = m->k / m->group;
    for (int64_t o = 0; o < m->n; o++)
        for (int64_t g = 0; g < gpr; g++) {
            int64_t s = 0;
            int zp = m->zp[o * gpr + g];
            for (int64_t j = 0; j < m->group; j++) {
                int64_t k = g * m->group + j;
                s += (int64_t)xq[k] * (get_code(m, o, k) - zp);
            }
            G[o * gpr + g] = s;
        }
}

/* ------------------------------------------------------------------------ */
/* Activations and the integer matmul driver (kernels.mojo:400-652)          */
/* ------------------------------------------------------------------------ */

/* quantize_rows (kernels.mojo:400-416) */
void orc_quantize_rows(const float *x, int64_t T, int64_t IN, int16_t *xq, float *sx) {
    for (int64_t t = 0; t < T; t++) {
        const float *row = x + t * IN;
        float mx = 0.0f;
        for (int64_t i = 0; i < IN; i++) {
            float a = fabsf(row[i]);
            mx = a > mx ? a : mx;
        }
        float s = mx / 32767.0f;
        if (s == 0.0f) s = 1.0f;
        sx[t] = s;
        float inv = 1.0f / s;
        for (int64_t i = 0; i < IN; i++) xq[t * IN + i] = (int16_t)orc_to_int(orc_round_at(row[i] * inv, 1));
    }
}

/* dot1_i16 (kernels.mojo:617-628): rows_i16 and head_i16's per-row dot. */
static float dot1_i16(const int16_t *wq, const float *ws, const int16_t *xq, int64_t IN, int64_t G) {
    float accf[L16] = {0};
    for (int64_t g = 0; g < IN / G; g++) {
        int32_t acc[L16] = {0};
        for (int64_t k = g * G; k < (g + 1) * G; k += 32) dot_pairs(acc, xq + k, wq + k);
        for (int i = 0; i < L16; i++) accf[i] = fmaf((float)acc[i], ws[g], accf[i]);
    }
    return red16(accf);
}

static int g_threads = 1;
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_get_threads(void) { return g_threads; }

/* tile_i16 (kernels.mojo:512-573) for TM tokens at t0 and the TN = 32 rows at
 * o0 held in wt (VNNI pair layout) and st ([group][row]). */
static void tile_i16(int TM, float *out, const int16_t *xq, const float *sx, const int16_t *wt, const float *st,
                     const float *b, int64_t t0, int64_t o0, int64_t IN, int64_t OUT, int64_t G, int flags) {
    const int TN = 32, SEG = 256;
    float accf[4][32];
    memset(accf, 0, sizeof(accf));
    int64_t seg = G < SEG ? G : SEG;
    for (int64_t k0 = 0; k0 < IN; k0 += seg) {
        int64_t g = k0 / G;
        int32_t acc[4][32];
        memset(acc, 0, sizeof(acc));
        for (int64_t kp = k0 / 2; kp < (k0 + seg) / 2; kp++) {
            for (int m = 0; m < TM; m++) {
                int64_t xoff = (t0 + m) * IN + 2 * kp;
                int16_t x0 = xq[xoff], x1 = xq[xoff + 1];
                for (int j = 0; j < TN; j++) {
                    int16_t w0 = wt[(kp * TN + j) * 2], w1 = wt[(kp * TN + j) * 2 + 1];
                    int64_t s = (int64_t)x0 * w0 + (int64_t)x1 * w1;
                    acc[m][j] = (int32_t)(uint32_t)((uint32_t)acc[m][j] + (uint32_t)(int32_t)s);
                }
            }
        }
        for (int m = 0; m < TM; m++)
            for (int j = 0; j < TN; j++) accf[m][j] = fmaf((float)acc[m][j], st[g * TN + j], accf[m][j]);
    }
    for (int m = 0; m < TM; m++) {
        float sxm = sx[t0 + m];
        for (int j = 0; j < TN; j++) {
            float r = accf[m][j] * sxm;
            if (flags & EPI_BIAS) r += b[o0 + j];
            finish(out, (t0 + m) * OUT + o0 + j, r, flags);
        }
    }
}

/* CPU-baseline hooks (orc_cpu_set_fast, in the baseline section below):
 * AVX-512 VNNI forms of the tile, the one-token row dot, the row quantizer
 * and one head's attention, each bit-identical to the scalar code it
 * stands in for (tests/test_cpu_baseline.py).  NULL: the scalar oracle. */
typedef void (*orc_tile_fn)(int, float *, const int16_t *, const float *, const int16_t *, const float *,
                            const float *, int64_t, int64_t, int64_t, int64_t, int64_t, int);
static orc_tile_fn g_fast_tile = NULL;
static float (*g_fast_row)(const orc_qm *, int64_t, const int16_t *, const float *) = NULL;
static void (*g_fast_quant)(const float *, int64_t, int16_t *, float *) = NULL;

/* matmul_rows_a16 (kernels.mojo:419-509): out[T, OUT] (+)= act(x @ w^T + b).
 * flags: EPI_BIAS | EPI_GELU | EPI_RESID.  Rows (T == 1) or 32-row tiles
 * (T > 1) are split across g_threads threads; the arithmetic per output does
 * not depend on the split. */
void orc_matmul_rows_a16(float *out, const float *x, const orc_qm *w, const float *b, int64_t T, int64_t IN,
                         int64_t OUT, int flags) {
    int16_t *xq = (int16_t *)malloc(sizeof(int16_t) * (size_t)(T * IN));
    float *sx = (float *)malloc(sizeof(float) * (size_t)T);
    if (g_fast_quant && IN % 16 == 0) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1 && T > 1)
        for (int64_t t = 0; t < T; t++) g_fast_quant(x + t * IN, IN, xq + t * IN, sx + t);
    } else {
        orc_quantize_rows(x, T, IN, xq, sx);
    }
    if (T == 1) {
        int16_t *xp = (int16_t *)malloc(sizeof(int16_t) * (size_t)IN);
        float *xs = (float *)malloc(sizeof(float) * (size_t)(IN / 16 + 1));
        const int16_t *x1 = orc_qm_permute_x_i16(w, xq, IN, xp, xs) ? xp : xq;
        float s = sx[0];
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
        for (int64_t o = 0; o < OUT; o++) {
            float r = (g_fast_row ? g_fast_row(w, o, x1, xs) : orc_qm_dot_row_i16(w, o, x1, xs)) * s;
            if (flags & EPI_BIAS) r += b[o];
            finish(out, o, r, flags);
        }
        free(xp);
        free(xs);
    } else {
        int64_t G = w->group;
        const int TN = 32;
        int64_t full = OUT / TN;
        int64_t ntasks = full + (OUT % TN != 0);
#pragma omp parallel for schedule(dynamic) num_threads(g_threads) if (g_threads > 1)
        for (int64_t ti = 0; ti < ntasks; ti++) {
            int16_t *row = (int16_t *)malloc(sizeof(int16_t) * (size_t)IN);
            float *rs = (float *)malloc(sizeof(float) * (size_t)(IN / G));
            if (ti == full) { /* rows_i16 (kernels.mojo:576-614) */
                for (int64_t o = full * TN; o < OUT; o++) {
                    orc_qm_unpack_row_i16(w, o, row, rs);
                    float bias = (flags & EPI_BIAS) ? b[o] : 0.0f;
                    for (int64_t t = 0; t < T; t++) {
                        float d = dot1_i16(row, rs, xq + t * IN, IN, G);
                        finish(out, t * OUT + o, d * sx[t] + bias, flags);
                    }
                }
            } else {
                int64_t o0 = ti * TN;
                int16_t *wt = (int16_t *)malloc(sizeof(int16_t) * (size_t)(IN * TN));
                float *st = (float *)malloc(sizeof(float) * (size_t)(IN / G * TN));
                for (int j = 0; j < TN; j++) {
                    orc_qm_unpack_row_i16(w, o0 + j, row, rs);
                    for (int64_t k = 0; k < IN; k++) wt[((k / 2) * TN + j) * 2 + k % 2] = row[k];
                    for (int64_t g = 0; g < IN / G; g++) st[g * TN + j] = rs[g];
                }
                int64_t t = 0;
                const orc_tile_fn tile = g_fast_tile ? g_fast_tile : tile_i16;
                for (; t + 4 <= T; t += 4) tile(4, out, xq, sx, wt, st, b, t, o0, IN, OUT, G, flags);
                for (; t < T; t++) tile(1, out, xq, sx, wt, st, b, t, o0, IN, OUT, G, flags);
                free(wt);
                free(st);
            }
            free(row);
            free(rs);
        }
    }
    free(xq);
    free(sx);
}

/* ------------------------------------------------------------------------ */
/* GGUF block formats (gguf.mojo:41-511)                                     */
/* ------------------------------------------------------------------------ */

enum { GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q4_1 = 3, GGML_Q8_0 = 8, GGML_Q4_K = 12, GGML_Q5_K = 13, GGML_Q6_K = 14 };

int orc_gguf_block_size(int t) { /* gguf.mojo:72-78 */
    if (t == GGML_F32 || t == GGML_F16) return 1;
    if (t == GGML_Q4_0 || t == GGML_Q4_1 || t == GGML_Q8_0) return 32;
    return 256;
}
int orc_gguf_block_bytes(int t) { /* gguf.mojo:81-98 */
    switch (t) {
    case GGML_F32: return 4;
    case GGML_F16: return 2;
    case GGML_Q4_0: return 18;
    case GGML_Q4_1: return 20;
    case GGML_Q8_0: return 34;
    case GGML_Q4_K: return 144;
    case GGML_Q5_K: return 176;
    case GGML_Q6_K: return 210;
    default: return 0;
    }
}
static inline float f16_at(const uint8_t *p, int i) { return orc_f16_to_f32((uint16_t)(p[i] | (p[i + 1] << 8))); }

/* put (gguf.mojo:166-175): store 16 values, or fma them into the lanes. */
static inline void put(int dot, float *dst, const float *x, float *acc, int off, const float *v) {
    if (dot)
        for (int i = 0; i < L16; i++) acc[i] = fmaf(v[i], x[off + i], acc[i]);
    else
        for (int i = 0; i < L16; i++) dst[off + i] = v[i];
}

/* k_scale_min (gguf.mojo:205-221) */
static inline void k_scale_min(const uint8_t *q, int j, int *sc, int *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
        return;
    }
    *sc = (q[j + 4] & 0xf) | ((q[j - 4] >> 6) << 4);
    *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
}
void orc_k_scale_min(const uint8_t *q, int j, int *sc, int *mn) { k_scale_min(q, j, sc, mn); }

/* One block at b: dequantize into dst, or fma with x into acc
 * (dequant_q4_0 ... dequant_q6_k, gguf.mojo:178-297). */
static void gguf_block(int t, int dot, const uint8_t *b, float *dst, const float *x, float *acc) {
    float v[L16];
    if (t == GGML_Q4_0) { /* 178-184 */
        float d = f16_at(b, 0);
        const uint8_t *q = b + 2;
        for (int i = 0; i < 16; i++) v[i] = ((float)(q[i] & 0xf) - 8.0f) * d;
        put(dot, dst, x, acc, 0, v);
        for (int i = 0; i < 16; i++) v[i] = ((float)(q[i] >> 4) - 8.0f) * d;
        put(dot, dst, x, acc, 16, v);
    } else if (t == GGML_Q4_1) { /* 187-193 */
        float d = f16_at(b, 0), mm = f16_at(b, 2);
        const uint8_t *q = b + 4;
        for (int i = 0; i < 16; i++) v[i] = d * (float)(q[i] & 0xf) + mm;
        put(dot, dst, x, acc, 0, v);
        for (int i = 0; i < 16; i++) v[i] = d * (float)(q[i] >> 4) + mm;
        put(dot, dst, x, acc, 16, v);
    } else if (t == GGML_Q8_0) { /* 196-202 */
        float d = f16_at(b, 0);
        for (int h = 0; h < 2; h++) {
            for (int i = 0; i < 16; i++) v[i] = d * (float)(int8_t)b[2 + 16 * h + i];
            put(dot, dst, x, acc, 16 * h, v);
        }
    } else if (t == GGML_Q4_K || t == GGML_Q5_K) { /* 224-268 */
        float d = f16_at(b, 0), dmin = f16_at(b, 2);
        const uint8_t *scales = b + 4;
        int five = t == GGML_Q5_K;
        for (int j = 0; j < 4; j++) {
            int sc1, m1i, sc2, m2i;
            k_scale_min(scales, 2 * j, &sc1, &m1i);
            k_scale_min(scales, 2 * j + 1, &sc2, &m2i);
            float d1 = d * (float)sc1, m1 = dmin * (float)m1i;
            float d2 = d * (float)sc2, m2 = dmin * (float)m2i;
            for (int h = 0; h < 2; h++) {
                const uint8_t *q = five ? b + 48 + 32 * j + 16 * h : b + 16 + 32 * j + 16 * h;
                const uint8_t *qh = b + 16 + 16 * h;
                for (int i = 0; i < 16; i++) {
                    int lo = q[i] & 0xf;
                    if (five) lo |= ((qh[i] >> (2 * j)) & 1) << 4;
                    v[i] = d1 * (float)lo - m1;
                }
                put(dot, dst, x, acc, 64 * j + 16 * h, v);
                for (int i = 0; i < 16; i++) {
                    int hi = q[i] >> 4;
                    if (five) hi |= ((qh[i] >> (2 * j + 1)) & 1) << 4;
                    v[i] = d2 * (float)hi - m2;
                }
                put(dot, dst, x, acc, 64 * j + 32 + 16 * h, v);
            }
        }
    } else if (t == GGML_Q6_K) { /* 271-297 */
        float d = f16_at(b, 208);
        for (int n = 0; n < 2; n++) {
            int ql = 64 * n, qhoff = 128 + 32 * n, sc = 192 + 8 * n;
            for (int h = 0; h < 2; h++) {
                const uint8_t *lo0 = b + ql + 16 * h, *lo1 = b + ql + 32 + 16 * h, *hi = b + qhoff + 16 * h;
                int base = 128 * n + 16 * h;
                for (int k = 0; k < 4; k++) {
                    float s = (float)(int8_t)b[sc + h + 2 * k];
                    float ds = d * s;
                    for (int i = 0; i < 16; i++) {
                        int q;
                        if (k == 0) q = (lo0[i] & 0xf) | ((hi[i] & 3) << 4);
                        else if (k == 1) q = (lo1[i] & 0xf) | (((hi[i] >> 2) & 3) << 4);
                        else if (k == 2) q = (lo0[i] >> 4) | (((hi[i] >> 4) & 3) << 4);
                        else q = (lo1[i] >> 4) | (((hi[i] >> 6) & 3) << 4);
                        v[i] = ds * ((float)q - 32.0f);
                    }
                    put(dot, dst, x, acc, base + 32 * k, v);
                }
            }
        }
    }
}

/* GGUFMatrix.each_block / blocks (gguf.mojo:388-434) */
static float gguf_row(int t, const uint8_t *p, int64_t cols, float *dst, const float *x, int dot) {
    float acc[L16] = {0};
    if (t == GGML_F32 || t == GGML_F16) {
        float v[L16];
        for (int64_t i = 0; i < cols; i += 16) {
            for (int l = 0; l < 16; l++) {
                if (t == GGML_F32) {
                    float f;
                    memcpy(&f, p + 4 * (i + l), 4);
                    v[l] = f;
                } else {
                    v[l] = f16_at(p, (int)(2 * (i + l)));
                }
            }
            put(dot, dst ? dst + i : NULL, x ? x + i : NULL, acc, 0, v);
        }
        return red16(acc);
    }
    int bs = orc_gguf_block_size(t), bb = orc_gguf_block_bytes(t);
    for (int64_t blk = 0; blk < cols / bs; blk++)
        gguf_block(t, dot, p + blk * bb, dst ? dst + blk * bs : NULL, x ? x + blk * bs : NULL, acc);
    return red16(acc);
}
void orc_gguf_dequant_row(int t, const uint8_t *row, int64_t cols, float *dst) { (void)gguf_row(t, row, cols, dst, NULL, 0); }
/* Every row of a GGUF matrix (rows of row_bytes each) into dst[rows, cols]. */
void orc_gguf_dequant_rows(int t, const uint8_t *blocks, int64_t rows, int64_t row_bytes, int64_t cols, float *dst) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int64_t r = 0; r < rows; r++) (void)gguf_row(t, blocks + r * row_bytes, cols, dst + r * cols, NULL, 0);
}
float orc_gguf_dot_row(int t, const uint8_t *row, int64_t cols, const float *x) { return gguf_row(t, row, cols, NULL, x, 1); }

/* q6_k_i16 (gguf.mojo:322-336): weights 128n + 32k .. +31 as (q - 32) * scale. */
static void q6_k_i16(const uint8_t *b, int n, int k, int16_t *out) {
    const uint8_t *L = b + 64 * n + (k % 2 ? 32 : 0), *H = b + 128 + 32 * n;
    for (int j = 0; j < 32; j++) {
        int lo = k >= 2 ? (L[j] >> 4) : (L[j] & 0xf);
        int q = lo | (((H[j] >> (2 * k)) & 3) << 4);
        int s = (int8_t)b[192 + 8 * n + 2 * k + (j < 16 ? 0 : 1)];
        out[j] = (int16_t)((q - 32) * s);
    }
}

int orc_gguf_has_i16(int t) { return t == GGML_Q6_K || t == GGML_Q8_0; } /* gguf.mojo:456-457 */
int orc_gguf_group_size(int t) { return t == GGML_Q6_K ? 256 : 32; }  /* 459-460 */

/* GGUFMatrix.dot_row_i16 (gguf.mojo:462-487) */
float orc_gguf_dot_row_i16(int t, const uint8_t *p, int64_t cols, const int16_t *xq) {
    float accf[L16] = {0};
    if (t == GGML_Q8_0) {
        for (int64_t blk = 0; blk < cols / 32; blk++) {
            const uint8_t *b = p + blk * 34;
            int16_t w[32];
            for (int j = 0; j < 32; j++) w[j] = (int16_t)(int8_t)b[2 + j];
            int32_t acc[L16] = {0};
            dot_pairs(acc, xq + blk * 32, w);
            float d = f16_at(b, 0);
            for (int i = 0; i < L16; i++) accf[i] = fmaf((float)acc[i], d, accf[i]);
        }
        return red16(accf);
    }
    for (int64_t sb = 0; sb < cols / 256; sb++) {
        const uint8_t *b = p + sb * 210;
        int32_t acc[L16] = {0};
        int16_t w[32];
        for (int n = 0; n < 2; n++)
            for (int k = 0; k < 4; k++) {
                q6_k_i16(b, n, k, w);
                dot_pairs(acc, xq + sb * 256 + 128 * n + 32 * k, w);
            }
        float d = f16_at(b, 208);
        for (int i = 0; i < L16; i++) accf[i] = fmaf((float)acc[i], d, accf[i]);
    }
    return red16(accf);
}

/* GGUFMatrix.unpack_row_i16 (gguf.mojo:489-505) */
void orc_gguf_unpack_row_i16(int t, const uint8_t *p, int64_t cols, int16_t *dst, float *scales) {
    if (t == GGML_Q8_0) {
        for (int64_t blk = 0; blk < cols / 32; blk++) {
            const uint8_t *b = p + blk * 34;
            for (int j = 0; j < 32; j++) dst[blk * 32 + j] = (int16_t)(int8_t)b[2 + j];
            scales[blk] = f16_at(b, 0);
        }
        return;
    }
    for (int64_t sb = 0; sb < cols / 256; sb++) {
        const uint8_t *b = p + sb * 210;
        for (int n = 0; n < 2; n++)
            for (int k = 0; k < 4; k++) q6_k_i16(b, n, k, dst + sb * 256 + 128 * n + 32 * k);
        scales[sb] = f16_at(b, 208);
    }
}

/* matmul_rows (kernels.mojo:285-349) over a QuantMatrix with A16 = 0
 * (OUT_MAJOR, tensor.mojo:293; linear's branch, kernels.mojo:670-671):
 * out[T, OUT] (+)= act(x @ w^T + b).  T == 1: dot_row (row_op) + b, finish
 * (301-312).  T > 1: tiles of TN = 32 rows dequantized (dequant_row) and
 * multiplied by mm_tile (52-85: one float32 FMA chain over i per output,
 * then + b, store_out); the last OUT % 32 rows by rows_dot (352-397: 16-lane
 * FMA partials over i, reduce_add, + b).  The vector width is taken as 16
 * lanes (simd_width_of[float32] with AVX-512). */
void orc_qm_matmul_rows(float *out, const float *x, const orc_qm *w, const float *b, int64_t T, int64_t IN,
                        int64_t OUT, int flags) {
    if (T == 1) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
        for (int64_t o = 0; o < OUT; o++) {
            float r = orc_qm_dot_row(w, o, x);
            if (flags & EPI_BIAS) r += b[o];
            finish(out, o, r, flags);
        }
        return;
    }
    const int64_t TN = 32, full = OUT / TN;
#pragma omp parallel for schedule(dynamic) num_threads(g_threads) if (g_threads > 1)
    for (int64_t o = 0; o < OUT; o++) {
        float *row = (float *)malloc(sizeof(float) * (size_t)IN);
        orc_qm_dequant_row(w, o, row);
        const float bias = (flags & EPI_BIAS) ? b[o] : 0.0f;
        for (int64_t t = 0; t < T; t++) {
            const float *xt = x + t * IN;
            float r;
            if (o < full * TN) { /* mm_tile */
                r = 0.0f;
                for (int64_t i = 0; i < IN; i++) r = fmaf(xt[i], row[i], r);
                r += bias;
            } else { /* rows_dot */
                float d[L16] = {0};
                for (int64_t i = 0; i < IN; i += L16)
                    for (int l = 0; l < L16; l++) d[l] = fmaf(xt[i + l], row[i + l], d[l]);
                r = red16(d) + bias;
            }
            finish(out, t * OUT + o, r, flags);
        }
        free(row);
    }
}

/* matmul_rows T == 1 (kernels.mojo:301-312) / linear_team OUT_MAJOR branch
 * (817-826): the GGUF decode GEMV, out[o] (+)= act(dot_row(o, x) + b[o]). */
void orc_gguf_gemv(int t, const uint8_t *w, int64_t rows, int64_t cols, const float *x, const float *b, float *out,
                   int flags) {
    int64_t rb = cols / orc_gguf_block_size(t) * orc_gguf_block_bytes(t);
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int64_t o = 0; o < rows; o++) {
        float r = orc_gguf_dot_row(t, w + o * rb, cols, x);
        if (flags & EPI_BIAS) r += b[o];
        finish(out, o, r, flags);
    }
}

/* head_i16 (kernels.mojo:693-736) for Q6_K / Q8_0: logits[T, V]. */
void orc_gguf_head_i16(int t, const uint8_t *w, int64_t V, int64_t C, const float *h, int64_t T, float *logits) {
    int16_t *xq = (int16_t *)malloc(sizeof(int16_t) * (size_t)(T * C));
    float *sx = (float *)malloc(sizeof(float) * (size_t)T);
    orc_quantize_rows(h, T, C, xq, sx);
    int64_t G = orc_gguf_group_size(t);
    int64_t rb = C / orc_gguf_block_size(t) * orc_gguf_block_bytes(t);
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int64_t v = 0; v < V; v++) {
        if (T == 1) {
            logits[v] = orc_gguf_dot_row_i16(t, w + v * rb, C, xq) * sx[0];
            continue;
        }
        int16_t *row = (int16_t *)malloc(sizeof(int16_t) * (size_t)C);
        float *rs = (float *)malloc(sizeof(float) * (size_t)(C / G));
        orc_gguf_unpack_row_i16(t, w + v * rb, C, row, rs);
        for (int64_t tt = 0; tt < T; tt++) logits[tt * V + v] = dot1_i16(row, rs, xq + tt * C, C, G) * sx[tt];
        free(row);
        free(rs);
    }
    free(xq);
    free(sx);
}

/* ------------------------------------------------------------------------ */
/* LayerNorm and the int8 KV cache (kernels.mojo:179-210; kvcache.mojo)     */
/* ------------------------------------------------------------------------ */

/* layernorm (kernels.mojo:179-197), 16-lane partial sums. */
void orc_layernorm(float *out, const float *x, const float *w, const float *b, int64_t T, int64_t C) {
    for (int64_t t = 0; t < T; t++) {
        const float *xr = x + t * C;
        float *o = out + t * C;
        float s[L16] = {0}, sq[L16] = {0};
        for (int64_t i = 0; i < C; i += 16)
            for (int l = 0; l < 16; l++) s[l] += xr[i + l];
        float mean = red16(s) / (float)C;
        for (int64_t i = 0; i < C; i += 16)
            for (int l = 0; l < 16; l++) {
                float d = xr[i + l] - mean;
                sq[l] += d * d;
            }
        float rstd = 1.0f / sqrtf(red16(sq) / (float)C + 1e-5f);
        for (int64_t i = 0; i < C; i++) {
            float n = (xr[i] - mean) * rstd;
            o[i] = n * w[i] + b[i];
        }
    }
}

typedef struct {
    int32_t n_layer, max_t, n_head, head_dim;
    int8_t *k, *v;  /* [layer, pos, head, head_dim] */
    float *ks, *vs; /* [layer, pos, head] */
} orc_kv;

/* QuantKV.quantize (kvcache.mojo:320-331) with QMAX = 127. */
static float kv_quantize(const float *x, int n, int8_t *dst) {
    float mx = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        mx = a > mx ? a : mx;
    }
    float s = mx / 127.0f;
    if (s == 0.0f) s = 1.0f;
    float inv = 1.0f / s;
    for (int i = 0; i < n; i++) dst[i] = (int8_t)orc_to_int(orc_round_at(x[i] * inv, 2));
    return s;
}

/* QuantKV.store (kvcache.mojo:333-342) */
void orc_kv_store(orc_kv *kv, int layer, int pos, const float *k, const float *v) {
    for (int h = 0; h < kv->n_head; h++) {
        int64_t sl = ((int64_t)layer * kv->max_t + pos) * kv->n_head + h;
        int o = h * kv->head_dim;
        kv->ks[sl] = kv_quantize(k + o, kv->head_dim, kv->k + sl * kv->head_dim);
        kv->vs[sl] = kv_quantize(v + o, kv->head_dim, kv->v + sl * kv->head_dim);
    }
}

/* attend_float_one (kvcache.mojo:113-150) through QuantKV.score / add_value
 * (344-370): token t (position pos0 + t), head h, of `layer`; q from qkv row
 * t ([T, 3C]), output into row t of out ([T, C]).  HS must be a multiple of
 * 16. */
void orc_kv_attend_one(const orc_kv *kv, float *out, const float *qkv, int layer, int t, int h, int pos0) {
    int HS = kv->head_dim, C = kv->n_head * HS;
    float scale = 1.0f / sqrtf((float)HS);
    int npos = pos0 + t + 1;
    const float *q = qkv + (int64_t)t * 3 * C + h * HS;
    float *scores = (float *)malloc(sizeof(float) * (size_t)npos);
    float mx = -INFINITY;
    for (int s = 0; s < npos; s++) {
        int64_t sl = ((int64_t)layer * kv->max_t + s) * kv->n_head + h;
        const int8_t *kp = kv->k + sl * HS;
        float d[L16] = {0};
        for (int i = 0; i < HS; i += 16)
            for (int l = 0; l < 16; l++) d[l] += q[i + l] * (float)kp[i + l];
        float sc = red16(d) * kv->ks[sl] * scale;
        scores[s] = sc;
        mx = sc > mx ? sc : mx;
    }
    for (int s = 0; s < npos; s++) scores[s] = orc_exp(scores[s] - mx);
    float total = 0.0f;
    for (int s = 0; s < npos; s++) total += scores[s];
    float *o = out + (int64_t)t * C + h * HS;
    float *acc = (float *)calloc((size_t)HS, sizeof(float));
    for (int s = 0; s < npos; s++) {
        float p = scores[s] / total;
        int64_t sl = ((int64_t)layer * kv->max_t + s) * kv->n_head + h;
        const int8_t *vp = kv->v + sl * HS;
        float ps = p * kv->vs[sl];
        for (int i = 0; i < HS; i++) acc[i] = fmaf(ps, (float)vp[i], acc[i]);
    }
    for (int i = 0; i < HS; i++) o[i] = acc[i];
    free(acc);
    free(scores);
}

/* KVCache.attend (kvcache.mojo:62-79): every token and head. */
/* (CPU baseline: one head of one token at a position below ORC_FAST_MAXT) */
#define ORC_FAST_MAXT 1024
static void (*g_fast_attend)(const orc_kv *, float *, const float *, int, int, int) = NULL;
void orc_kv_attend(const orc_kv *kv, float *out, const float *qkv, int layer, int T, int pos0) {
    const int C = kv->n_head * kv->head_dim;
#pragma omp parallel for schedule(dynamic) num_threads(g_threads) if (g_threads > 1 && T * (pos0 + T) >= 256)
    for (int idx = 0; idx < kv->n_head * T; idx++) {
        const int t = idx / kv->n_head, h = idx % kv->n_head;
        if (g_fast_attend && kv->head_dim == 64 && pos0 + t < ORC_FAST_MAXT)
            g_fast_attend(kv, out + (int64_t)t * C, qkv + (int64_t)t * 3 * C, layer, h, pos0 + t);
        else
            orc_kv_attend_one(kv, out, qkv, layer, t, h, pos0);
    }
}

/* ------------------------------------------------------------------------ */
/* Integer attention: intmath.mojo (masked softmax in fixed point) and      */
/* int_attention.mojo (IntAttnKV).  The cache uses QuantKV's natural layout  */
/* [layer, pos, head, head_dim]; the reference's VNNI blocking changes no    */
/* arithmetic.                                                               */
/* ------------------------------------------------------------------------ */

#define IM_FB 16                       /* intmath.mojo:33 */
#define IM_MB 24                       /* :34 */
#define IM_MASKED INT32_MIN            /* :35 */
#define IM_D_CAP ((int64_t)1 << 31)    /* :37 */
#define IA_KS 24                       /* int_attention.mojo:62 */
#define IA_SF 16                       /* :63 */

/* exp_multiplier (intmath.mojo:50-52) */
int64_t orc_exp_multiplier(double scale) {
    return (int64_t)(scale * 1.4426950408889634 * (double)((int64_t)1 << (IM_FB + IM_MB)) + 0.5);
}

/* exp2_neg (intmath.mojo:55-67) for one lane: 2^(-d scale log2 e) in Q30. */
int64_t orc_exp2_neg(int64_t d, int64_t mult) {
    const int64_t C0 = 1073741824, C1 = -742598100, C2 = 248207216, C3 = -42480028; /* :42-45 */
    int64_t y = ((d < IM_D_CAP ? d : IM_D_CAP) * mult) >> IM_MB;
    int64_t q = y >> IM_FB;
    int64_t r = y & (((int64_t)1 << IM_FB) - 1);
    int64_t p = C3;
    p = ((p * r) >> IM_FB) + C2;
    p = ((p * r) >> IM_FB) + C1;
    p = ((p * r) >> IM_FB) + C0;
    return q >= 31 ? 0 : p >> (q < 63 ? q : 63);
}

/* masked_exp (intmath.mojo:96-123): e_i in Q30 for i < n (0 when masked or
 * i >= n, up to n rounded to 16), returns the int64 sum. */
int64_t orc_masked_exp(const int32_t *x, const int32_t *mask, int has_mask, int n, int64_t mult, int32_t *e) {
    int nr = (n + 15) / 16 * 16;
    int64_t m = INT64_MIN;
    for (int i = 0; i < n; i++) {
        if (has_mask && mask[i] == IM_MASKED) continue;
        int64_t v = (int64_t)x[i] + (has_mask ? (int64_t)mask[i] : 0);
        m = v > m ? v : m;
    }
    int64_t total = 0;
    for (int i = 0; i < nr; i++) {
        int64_t ev = 0;
        if (i < n && !(has_mask && mask[i] == IM_MASKED)) {
            int64_t v = (int64_t)x[i] + (has_mask ? (int64_t)mask[i] : 0);
            ev = orc_exp2_neg(m - v, mult);
        }
        if (e) e[i] = (int32_t)ev;
        total += ev;
    }
    return total;
}

/* masked_softmax (intmath.mojo:126-140): Q15 probabilities. */
void orc_masked_softmax(const int32_t *x, const int32_t *mask, int has_mask, int n, int64_t mult, uint16_t *probs) {
    int nr = (n + 15) / 16 * 16;
    int32_t *e = (int32_t *)malloc(sizeof(int32_t) * (size_t)nr);
    int64_t t = orc_masked_exp(x, mask, has_mask, n, mult, e);
    int64_t inv = t > 0 ? ((int64_t)1 << 61) / t : 0;
    for (int i = 0; i < nr; i++) probs[i] = (uint16_t)(((int64_t)e[i] * inv + ((int64_t)1 << 45)) >> 46);
    free(e);
}

typedef struct {
    int32_t n_layer, max_t, n_head, head_dim;
    int8_t *k, *v;     /* [layer, pos, head, head_dim] */
    int32_t *kq, *vq;  /* scales * 2^24, [layer, pos, head] */
} orc_ikv;

/* IntAttnKV.quantize_head (int_attention.mojo:140-168): int8 codes, and the
 * scale * 2^24 as an int32. */
static int32_t ikv_quantize(const float *x, int n, int8_t *dst) {
    float mx = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        mx = a > mx ? a : mx;
    }
    float s = mx / 127.0f;
    if (s == 0.0f) s = 1.0f;
    float inv = 1.0f / s;
    for (int i = 0; i < n; i++) dst[i] = (int8_t)orc_to_int(orc_round(x[i] * inv));
    return (int32_t)(int64_t)orc_round_d((double)s * (double)(1 << IA_KS));
}

/* IntAttnKV.store (int_attention.mojo:132-138) */
void orc_ikv_store(orc_ikv *kv, int layer, int pos, const float *k, const float *v) {
    for (int h = 0; h < kv->n_head; h++) {
        int64_t sl = ((int64_t)layer * kv->max_t + pos) * kv->n_head + h;
        kv->kq[sl] = ikv_quantize(k + h * kv->head_dim, kv->head_dim, kv->k + sl * kv->head_dim);
        kv->vq[sl] = ikv_quantize(v + h * kv->head_dim, kv->head_dim, kv->v + sl * kv->head_dim);
    }
}

/* IntAttnKV.attend_one (int_attention.mojo:170-269): token t (position
 * pos0 + t) and head h; q from qkv row t ([T, 3C]), output into row t of
 * out ([T, C]). */
void orc_ikv_attend_one(const orc_ikv *kv, float *out, const float *qkv, int layer, int t, int h, int pos0) {
    const int HS = kv->head_dim, C = kv->n_head * HS;
    const int64_t mult = orc_exp_multiplier(1.0 / (double)(1 << IA_SF));
    const int npos = pos0 + t + 1, nr = (npos + 15) / 16 * 16;
    const float *q = qkv + (int64_t)t * 3 * C + h * HS;
    const int64_t base = (int64_t)layer * kv->max_t * kv->n_head + h; /* slot of position 0 */
    const int64_t stride = kv->n_head;
    /* 1. query -> int16 */
    float mq = 0.0f;
    for (int d = 0; d < HS; d++) mq = fabsf(q[d]) > mq ? fabsf(q[d]) : mq;
    float sq = mq / 32767.0f;
    if (sq == 0.0f) sq = 1.0f;
    float invq = 1.0f / sq;
    int16_t *qi = (int16_t *)malloc(sizeof(int16_t) * (size_t)HS);
    for (int d = 0; d < HS; d++) qi[d] = (int16_t)orc_to_int(orc_round(q[d] * invq));
    const int64_t qm = (int64_t)orc_round_d((double)sq / sqrt((double)HS) * (double)((int64_t)1 << (IA_SF + IA_KS)));
    /* 2-3. fixed-point scores (positions past npos are masked below) */
    int32_t *scores = (int32_t *)calloc((size_t)nr, sizeof(int32_t));
    int32_t *e = (int32_t *)calloc((size_t)nr, sizeof(int32_t));
    for (int s = 0; s < npos; s++) {
        const int8_t *kp = kv->k + (base + s * stride) * HS;
        int32_t acc = 0;
        for (int d = 0; d < HS; d++) acc += (int32_t)qi[d] * (int32_t)kp[d];
        int64_t t1 = ((int64_t)acc * kv->kq[base + s * stride] + ((int64_t)1 << (IA_KS - 1))) >> IA_KS;
        int64_t sfix = (t1 * qm + ((int64_t)1 << (IA_KS - 1))) >> IA_KS;
        scores[s] = (int32_t)sfix;
    }
    /* 4. unnormalized integer softmax */
    int64_t total = orc_masked_exp(scores, NULL, 0, npos, mult, e);
    /* 5. value scales folded into int16 weights */
    int64_t vmax = 0;
    for (int s = 0; s < npos; s++) vmax = kv->vq[base + s * stride] > vmax ? kv->vq[base + s * stride] : vmax;
    float *o = out + (int64_t)t * C + h * HS;
    if (vmax == 0 || total == 0) {
        for (int d = 0; d < HS; d++) o[d] = 0.0f;
    } else {
        const int64_t inv47 = ((int64_t)1 << 47) / vmax;
        int16_t *w = (int16_t *)calloc((size_t)nr + 2, sizeof(int16_t));
        for (int s = 0; s < npos; s++) {
            int64_t r16 = ((int64_t)kv->vq[base + s * stride] * inv47) >> 31;
            int64_t ww = ((int64_t)e[s] * r16 + ((int64_t)1 << 30)) >> 31;
            if (ww > 32767) ww = 32767;
            w[s] = e[s] == 0 ? 0 : (int16_t)ww;
        }
        /* weighted sums, int32 per 128 position pairs, then float */
        float *accf = (float *)calloc((size_t)HS, sizeof(float));
        int32_t *accv = (int32_t *)malloc(sizeof(int32_t) * (size_t)HS);
        const int npairs = (npos + 1) / 2;
        for (int seg = 0; seg < npairs; seg += 128) {
            memset(accv, 0, sizeof(int32_t) * (size_t)HS);
            int pend = seg + 128 < npairs ? seg + 128 : npairs;
            for (int pp = seg; pp < pend; pp++) {
                for (int j = 0; j < 2; j++) {
                    int s = 2 * pp + j;
                    if (s >= npos) continue; /* weight 0 */
                    const int8_t *vp = kv->v + (base + s * stride) * HS;
                    for (int d = 0; d < HS; d++) accv[d] = (int32_t)((uint32_t)accv[d] + (uint32_t)((int32_t)w[s] * vp[d]));
                }
            }
            for (int d = 0; d < HS; d++) accf[d] += (float)accv[d];
        }
        /* 6. back to float */
        const float fs = (float)((double)vmax * (double)(1 << 15) / ((double)(1 << IA_KS) * (double)total));
        for (int d = 0; d < HS; d++) o[d] = accf[d] * fs;
        free(accf);
        free(accv);
        free(w);
    }
    free(qi);
    free(scores);
    free(e);
}

/* KVCache.attend over IntAttnKV (kvcache.mojo:62-79): every token and head. */
void orc_ikv_attend(const orc_ikv *kv, float *out, const float *qkv, int layer, int T, int pos0) {
#pragma omp parallel for schedule(dynamic) num_threads(g_threads) if (g_threads > 1 && T * (pos0 + T) >= 256)
    for (int idx = 0; idx < kv->n_head * T; idx++)
        orc_ikv_attend_one(kv, out, qkv, layer, idx / kv->n_head, idx % kv->n_head, pos0);
}

/* ------------------------------------------------------------------------ */
/* GPT-2 (gpt2t.mojo:74-118, 198-609, 777-797)                              */
/* ------------------------------------------------------------------------ */

#define G_NL 12
#define G_NH 12
#define G_C 768
#define G_HS 64
#define G_MAXT 1024
_Static_assert(G_MAXT == ORC_FAST_MAXT, "the fast attention's score buffer holds G_MAXT positions");
#define G_V 50257

/* Rng (gpt2t.mojo:777-789): xorshift64*. */
typedef struct {
    uint64_t state;
} orc_rng;
void orc_rng_init(orc_rng *r, int64_t seed) { r->state = (uint64_t)seed * 0x9E3779B97F4A7C15ull + 1; }
float orc_rng_uniform(orc_rng *r) {
    r->state ^= r->state >> 12;
    r->state ^= r->state << 25;
    r->state ^= r->state >> 27;
    uint64_t x = (r->state * 0x2545F4914F6CDD1Dull) >> 40;
    return (float)x / (float)(1 << 24);
}

/* argmax (gpt2t.mojo:792-797): the first maximum wins (strict >). */
int64_t orc_argmax(const float *logits, int64_t V) {
    int64_t best = 0;
    for (int64_t v = 1; v < V; v++)
        if (logits[v] > logits[best]) best = v;
    return best;
}

/* Per-layer float32 vectors, in gpt2t.mojo's VEC_NAMES order (108-118). */
enum { LN1_W, LN1_B, QKV_B, PROJ_B, LN2_W, LN2_B, FC_B, FCPROJ_B, N_VECS };

typedef struct {
    orc_qm wte;              /* E: [V, C] int8 per-channel A16 (the tied embedding and head) */
    orc_qm mats[G_NL * 4];   /* W: qkv, proj, fc, fcproj per layer ([OUT, IN]) */
    float *vecs[G_NL * N_VECS];
    float *wpe, *lnf_w, *lnf_b;
    orc_kv kv;
    int integer; /* 1: IntAttnKV over the same storage (int32 scales in ks / vs) */
    float *x, *xn, *qkv, *att, *fc, *logits;
    int16_t *capture; /* one-token forwards: each linear's int16 input codes, [49][3072] */
} orc_gpt2;

static void qm_alloc(orc_qm *m, int bits, int group, int sym, int a16, int64_t n, int64_t k) {
    m->bits = bits;
    m->sym = sym;
    m->a16 = a16;
    m->group = group;
    int64_t g = group == 0 ? k : group;
    m->data = (uint8_t *)malloc((size_t)(n * k * bits / 8));
    m->scale = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(n * k / g));
    m->zp = (uint8_t *)malloc((size_t)(n * k / g));
}
static void qm_free(orc_qm *m) {
    free(m->data);
    free(m->scale);
    free(m->zp);
}

/* load_model (gpt2t.mojo:579-609) from float32 tensors in Hugging Face
 * layout.  params: wte [V, C], wpe [MAX_T, C], ln_f.weight, ln_f.bias, then
 * per layer the 12 tensors ln_1.weight, ln_1.bias, attn.c_attn.weight
 * [C, 3C], attn.c_attn.bias, attn.c_proj.weight [C, C], attn.c_proj.bias,
 * ln_2.weight, ln_2.bias, mlp.c_fc.weight [C, 4C], mlp.c_fc.bias,
 * mlp.c_proj.weight [4C, C], mlp.c_proj.bias.  Layers in QuantMatrix[bits,
 * group, sym, A16=True], the head in E = QuantMatrix[8, 0, False, True]
 * (HEAD8_A16, gpt2t.mojo:1234), the cache QuantKV[8]. */
orc_gpt2 *orc_gpt2_new_fmt(const float *const *params, int bits, int group, int sym, int a16, int e_bits,
                           int e_group, int e_sym, int e_a16);
orc_gpt2 *orc_gpt2_new(const float *const *params, int bits, int group, int sym) {
    return orc_gpt2_new_fmt(params, bits, group, sym, 1, 8, 0, 0, 1);
}

/* Model[W, E] for any QuantMatrix layer format W = [bits, group, sym, a16]
 * and head format E = [e_bits, e_group, e_sym, e_a16] (run_quantized,
 * gpt2t.mojo:1282-1292). */
orc_gpt2 *orc_gpt2_new_fmt(const float *const *params, int bits, int group, int sym, int a16, int e_bits,
                           int e_group, int e_sym, int e_a16) {
    orc_gpt2 *m = (orc_gpt2 *)calloc(1, sizeof(orc_gpt2));
    qm_alloc(&m->wte, e_bits, e_group, e_sym, e_a16, G_V, G_C);
    orc_qm_from_f32(&m->wte, params[0], G_V, G_C, 0);
    static const int64_t rows[4] = {G_C, G_C, G_C, 4 * G_C}, cols[4] = {3 * G_C, G_C, 4 * G_C, G_C};
    static const int mat_idx[4] = {2, 4, 8, 10};
    static const int vec_idx[N_VECS] = {0, 1, 3, 5, 6, 7, 9, 11};
    static const int64_t vec_len[N_VECS] = {G_C, G_C, 3 * G_C, G_C, G_C, G_C, 4 * G_C, G_C};
    for (int l = 0; l < G_NL; l++) {
        const float *const *lp = params + 4 + 12 * l;
        for (int j = 0; j < 4; j++) {
            orc_qm *q = &m->mats[l * 4 + j];
            qm_alloc(q, bits, group, sym, a16, cols[j], rows[j]);
            orc_qm_from_f32(q, lp[mat_idx[j]], rows[j], cols[j], 1);
        }
        for (int s = 0; s < N_VECS; s++) {
            m->vecs[l * N_VECS + s] = (float *)malloc(sizeof(float) * (size_t)vec_len[s]);
            memcpy(m->vecs[l * N_VECS + s], lp[vec_idx[s]], sizeof(float) * (size_t)vec_len[s]);
        }
    }
    m->wpe = (float *)malloc(sizeof(float) * G_MAXT * G_C);
    memcpy(m->wpe, params[1], sizeof(float) * G_MAXT * G_C);
    m->lnf_w = (float *)malloc(sizeof(float) * G_C);
    m->lnf_b = (float *)malloc(sizeof(float) * G_C);
    memcpy(m->lnf_w, params[2], sizeof(float) * G_C);
    memcpy(m->lnf_b, params[3], sizeof(float) * G_C);
    m->kv.n_layer = G_NL;
    m->kv.max_t = G_MAXT;
    m->kv.n_head = G_NH;
    m->kv.head_dim = G_HS;
    size_t nkv = (size_t)G_NL * G_MAXT * G_C, ns = (size_t)G_NL * G_MAXT * G_NH;
    m->kv.k = (int8_t *)calloc(nkv, 1);
    m->kv.v = (int8_t *)calloc(nkv, 1);
    m->kv.ks = (float *)calloc(ns, sizeof(float));
    m->kv.vs = (float *)calloc(ns, sizeof(float));
    m->x = (float *)malloc(sizeof(float) * G_MAXT * G_C);
    m->xn = (float *)malloc(sizeof(float) * G_MAXT * G_C);
    m->qkv = (float *)malloc(sizeof(float) * G_MAXT * 3 * G_C);
    m->att = (float *)malloc(sizeof(float) * G_MAXT * G_C);
    m->fc = (float *)malloc(sizeof(float) * G_MAXT * 4 * G_C);
    m->logits = (float *)malloc(sizeof(float) * G_V);
    return m;
}

void orc_gpt2_free(orc_gpt2 *m) {
    if (!m) return;
    qm_free(&m->wte);
    for (int i = 0; i < G_NL * 4; i++) qm_free(&m->mats[i]);
    for (int i = 0; i < G_NL * N_VECS; i++) free(m->vecs[i]);
    free(m->wpe);
    free(m->lnf_w);
    free(m->lnf_b);
    free(m->kv.k);
    free(m->kv.v);
    free(m->kv.ks);
    free(m->kv.vs);
    free(m->x);
    free(m->xn);
    free(m->qkv);
    free(m->att);
    free(m->fc);
    free(m->logits);
    free(m);
}

const orc_qm *orc_gpt2_mat(const orc_gpt2 *m, int i) { return i < 0 ? &m->wte : &m->mats[i]; }
const orc_kv *orc_gpt2_kv(const orc_gpt2 *m) { return &m->kv; }

/* --attention int (gpt2t.mojo:1251-1257): IntAttnKV instead of QuantKV[8].
 * The cache must be empty (set before the first forward). */
void orc_gpt2_set_attention(orc_gpt2 *m, int integer) { m->integer = integer; }

static orc_ikv gpt2_ikv(const orc_gpt2 *m) {
    orc_ikv k = {m->kv.n_layer, m->kv.max_t, m->kv.n_head, m->kv.head_dim,
                 m->kv.k,       m->kv.v,     (int32_t *)m->kv.ks, (int32_t *)m->kv.vs};
    return k;
}
float *orc_gpt2_act(orc_gpt2 *m, int which) {
    switch (which) {
    case 0: return m->x;
    case 1: return m->xn;
    case 2: return m->qkv;
    case 3: return m->att;
    case 4: return m->fc;
    default: return m->logits;
    }
}

/* kernels.linear / head (kernels.mojo:655-690) for a QuantMatrix: the
 * integer kernels for A16, matmul_rows otherwise. */
static void linear(float *out, const float *x, const orc_qm *w, const float *b, int64_t T, int64_t IN, int64_t OUT,
                   int flags) {
    if (w->a16)
        orc_matmul_rows_a16(out, x, w, b, T, IN, OUT, flags);
    else
        orc_qm_matmul_rows(out, x, w, b, T, IN, OUT, flags);
}

/* Test hook: with codes set, one-token forwards store quantize_rows' codes
 * of every linear's input (slot 4 l + k: qkv, proj, fc, fcproj; 48 the
 * head; 3072 entries a slot). */
void orc_gpt2_set_capture(orc_gpt2 *m, int16_t *codes) { m->capture = codes; }
static void capture(orc_gpt2 *m, int T, int slot, const float *x, int64_t IN) {
    float sx;
    if (m->capture && T == 1) orc_quantize_rows(x, 1, IN, m->capture + (int64_t)slot * 3072, &sx);
}

/* Model.blocks (gpt2t.mojo:485-571): embed tokens at pos0.., all layers. */
static void gpt2_blocks(orc_gpt2 *m, const int64_t *tokens, int T, int pos0) {
    const int C = G_C;
    for (int t = 0; t < T; t++) { /* 495-502 */
        float *xt = m->x + (int64_t)t * C;
        orc_qm_dequant_row(&m->wte, tokens[t], xt);
        const float *p = m->wpe + (int64_t)(pos0 + t) * C;
        for (int i = 0; i < C; i++) xt[i] = xt[i] + p[i];
    }
    for (int l = 0; l < G_NL; l++) {
        orc_qm *w = &m->mats[l * 4];
        float **v = &m->vecs[l * N_VECS];
        orc_layernorm(m->xn, m->x, v[LN1_W], v[LN1_B], T, C);
        capture(m, T, 4 * l, m->xn, C);
        linear(m->qkv, m->xn, &w[0], v[QKV_B], T, C, 3 * C, EPI_BIAS);
        if (m->integer) {
            orc_ikv ik = gpt2_ikv(m);
            for (int t = 0; t < T; t++) {
                const float *row = m->qkv + (int64_t)t * 3 * C;
                orc_ikv_store(&ik, l, pos0 + t, row + C, row + 2 * C);
            }
            orc_ikv_attend(&ik, m->att, m->qkv, l, T, pos0);
        } else {
            for (int t = 0; t < T; t++) {
                const float *row = m->qkv + (int64_t)t * 3 * C;
                orc_kv_store(&m->kv, l, pos0 + t, row + C, row + 2 * C);
            }
            orc_kv_attend(&m->kv, m->att, m->qkv, l, T, pos0);
        }
        capture(m, T, 4 * l + 1, m->att, C);
        linear(m->x, m->att, &w[1], v[PROJ_B], T, C, C, EPI_BIAS | EPI_RESID);
        orc_layernorm(m->xn, m->x, v[LN2_W], v[LN2_B], T, C);
        capture(m, T, 4 * l + 2, m->xn, C);
        linear(m->fc, m->xn, &w[2], v[FC_B], T, C, 4 * C, EPI_BIAS | EPI_GELU);
        capture(m, T, 4 * l + 3, m->fc, 4 * C);
        linear(m->x, m->fc, &w[3], v[FCPROJ_B], T, 4 * C, C, EPI_BIAS | EPI_RESID);
    }
}

/* Model.forward (gpt2t.mojo:329-342) and Model.decode (350-447): runs the
 * tokens at positions pos0.. and returns the last token's logits.  decode's
 * team arithmetic equals the region-per-call kernels' (kernels.mojo:743-747),
 * so one token goes through the same blocks() with T = 1. */
const float *orc_gpt2_forward(orc_gpt2 *m, const int64_t *tokens, int T, int pos0) {
    gpt2_blocks(m, tokens, T, pos0);
    const float *last = m->x + (int64_t)(T - 1) * G_C;
    orc_layernorm(m->xn, last, m->lnf_w, m->lnf_b, 1, G_C);
    capture(m, T, 4 * G_NL, m->xn, G_C);
    linear(m->logits, m->xn, &m->wte, NULL, 1, G_C, G_V, 0);
    return m->logits;
}

/* Model.forward_all (gpt2t.mojo:448-459): tokens from position 0, LN_f on
 * every row, the head on all T rows: logits[T, V], row t predicting t + 1. */
void orc_gpt2_forward_all(orc_gpt2 *m, const int64_t *tokens, int T, float *logits) {
    gpt2_blocks(m, tokens, T, 0);
    orc_layernorm(m->xn, m->x, m->lnf_w, m->lnf_b, T, G_C);
    linear(logits, m->xn, &m->wte, NULL, T, G_C, G_V, 0);
}

/* log_sum_exp (gpt2t.mojo:1027-1036): the row maximum, then exp(l - max) in
 * float32 summed in float64 in vocabulary order. */
static double log_sum_exp(const float *row, int V) {
    float mx = row[0];
    for (int v = 1; v < V; v++) mx = row[v] > mx ? row[v] : mx;
    double s = 0.0;
    for (int v = 0; v < V; v++) s += (double)expf(row[v] - mx);
    return (double)mx + log(s);
}

/* score_rows (gpt2t.mojo:1040-1095) for rows r0..r1-1: stats[k * ld + r]
 * for k = NLL, and with base != NULL NLL_BASE, AGREE, KL, DIFF_MAX,
 * DIFF_SUM. */
void orc_score_rows(double *stats, int64_t ld, const float *logits, const float *base, const int64_t *targets,
                    int r0, int r1, int V) {
    for (int r = r0; r < r1; r++) {
        const float *lm = logits + (int64_t)r * V;
        const int64_t target = targets[r];
        const double lse = log_sum_exp(lm, V);
        stats[r] = lse - (double)lm[target];
        if (!base) continue;
        const float *lb = base + (int64_t)r * V;
        const double lse_b = log_sum_exp(lb, V);
        double kl = 0.0, dmax = 0.0, dsum = 0.0;
        int best = 0, best_b = 0;
        for (int v = 0; v < V; v++) {
            const double lpb = (double)lb[v] - lse_b;
            kl += exp(lpb) * (lpb - ((double)lm[v] - lse));
            const double d = fabs((double)lm[v] - (double)lb[v]);
            dmax = d > dmax ? d : dmax;
            dsum += d;
            if (lm[v] > lm[best]) best = v;
            if (lb[v] > lb[best_b]) best_b = v;
        }
        stats[1 * ld + r] = lse_b - (double)lb[target];
        stats[2 * ld + r] = best == best_b ? 1.0 : 0.0;
        stats[3 * ld + r] = kl;
        stats[4 * ld + r] = dmax;
        stats[5 * ld + r] = dsum;
    }
}

/* generate's greedy loop (gpt2t.mojo:949-981 with -t 0): prompt, then up to
 * `steps` tokens (stopping at EOT 50256); returns the count generated.  The
 * decode loop runs steps - 1 forwards for steps tokens. */
int orc_gpt2_generate(orc_gpt2 *m, const int64_t *prompt, int n_prompt, int steps, int64_t *out_tokens) {
    const float *logits = orc_gpt2_forward(m, prompt, n_prompt, 0);
    int pos = n_prompt, generated = 0;
    for (int i = 0; i < steps; i++) {
        int64_t next = orc_argmax(logits, G_V);
        if (next == 50256) break;
        out_tokens[generated++] = next;
        if (generated == steps) break;
        logits = orc_gpt2_forward(m, &next, 1, pos);
        pos++;
    }
    return generated;
}

/* ------------------------------------------------------------------------ */
/* CPU baseline: the team decode (gpt2t.mojo:350-447) on AVX-512 VNNI        */
/* ------------------------------------------------------------------------ */
/* A restatement of the reference's decode as it runs on its own CPU: one
 * parallel region per token, a team of nt threads meeting at a spin-then-
 * yield barrier after each operation (team.mojo:36-82), thread 0 doing the
 * serial pieces (embedding, LayerNorm, quantize_rows / permute_x_i16, the
 * cache store), rows of every linear split into nt contiguous ranges
 * (linear_team, kernels.mojo:774-866), heads dealt round-robin.  The integer
 * dots run on VPDPWSSD (_mm512_dpwssd_epi32, the reference's dot_pairs,
 * tensor.mojo:34-46) for the BLOCKED int4-g32 rows (tensor.mojo:522-540)
 * and the int8 per-channel head (541-566, four rows at a time with the
 * next rows prefetched).  Every float operation is the scalar oracle's, in
 * its order, so the results are bit-identical to orc_gpt2_forward (tests/).
 * Without AVX-512 VNNI (checked by cpuid) the scalar lane emulation runs
 * instead and orc_cpu_vnni() reports 0. */
#include <cpuid.h>
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <time.h>

#define VNNI __attribute__((target("avx512f,avx512bw,avx512dq,avx512vl,avx512vnni,f16c,fma")))

/* cpuid leaf 7: AVX512F (EBX 16), AVX512DQ (17), AVX512BW (30), AVX512VL
 * (31), AVX512_VNNI (ECX 11); leaf 1: F16C (ECX 29), FMA (12), OSXSAVE
 * (27); XCR0 must enable the SSE, AVX and the three AVX-512 state parts. */
int orc_cpu_vnni(void) {
    unsigned a, b, c, d;
    if (!__get_cpuid(1, &a, &b, &c, &d)) return 0;
    if (!(c & (1u << 27)) || !(c & (1u << 29)) || !(c & (1u << 12))) return 0;
    unsigned lo, hi;
    __asm__ volatile("xgetbv" : "=a"(lo), "=d"(hi) : "c"(0));
    if ((lo & 0xE6u) != 0xE6u) return 0;
    if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return 0;
    const unsigned need_b = (1u << 16) | (1u << 17) | (1u << 30) | (1u << 31);
    return (b & need_b) == need_b && (c & (1u << 11)) ? 1 : 0;
}

/* dot_row_i16, BLOCKED branch (tensor.mojo:522-540): per 256-weight block
 * eight VPDPWSSD steps of 32 codes (low nibbles of the step's 16 bytes, then
 * high nibbles) against the permuted activations, then per lane
 * accf = fma(f32(acc) - zp * xs, scale, accf) with lane i in group i % 8. */
VNNI static float dot_blocked_vnni(const orc_qm *m, int64_t row, const int16_t *xp, const float *xs) {
    const uint8_t *p = m->data + row * m->k / 2;
    const int64_t gpr = m->k / 32;
    const __m128i nib = _mm_set1_epi8(0x0f);
    __m512 accf = _mm512_setzero_ps();
    for (int64_t blk = 0; blk < m->k / 256; blk++) {
        __m512i acc = _mm512_setzero_si512();
        for (int step = 0; step < 8; step++) {
            const __m128i b = _mm_loadu_si128((const __m128i *)(p + blk * 128 + step * 16));
            const __m256i lo = _mm256_cvtepu8_epi16(_mm_and_si128(b, nib));
            const __m256i hi = _mm256_cvtepu8_epi16(_mm_and_si128(_mm_srli_epi16(b, 4), nib));
            const __m512i u = _mm512_inserti64x4(_mm512_castsi256_si512(lo), hi, 1);
            acc = _mm512_dpwssd_epi32(acc, _mm512_loadu_si512((const void *)(xp + blk * 256 + step * 32)), u);
        }
        const int64_t g0 = row * gpr + blk * 8;
        const __m256i zp8 = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(m->zp + g0)));
        const __m512 zp = _mm512_cvtepi32_ps(_mm512_broadcast_i32x8(zp8));
        const __m512 sc = _mm512_broadcast_f32x8(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(m->scale + g0))));
        const __m512 t = _mm512_sub_ps(_mm512_cvtepi32_ps(acc), _mm512_mul_ps(zp, _mm512_loadu_ps(xs + blk * 16)));
        accf = _mm512_fmadd_ps(t, sc, accf);
    }
    float v[L16];
    _mm512_storeu_ps(v, accf);
    return red16(v);
}

/* dot_row_i16, int8 per-channel branch (tensor.mojo:541-566): codes - zp
 * as int16, VPDPWSSD over 32 inputs a step, then fma(f32(acc), scale, 0).
 * Four rows at a time share the activation loads (the reference's 4x
 * unroll), the rows eight ahead prefetched; a single row for the tail. */
VNNI static inline float ch8_finish(const orc_qm *m, int64_t row, __m512i acc) {
    const float s = orc_f16_to_f32(m->scale[row]);
    float v[L16];
    _mm512_storeu_ps(v, _mm512_fmadd_ps(_mm512_cvtepi32_ps(acc), _mm512_set1_ps(s), _mm512_setzero_ps()));
    return red16(v);
}
VNNI static inline __m512i ch8_step(const uint8_t *p, __m512i zp, __m512i xv, __m512i acc) {
    const __m512i w = _mm512_sub_epi16(_mm512_cvtepu8_epi16(_mm256_loadu_si256((const __m256i *)p)), zp);
    return _mm512_dpwssd_epi32(acc, xv, w);
}
VNNI static void dot_ch8_vnni4(const orc_qm *m, int64_t r, const int16_t *xq, float *out) {
    const int64_t K = m->k;
    const uint8_t *p0 = m->data + r * K, *p1 = p0 + K, *p2 = p1 + K, *p3 = p2 + K;
    const __m512i z0 = _mm512_set1_epi16((short)m->zp[r]), z1 = _mm512_set1_epi16((short)m->zp[r + 1]),
                  z2 = _mm512_set1_epi16((short)m->zp[r + 2]), z3 = _mm512_set1_epi16((short)m->zp[r + 3]);
    __m512i a0 = _mm512_setzero_si512(), a1 = a0, a2 = a0, a3 = a0;
    const char *pf = (const char *)(p0 + 8 * K);
    const int64_t pf_end = (m->n - r - 8) * K; /* bytes the prefetch may touch */
    for (int64_t k = 0; k < K; k += 32) {
        if (k * 4 < pf_end) _mm_prefetch(pf + 4 * k, _MM_HINT_T0);
        if (k * 4 + 64 < pf_end) _mm_prefetch(pf + 4 * k + 64, _MM_HINT_T0);
        const __m512i xv = _mm512_loadu_si512((const void *)(xq + k));
        a0 = ch8_step(p0 + k, z0, xv, a0);
        a1 = ch8_step(p1 + k, z1, xv, a1);
        a2 = ch8_step(p2 + k, z2, xv, a2);
        a3 = ch8_step(p3 + k, z3, xv, a3);
    }
    out[0] = ch8_finish(m, r, a0);
    out[1] = ch8_finish(m, r + 1, a1);
    out[2] = ch8_finish(m, r + 2, a2);
    out[3] = ch8_finish(m, r + 3, a3);
}
VNNI static float dot_ch8_vnni1(const orc_qm *m, int64_t r, const int16_t *xq) {
    const uint8_t *p = m->data + r * m->k;
    const __m512i z = _mm512_set1_epi16((short)m->zp[r]);
    __m512i a = _mm512_setzero_si512();
    for (int64_t k = 0; k < m->k; k += 32) a = ch8_step(p + k, z, _mm512_loadu_si512((const void *)(xq + k)), a);
    return ch8_finish(m, r, a);
}

/* quantize_rows (kernels.mojo:400-416) for one row, 16 values a step:
 * the same max, scale and product as orc_quantize_rows, and half-away
 * rounding built exactly as t = trunc(v), t + sign(v) where |v - t| >= 0.5
 * (roundf's result for every |v| < 2^23); ties are counted as the scalar
 * path counts them.  IN must be a multiple of 16. */
VNNI static void quantize_row_vnni(const float *x, int64_t IN, int16_t *xq, float *sx) {
    __m512 mxv = _mm512_setzero_ps();
    const __m512 absmask = _mm512_castsi512_ps(_mm512_set1_epi32(0x7fffffff));
    for (int64_t i = 0; i < IN; i += 16) mxv = _mm512_max_ps(mxv, _mm512_and_ps(_mm512_loadu_ps(x + i), absmask));
    const float mx = _mm512_reduce_max_ps(mxv);
    float s = mx / 32767.0f;
    if (s == 0.0f) s = 1.0f;
    *sx = s;
    const __m512 inv = _mm512_set1_ps(1.0f / s), half = _mm512_set1_ps(0.5f), one = _mm512_set1_ps(1.0f);
    const __m512 signmask = _mm512_castsi512_ps(_mm512_set1_epi32((int)0x80000000u));
    int64_t ties = 0;
    for (int64_t i = 0; i < IN; i += 16) {
        const __m512 v = _mm512_mul_ps(_mm512_loadu_ps(x + i), inv);
        const __m512 t = _mm512_roundscale_ps(v, _MM_FROUND_TO_ZERO | _MM_FROUND_NO_EXC);
        const __m512 d = _mm512_and_ps(_mm512_sub_ps(v, t), absmask);
        const __mmask16 up = _mm512_cmp_ps_mask(d, half, _CMP_GE_OQ);
        ties += __builtin_popcount((unsigned)_mm512_cmp_ps_mask(d, half, _CMP_EQ_OQ));
        const __m512 step = _mm512_or_ps(one, _mm512_and_ps(v, signmask));
        const __m512 r = _mm512_mask_add_ps(t, up, t, step);
        _mm256_storeu_si256((__m256i *)(xq + i), _mm512_cvtepi32_epi16(_mm512_cvttps_epi32(r)));
    }
    if (ties) __atomic_fetch_add(&g_ties[1], ties, __ATOMIC_RELAXED);
}

/* attend_float_one (kvcache.mojo:113-150) for head h of one token at
 * position pos, as orc_kv_attend_one computes it (the 16-lane score
 * partials, the scale products, the sequential total, the fma chain per
 * dimension), 16 values a step.  head_dim 64. */
VNNI static void attend_one_vnni(const orc_kv *kv, float *out, const float *qkv, int layer, int h, int pos) {
    const int HS = 64, C = kv->n_head * HS, npos = pos + 1;
    const float scale = 1.0f / sqrtf((float)HS);
    const float *q = qkv + h * HS;
    const __m512 q0 = _mm512_loadu_ps(q), q1 = _mm512_loadu_ps(q + 16), q2 = _mm512_loadu_ps(q + 32),
                 q3 = _mm512_loadu_ps(q + 48);
    float scores[G_MAXT];
    float mx = -INFINITY;
    for (int s = 0; s < npos; s++) {
        const int64_t sl = ((int64_t)layer * kv->max_t + s) * kv->n_head + h;
        const int8_t *kp = kv->k + sl * HS;
        __m512 d = _mm512_setzero_ps();
        d = _mm512_add_ps(d, _mm512_mul_ps(q0, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)kp)))));
        d = _mm512_add_ps(d, _mm512_mul_ps(q1, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(kp + 16))))));
        d = _mm512_add_ps(d, _mm512_mul_ps(q2, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(kp + 32))))));
        d = _mm512_add_ps(d, _mm512_mul_ps(q3, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(kp + 48))))));
        float dv[L16];
        _mm512_storeu_ps(dv, d);
        const float sc = red16(dv) * kv->ks[sl] * scale;
        scores[s] = sc;
        mx = sc > mx ? sc : mx;
    }
    for (int s = 0; s < npos; s++) scores[s] = orc_exp(scores[s] - mx);
    float total = 0.0f;
    for (int s = 0; s < npos; s++) total += scores[s];
    __m512 a0 = _mm512_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int s = 0; s < npos; s++) {
        const float p = scores[s] / total;
        const int64_t sl = ((int64_t)layer * kv->max_t + s) * kv->n_head + h;
        const int8_t *vp = kv->v + sl * HS;
        const __m512 ps = _mm512_set1_ps(p * kv->vs[sl]);
        a0 = _mm512_fmadd_ps(ps, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)vp))), a0);
        a1 = _mm512_fmadd_ps(ps, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(vp + 16)))), a1);
        a2 = _mm512_fmadd_ps(ps, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(vp + 32)))), a2);
        a3 = _mm512_fmadd_ps(ps, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(vp + 48)))), a3);
    }
    float *o = out + h * HS;
    (void)C;
    _mm512_storeu_ps(o, a0);
    _mm512_storeu_ps(o + 16, a1);
    _mm512_storeu_ps(o + 32, a2);
    _mm512_storeu_ps(o + 48, a3);
}

/* dot_row_i16's general loop (tensor.mojo:567-577) for the formats that are
 * neither BLOCKED nor int8 per channel: per group, VPDPWSSD over its 32-code
 * pieces (codes_i16: int4 low nibbles of 16 bytes, then their high
 * nibbles; int8 bytes; minus the zero point), then fma(f32(acc), scale). */
VNNI static float dot_generic_vnni(const orc_qm *m, int64_t row, const int16_t *xq) {
    const int64_t gpr = m->k / m->group;
    const uint8_t *p = m->data + row * m->k * m->bits / 8;
    const __m128i nib = _mm_set1_epi8(0x0f);
    __m512 accf = _mm512_setzero_ps();
    for (int64_t g = 0; g < gpr; g++) {
        const __m512i zp = _mm512_set1_epi16((short)m->zp[row * gpr + g]);
        __m512i acc = _mm512_setzero_si512();
        for (int64_t k0 = g * m->group; k0 < (g + 1) * m->group; k0 += 32) {
            __m512i u;
            if (m->bits == 4) {
                const __m128i b = _mm_loadu_si128((const __m128i *)(p + k0 / 2));
                const __m256i lo = _mm256_cvtepu8_epi16(_mm_and_si128(b, nib));
                const __m256i hi = _mm256_cvtepu8_epi16(_mm_and_si128(_mm_srli_epi16(b, 4), nib));
                u = _mm512_inserti64x4(_mm512_castsi256_si512(lo), hi, 1);
            } else {
                u = _mm512_cvtepu8_epi16(_mm256_loadu_si256((const __m256i *)(p + k0)));
            }
            acc = _mm512_dpwssd_epi32(acc, _mm512_loadu_si512((const void *)(xq + k0)), _mm512_sub_epi16(u, zp));
        }
        const float sc = orc_f16_to_f32(m->scale[row * gpr + g]);
        accf = _mm512_fmadd_ps(_mm512_cvtepi32_ps(acc), _mm512_set1_ps(sc), accf);
    }
    float v[L16];
    _mm512_storeu_ps(v, accf);
    return red16(v);
}

/* One row of dot_row_i16 by its branch (the scalar oracle's arithmetic). */
VNNI static float fast_row(const orc_qm *m, int64_t row, const int16_t *x1, const float *xs) {
    if (m->blocked) return dot_blocked_vnni(m, row, x1, xs);
    if (m->perch && m->bits == 8) return dot_ch8_vnni1(m, row, x1);
    if (m->group % 32 == 0) return dot_generic_vnni(m, row, x1);
    return orc_qm_dot_row_i16(m, row, x1, xs);
}

/* tile_i16 (kernels.mojo:512-573) on VPDPWSSD: per input pair one token's
 * two int16 activations broadcast as an int32 against 16 outputs x 2
 * inputs of wt, per token two accumulators (32 outputs); at each segment
 * end fma(f32(acc), scale, accf); the epilogue as the scalar tile. */
VNNI static inline __attribute__((always_inline)) void tile_i16_vnni_tm(
    const int TM, float *out, const int16_t *xq, const float *sx, const int16_t *wt, const float *st,
    const float *b, int64_t t0, int64_t o0, int64_t IN, int64_t OUT, int64_t G, int flags) {
    const int TN = 32, SEG = 256;
    __m512 accf[4][2];
    for (int m = 0; m < 4; m++) accf[m][0] = accf[m][1] = _mm512_setzero_ps();
    const int64_t seg = G < SEG ? G : SEG;
    for (int64_t k0 = 0; k0 < IN; k0 += seg) {
        const int64_t g = k0 / G;
        __m512i acc[4][2];
        for (int m = 0; m < 4; m++) acc[m][0] = acc[m][1] = _mm512_setzero_si512();
        for (int64_t kp = k0 / 2; kp < (k0 + seg) / 2; kp++) {
            const __m512i w0 = _mm512_loadu_si512((const void *)(wt + kp * TN * 2));
            const __m512i w1 = _mm512_loadu_si512((const void *)(wt + kp * TN * 2 + 32));
            for (int m = 0; m < TM; m++) {
                int32_t pair;
                memcpy(&pair, xq + (t0 + m) * IN + 2 * kp, 4);
                const __m512i xb = _mm512_set1_epi32(pair);
                acc[m][0] = _mm512_dpwssd_epi32(acc[m][0], xb, w0);
                acc[m][1] = _mm512_dpwssd_epi32(acc[m][1], xb, w1);
            }
        }
        const __m512 s0 = _mm512_loadu_ps(st + g * TN), s1 = _mm512_loadu_ps(st + g * TN + 16);
        for (int m = 0; m < TM; m++) {
            accf[m][0] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(acc[m][0]), s0, accf[m][0]);
            accf[m][1] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(acc[m][1]), s1, accf[m][1]);
        }
    }
    for (int m = 0; m < TM; m++) {
        const __m512 sxm = _mm512_set1_ps(sx[t0 + m]);
        float r[32];
        __m512 r0 = _mm512_mul_ps(accf[m][0], sxm), r1 = _mm512_mul_ps(accf[m][1], sxm);
        if (flags & EPI_BIAS) {
            r0 = _mm512_add_ps(r0, _mm512_loadu_ps(b + o0));
            r1 = _mm512_add_ps(r1, _mm512_loadu_ps(b + o0 + 16));
        }
        _mm512_storeu_ps(r, r0);
        _mm512_storeu_ps(r + 16, r1);
        for (int j = 0; j < TN; j++) finish(out, (t0 + m) * OUT + o0 + j, r[j], flags);
    }
}
/* (TM a compile-time constant in each call, so the accumulators stay in registers) */
VNNI static void tile_i16_vnni(int TM, float *out, const int16_t *xq, const float *sx, const int16_t *wt,
                               const float *st, const float *b, int64_t t0, int64_t o0, int64_t IN, int64_t OUT,
                               int64_t G, int flags) {
    if (TM == 4)
        tile_i16_vnni_tm(4, out, xq, sx, wt, st, b, t0, o0, IN, OUT, G, flags);
    else
        for (int m = 0; m < TM; m++) tile_i16_vnni_tm(1, out, xq, sx, wt, st, b, t0 + m, o0, IN, OUT, G, flags);
}

/* Switches the oracle's matmuls, row quantizer and attention to their AVX-512
 * VNNI forms (on == 1, where the CPU has them) or back to the scalar code.
 * Returns whether the fast forms are on. */
int orc_cpu_set_fast(int on) {
    on = on && orc_cpu_vnni();
    g_fast_tile = on ? tile_i16_vnni : NULL;
    g_fast_row = on ? fast_row : NULL;
    g_fast_quant = on ? quantize_row_vnni : NULL;
    g_fast_attend = on ? attend_one_vnni : NULL;
    return on;
}

/* GGUFMatrix.dot_row (gguf.mojo:388-417) on AVX-512: per 16 weights the
 * block decoder's floats (gguf.mojo:178-297, the scalar oracle's operations
 * in its order) and one fma into the 16 lanes, then the 16-lane sum.  The
 * block formats Q4_0 / Q4_1 / Q8_0 / Q4_K / Q5_K / Q6_K. */
VNNI static inline __m512 u8f(const uint8_t *p) { return _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i *)p))); }
VNNI static inline __m512i u8i(const uint8_t *p) { return _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i *)p)); }
VNNI static float gguf_dot_row_avx512(int t, const uint8_t *p, int64_t cols, const float *x) {
    const int bs = orc_gguf_block_size(t), bb = orc_gguf_block_bytes(t);
    const __m512i m4 = _mm512_set1_epi32(0xf);
    __m512 acc = _mm512_setzero_ps();
#define PUT(off, v) acc = _mm512_fmadd_ps((v), _mm512_loadu_ps(xb + (off)), acc)
    for (int64_t blk = 0; blk < cols / bs; blk++) {
        const uint8_t *b = p + blk * bb;
        const float *xb = x + blk * bs;
        if (t == GGML_Q4_0) {
            const __m512 d = _mm512_set1_ps(f16_at(b, 0)), e8 = _mm512_set1_ps(8.0f);
            const __m512i q = u8i(b + 2);
            PUT(0, _mm512_mul_ps(_mm512_sub_ps(_mm512_cvtepi32_ps(_mm512_and_si512(q, m4)), e8), d));
            PUT(16, _mm512_mul_ps(_mm512_sub_ps(_mm512_cvtepi32_ps(_mm512_srli_epi32(q, 4)), e8), d));
        } else if (t == GGML_Q4_1) {
            const __m512 d = _mm512_set1_ps(f16_at(b, 0)), mm = _mm512_set1_ps(f16_at(b, 2));
            const __m512i q = u8i(b + 4);
            PUT(0, _mm512_add_ps(_mm512_mul_ps(d, _mm512_cvtepi32_ps(_mm512_and_si512(q, m4))), mm));
            PUT(16, _mm512_add_ps(_mm512_mul_ps(d, _mm512_cvtepi32_ps(_mm512_srli_epi32(q, 4))), mm));
        } else if (t == GGML_Q8_0) {
            const __m512 d = _mm512_set1_ps(f16_at(b, 0));
            for (int h = 0; h < 2; h++)
                PUT(16 * h, _mm512_mul_ps(d, _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(_mm_loadu_si128((const __m128i *)(b + 2 + 16 * h))))));
        } else if (t == GGML_Q4_K || t == GGML_Q5_K) {
            const float d = f16_at(b, 0), dmin = f16_at(b, 2);
            const uint8_t *scales = b + 4;
            const int five = t == GGML_Q5_K;
            for (int j = 0; j < 4; j++) {
                int sc1, m1i, sc2, m2i;
                k_scale_min(scales, 2 * j, &sc1, &m1i);
                k_scale_min(scales, 2 * j + 1, &sc2, &m2i);
                const __m512 d1 = _mm512_set1_ps(d * (float)sc1), m1 = _mm512_set1_ps(dmin * (float)m1i);
                const __m512 d2 = _mm512_set1_ps(d * (float)sc2), m2 = _mm512_set1_ps(dmin * (float)m2i);
                for (int h = 0; h < 2; h++) {
                    const __m512i q = u8i(five ? b + 48 + 32 * j + 16 * h : b + 16 + 32 * j + 16 * h);
                    __m512i lo = _mm512_and_si512(q, m4), hi = _mm512_srli_epi32(q, 4);
                    if (five) {
                        const __m512i qh = u8i(b + 16 + 16 * h);
                        lo = _mm512_or_si512(lo, _mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(qh, 2 * j), _mm512_set1_epi32(1)), 4));
                        hi = _mm512_or_si512(hi, _mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(qh, 2 * j + 1), _mm512_set1_epi32(1)), 4));
                    }
                    PUT(64 * j + 16 * h, _mm512_sub_ps(_mm512_mul_ps(d1, _mm512_cvtepi32_ps(lo)), m1));
                    PUT(64 * j + 32 + 16 * h, _mm512_sub_ps(_mm512_mul_ps(d2, _mm512_cvtepi32_ps(hi)), m2));
                }
            }
        } else if (t == GGML_Q6_K) {
            const float d = f16_at(b, 208);
            const __m512 e32 = _mm512_set1_ps(32.0f);
            const __m512i m3 = _mm512_set1_epi32(3);
            for (int n = 0; n < 2; n++) {
                const int ql = 64 * n, qhoff = 128 + 32 * n, sc = 192 + 8 * n;
                for (int h = 0; h < 2; h++) {
                    const __m512i lo0 = u8i(b + ql + 16 * h), lo1 = u8i(b + ql + 32 + 16 * h), hi = u8i(b + qhoff + 16 * h);
                    const int base = 128 * n + 16 * h;
                    for (int k = 0; k < 4; k++) {
                        const float ds = d * (float)(int8_t)b[sc + h + 2 * k];
                        const __m512i l = k == 0 ? _mm512_and_si512(lo0, m4) : k == 1 ? _mm512_and_si512(lo1, m4)
                                        : k == 2 ? _mm512_srli_epi32(lo0, 4) : _mm512_srli_epi32(lo1, 4);
                        const __m512i q = _mm512_or_si512(l, _mm512_slli_epi32(_mm512_and_si512(_mm512_srli_epi32(hi, 2 * k), m3), 4));
                        PUT(base + 32 * k, _mm512_mul_ps(_mm512_set1_ps(ds), _mm512_sub_ps(_mm512_cvtepi32_ps(q), e32)));
                    }
                }
            }
        }
    }
#undef PUT
    (void)u8f;
    float v[L16];
    _mm512_storeu_ps(v, acc);
    return red16(v);
}

/* One row through the AVX-512 decoder (tests: equal to orc_gguf_dot_row). */
float orc_cpu_gguf_dot_row(int t, const uint8_t *row, int64_t cols, const float *x) {
    if (!orc_cpu_vnni()) return orc_gguf_dot_row(t, row, cols, x);
    return gguf_dot_row_avx512(t, row, cols, x);
}

/* Team (team.mojo:36-82): arrival count and generation on separate cache
 * lines; the last arrival resets the count, then advances the generation;
 * the others spin (PAUSE) for up to 1000 polls, then yield. */
typedef struct {
    _Alignas(64) int64_t count;
    _Alignas(64) int64_t gen;
    _Alignas(64) int nt;
} orc_team_bar;

static void team_wait(orc_team_bar *t) {
    const int64_t g = __atomic_load_n(&t->gen, __ATOMIC_ACQUIRE);
    if (__atomic_fetch_add(&t->count, 1, __ATOMIC_ACQ_REL) == t->nt - 1) {
        __atomic_store_n(&t->count, 0, __ATOMIC_RELAXED);
        __atomic_store_n(&t->gen, g + 1, __ATOMIC_RELEASE);
    } else {
        int spins = 0;
        while (__atomic_load_n(&t->gen, __ATOMIC_ACQUIRE) == g) {
            if (spins < 1000) {
                __builtin_ia32_pause();
                spins++;
            } else {
                sched_yield();
            }
        }
    }
}

typedef struct {
    orc_gpt2 *m;
    orc_team_bar bar;
    int vnni, stop, job; /* job 0: a decode step; 1: the head alone; 2: one GEMV; 3: one GGUF GEMV */
    /* jobs 2 and 3: the matrix, activations and outputs */
    const orc_qm *gw;
    int gtype;
    const uint8_t *gblocks;
    int64_t grows, gcols, growbytes;
    const float *gx;
    float *gout;
    int64_t token;
    int pos;
    /* linear_team's shared activations (gpt2t.mojo:370-373) */
    int16_t xq[4 * G_C], xp[4 * G_C];
    float xs[4 * G_C / 16], sx;
    int permuted;
} orc_team;

static void team_split(int64_t n, int tid, int nt, int64_t *b, int64_t *e) { /* team.mojo split */
    const int64_t per = (n + nt - 1) / nt;
    *b = tid * per < n ? tid * per : n;
    *e = (tid + 1) * per < n ? (tid + 1) * per : n;
}

/* linear_team (kernels.mojo:774-866), ACT16 branch; ends with a barrier. */
static void team_linear(orc_team *c, int tid, float *out, const float *x, const orc_qm *w, const float *b,
                        int64_t IN, int64_t OUT, int flags) {
    if (tid == 0) {
        if (c->vnni && IN % 16 == 0)
            quantize_row_vnni(x, IN, c->xq, &c->sx);
        else
            orc_quantize_rows(x, 1, IN, c->xq, &c->sx);
        c->permuted = orc_qm_permute_x_i16(w, c->xq, IN, c->xp, c->xs);
    }
    team_wait(&c->bar);
    const int16_t *x1 = c->permuted ? c->xp : c->xq;
    const float s = c->sx;
    int64_t o0, o1;
    team_split(OUT, tid, c->bar.nt, &o0, &o1);
    if (c->vnni && w->perch && w->bits == 8) {
        for (int64_t o = o0; o < o1; o += 4) {
            const int n = o1 - o < 4 ? (int)(o1 - o) : 4;
            float d[4];
            if (n == 4)
                dot_ch8_vnni4(w, o, x1, d);
            else
                for (int j = 0; j < n; j++) d[j] = dot_ch8_vnni1(w, o + j, x1);
            for (int j = 0; j < n; j++) {
                float r = d[j] * s;
                if (flags & EPI_BIAS) r += b[o + j];
                finish(out, o + j, r, flags);
            }
        }
    } else {
        for (int64_t o = o0; o < o1; o++) {
            float r = (c->vnni ? fast_row(w, o, x1, c->xs) : orc_qm_dot_row_i16(w, o, x1, c->xs)) * s;
            if (flags & EPI_BIAS) r += b[o];
            finish(out, o, r, flags);
        }
    }
    team_wait(&c->bar);
}

/* Model.decode's worker (gpt2t.mojo:375-444) for one token. */
static void team_decode(orc_team *c, int tid) {
    orc_gpt2 *m = c->m;
    const int C = G_C, nt = c->bar.nt;
    if (tid == 0) {
        orc_qm_dequant_row(&m->wte, c->token, m->x);
        const float *p = m->wpe + (int64_t)c->pos * C;
        for (int i = 0; i < C; i++) m->x[i] = m->x[i] + p[i];
    }
    for (int l = 0; l < G_NL; l++) {
        const orc_qm *w = &m->mats[l * 4];
        float **v = &m->vecs[l * N_VECS];
        if (tid == 0) orc_layernorm(m->xn, m->x, v[LN1_W], v[LN1_B], 1, C);
        team_wait(&c->bar);
        team_linear(c, tid, m->qkv, m->xn, &w[0], v[QKV_B], C, 3 * C, EPI_BIAS);
        if (tid == 0) orc_kv_store(&m->kv, l, c->pos, m->qkv + C, m->qkv + 2 * C);
        team_wait(&c->bar);
        for (int h = tid; h < G_NH; h += nt) {
            if (c->vnni && m->kv.head_dim == 64)
                attend_one_vnni(&m->kv, m->att, m->qkv, l, h, c->pos);
            else
                orc_kv_attend_one(&m->kv, m->att, m->qkv, l, 0, h, c->pos);
        }
        team_wait(&c->bar);
        team_linear(c, tid, m->x, m->att, &w[1], v[PROJ_B], C, C, EPI_BIAS | EPI_RESID);
        if (tid == 0) orc_layernorm(m->xn, m->x, v[LN2_W], v[LN2_B], 1, C);
        team_wait(&c->bar);
        team_linear(c, tid, m->fc, m->xn, &w[2], v[FC_B], C, 4 * C, EPI_BIAS | EPI_GELU);
        team_linear(c, tid, m->x, m->fc, &w[3], v[FCPROJ_B], 4 * C, C, EPI_BIAS | EPI_RESID);
    }
    if (tid == 0) orc_layernorm(m->xn, m->x, m->lnf_w, m->lnf_b, 1, C);
    team_wait(&c->bar);
    team_linear(c, tid, m->logits, m->xn, &m->wte, NULL, C, G_V, 0); /* head_team, kernels.mojo:869-910 */
}

/* The team's work for one start: a decode step, or the head alone. */
static void team_job(orc_team *c, int tid) {
    if (c->job == 0) {
        team_decode(c, tid);
    } else if (c->job == 1) {
        team_linear(c, tid, c->m->logits, c->m->xn, &c->m->wte, NULL, G_C, G_V, 0);
    } else if (c->job == 2) {
        team_linear(c, tid, c->gout, c->gx, c->gw, NULL, c->gw->k, c->gw->n, 0);
    } else { /* linear_team's OUT_MAJOR branch (kernels.mojo:817-826): dot_row per row, contiguous ranges */
        int64_t o0, o1;
        team_split(c->grows, tid, c->bar.nt, &o0, &o1);
        for (int64_t o = o0; o < o1; o++)
            c->gout[o] = c->vnni ? gguf_dot_row_avx512(c->gtype, c->gblocks + o * c->growbytes, c->gcols, c->gx)
                                 : orc_gguf_dot_row(c->gtype, c->gblocks + o * c->growbytes, c->gcols, c->gx);
        team_wait(&c->bar);
    }
}

typedef struct {
    orc_team *c;
    int tid;
} orc_team_arg;

typedef struct {
    orc_team *c;
    pthread_t th[256];
    orc_team_arg args[256];
} orc_team_threads;

static void *team_worker(void *p) {
    orc_team_arg *a = (orc_team_arg *)p;
    for (;;) {
        team_wait(&a->c->bar); /* a job starts (or the team stops) */
        if (__atomic_load_n(&a->c->stop, __ATOMIC_ACQUIRE)) return NULL;
        team_job(a->c, a->tid);
    }
}

/* Starts nt - 1 workers (the caller is thread 0); NULL if that fails. */
static orc_team_threads *team_start(orc_gpt2 *m, int nt) {
    if (nt < 1 || nt > 256) return NULL;
    orc_team_threads *T = (orc_team_threads *)calloc(1, sizeof(orc_team_threads));
    orc_team *c = (orc_team *)aligned_alloc(64, (sizeof(orc_team) + 63) / 64 * 64);
    if (!T || !c) {
        free(T);
        free(c);
        return NULL;
    }
    memset(c, 0, sizeof(*c));
    c->m = m;
    c->bar.nt = nt;
    c->vnni = orc_cpu_vnni();
    T->c = c;
    int started = 0;
    for (int t = 1; t < nt; t++) {
        T->args[t].c = c;
        T->args[t].tid = t;
        if (pthread_create(&T->th[t], NULL, team_worker, &T->args[t]) != 0) break;
        started++;
    }
    if (started != nt - 1) { /* release the ones made */
        c->bar.nt = started + 1;
        __atomic_store_n(&c->stop, 1, __ATOMIC_RELEASE);
        team_wait(&c->bar);
        for (int t = 1; t <= started; t++) pthread_join(T->th[t], NULL);
        free(c);
        free(T);
        return NULL;
    }
    return T;
}

static void team_stop(orc_team_threads *T) {
    __atomic_store_n(&T->c->stop, 1, __ATOMIC_RELEASE);
    team_wait(&T->c->bar);
    for (int t = 1; t < T->c->bar.nt; t++) pthread_join(T->th[t], NULL);
    free(T->c);
    free(T);
}

/* Runs one job on the whole team (the caller as thread 0). */
static void team_run(orc_team *c, int job) {
    c->job = job;
    team_wait(&c->bar);
    team_job(c, 0);
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* generate's greedy loop (gpt2t.mojo:949-981): the prompt through
 * Model.forward (the oracle's, on g_threads OpenMP threads), then each
 * further token through the team decode on nt threads (nt - 1 workers plus
 * the caller, started before the timed loop).  secs[0] = the prompt's wall
 * time, secs[1] = the decode loop's (the forwards plus the argmax picks, as
 * gpt2t.mojo:968-1005 times it).  Returns the count generated, or -1. */
int orc_cpu_generate(orc_gpt2 *m, const int64_t *prompt, int n_prompt, int steps, int nt, int64_t *out_tokens,
                     double *secs) {
    if (nt < 1 || nt > 256 || n_prompt < 1 || steps < 1 || n_prompt + steps > G_MAXT) return -1;
    const double t0 = now_s();
    const float *logits = orc_gpt2_forward(m, prompt, n_prompt, 0);
    const double t1 = now_s();
    orc_team_threads *T = team_start(m, nt);
    if (!T) return -1;
    const double t2 = now_s();
    int pos = n_prompt, generated = 0;
    for (int i = 0; i < steps; i++) {
        int64_t next = orc_argmax(logits, G_V);
        if (next == 50256) break;
        out_tokens[generated++] = next;
        if (generated == steps) break;
        T->c->token = next;
        T->c->pos = pos++;
        team_run(T->c, 0);
        logits = m->logits;
    }
    const double t3 = now_s();
    team_stop(T);
    if (secs) {
        secs[0] = t1 - t0;
        secs[1] = t3 - t2;
    }
    return generated;
}

/* One token through the team decode at position pos (the cache holds
 * positions < pos); returns the logits (the model's buffer), NULL on a bad
 * argument. */
const float *orc_cpu_decode(orc_gpt2 *m, int64_t token, int pos, int nt) {
    if (pos < 0 || pos >= G_MAXT || token < 0 || token >= G_V) return NULL;
    orc_team_threads *T = team_start(m, nt);
    if (!T) return NULL;
    T->c->token = token;
    T->c->pos = pos;
    team_run(T->c, 0);
    team_stop(T);
    return m->logits;
}

/* The int8 per-channel head alone on a team of nt, one token: the median
 * seconds of `reps` calls (the reference's per-kernel anchor,
 * research/test_head.mojo:45-51).  Overwrites the model's xn and logits. */
double orc_cpu_head_seconds(orc_gpt2 *m, int nt, int reps) {
    if (reps < 1 || reps > 10000) return -1.0;
    orc_team_threads *T = team_start(m, nt);
    if (!T) return -1.0;
    for (int i = 0; i < G_C; i++) m->xn[i] = (float)((i * 37) % 101 - 50) / 50.0f;
    double *t = (double *)malloc(sizeof(double) * (size_t)reps);
    for (int r = 0; r < reps; r++) {
        const double a = now_s();
        team_run(T->c, 1);
        t[r] = now_s() - a;
    }
    team_stop(T);
    for (int i = 1; i < reps; i++)
        for (int j = i; j > 0 && t[j] < t[j - 1]; j--) {
            const double x = t[j];
            t[j] = t[j - 1];
            t[j - 1] = x;
        }
    const double med = t[reps / 2];
    free(t);
    return med;
}

static double median_of(double *t, int n) {
    for (int i = 1; i < n; i++)
        for (int j = i; j > 0 && t[j] < t[j - 1]; j--) {
            const double x = t[j];
            t[j] = t[j - 1];
            t[j - 1] = x;
        }
    return t[n / 2];
}

/* linear_team (kernels.mojo:774-866) of one token on a team of nt: the
 * median seconds of `reps` calls cycling over the nrot matrices ws (copies
 * of one, so that their codes come from memory rather than cache), x and
 * out of ws[0]'s shape.  -1 on a bad argument. */
double orc_cpu_gemv_seconds(const orc_qm *const *ws, int nrot, const float *x, float *out, int nt, int reps) {
    if (reps < 1 || reps > 100000 || nrot < 1 || !ws || !x || !out) return -1.0;
    if (ws[0]->k > 4 * G_C) return -1.0; /* the team's activation buffers */
    orc_team_threads *T = team_start(NULL, nt);
    if (!T) return -1.0;
    double *t = (double *)malloc(sizeof(double) * (size_t)reps);
    T->c->gx = x;
    T->c->gout = out;
    for (int r = -2; r < reps; r++) {
        T->c->gw = ws[(r + 2) % nrot];
        const double a = now_s();
        team_run(T->c, 2);
        if (r >= 0) t[r] = now_s() - a;
    }
    team_stop(T);
    const double med = median_of(t, reps);
    free(t);
    return med;
}

/* GGUFMatrix.dot_row over every row (linear_team's OUT_MAJOR branch) of a
 * rows x cols matrix of ggml type t on a team of nt: the median seconds of
 * `reps` calls cycling over the nrot copies blocks[i].  -1 on a bad argument. */
double orc_cpu_gguf_gemv_seconds(int t, const uint8_t *const *blocks, int nrot, int64_t rows, int64_t cols,
                                 const float *x, float *out, int nt, int reps) {
    const int bs = orc_gguf_block_size(t), bb = orc_gguf_block_bytes(t);
    if (reps < 1 || reps > 100000 || nrot < 1 || !blocks || bs < 32 || cols % bs) return -1.0;
    orc_team_threads *T = team_start(NULL, nt);
    if (!T) return -1.0;
    double *tt = (double *)malloc(sizeof(double) * (size_t)reps);
    T->c->gtype = t;
    T->c->grows = rows;
    T->c->gcols = cols;
    T->c->growbytes = cols / bs * bb;
    T->c->gx = x;
    T->c->gout = out;
    for (int r = -2; r < reps; r++) {
        T->c->gblocks = blocks[(r + 2) % nrot];
        const double a = now_s();
        team_run(T->c, 3);
        if (r >= 0) tt[r] = now_s() - a;
    }
    team_stop(T);
    const double med = median_of(tt, reps);
    free(tt);
    return med;
}

/* Model.forward of a T-token prompt from position 0 (gpt2t.mojo:329-342) with
 * the matmuls on VPDPWSSD tiles and the attention, quantizer and one-token
 * head on their AVX-512 forms (orc_cpu_set_fast), parallel over g_threads =
 * nt OpenMP threads as the reference's parallelize is over its tasks; the
 * logits are the scalar oracle's bit for bit.  secs[0] = wall time.  Returns
 * the logits (the model's buffer), NULL on a bad argument. */
const float *orc_cpu_prompt(orc_gpt2 *m, const int64_t *tokens, int T, int nt, double *secs) {
    if (!m || !tokens || T < 1 || T > G_MAXT || nt < 1 || nt > 256) return NULL;
    const int saved = g_threads;
    g_threads = nt;
    orc_cpu_set_fast(1);
    const double t0 = now_s();
    const float *lg = orc_gpt2_forward(m, tokens, T, 0);
    const double t1 = now_s();
    orc_cpu_set_fast(0);
    g_threads = saved;
    if (secs) secs[0] = t1 - t0;
    return lg;
}
