/*
 * tfq_oracle.c — CPU restatement of the reference's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see tfq_oracle.h.
 * Build with -ffp-contract=off (oracle/Makefile) so that every `a * b + c`
 * below rounds twice, as Swift evaluates it.
 */
#include "tfq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* PRNG                                                                      */
/* ------------------------------------------------------------------------ */

/* V/PRNG/SplitMix64.swift:11-17 */
uint64_t tfo_splitmix64_next(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* V/PRNG/SplitMix64.swift:20-23: u = Float(next() >> 40) / 2^24; lo + (hi - lo) * u */
float tfo_splitmix64_uniform(uint64_t *state, float lo, float hi) {
    float u = (float)(tfo_splitmix64_next(state) >> 40) / (float)(1u << 24);
    float span = hi - lo;
    float scaled = span * u;
    return lo + scaled;
}

/* V/PRNG/SeedTree.swift:12-19: FNV-1a-64 of the UTF-8 label, xor the root. */
uint64_t tfo_seedtree_key(uint64_t root, const char *label) {
    uint64_t h = 0xCBF29CE484222325ULL;
    for (const unsigned char *p = (const unsigned char *)label; *p; ++p) {
        h ^= (uint64_t)*p;
        h *= 0x100000001B3ULL;
    }
    return root ^ h;
}

/* ------------------------------------------------------------------------ */
/* 16-bit floats                                                             */
/* ------------------------------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Quantization.swift:16-23: RNE by adding 0x7FFF + lsb, no NaN special case. */
uint16_t tfo_f32_to_bf16(float x) {
    uint32_t bits = f2u(x);
    uint32_t lsb = (bits >> 16) & 1u;
    uint32_t rounded = (bits + 0x7FFFu + lsb) >> 16;
    return (uint16_t)rounded;
}

/* Quantization.swift:25-28 */
float tfo_bf16_to_f32(uint16_t bits) { return u2f((uint32_t)bits << 16); }

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even. */
uint16_t tfo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf / nan */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* rounds to inf */
    int e = (int)(ax >> 23) - 127;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    if (e < -14) {                                  /* binary16 subnormal or zero */
        if (ax == 0) return (uint16_t)sign;
        int s = -(e + 1);                           /* value / 2^-24 = m >> s */
        if (s > 31) return (uint16_t)sign;
        uint32_t h = m >> s;
        uint32_t rem = m & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)(e + 15) << 10) | ((m >> 13) & 0x3FFu);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* carry may bump the exponent */
    return (uint16_t)(sign | h);
}

float tfo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

float tfo_decode_scale(uint16_t bits, int scale_fmt) {
    return scale_fmt == TFO_FMT_BF16 ? tfo_bf16_to_f32(bits) : tfo_f16_to_f32(bits);
}

/* ------------------------------------------------------------------------ */
/* Affine format                                                             */
/* ------------------------------------------------------------------------ */

/* Per-group min/max affine quantiser shared by the 4- and 8-bit fixtures:
 * Quantization.swift:59-100 (int4) and :144-175 (int8). */
static void quantize_affine_row(const float *row, int n, int levels, int bits,
                                uint8_t *packed, uint16_t *scales, uint16_t *biases) {
    int n_groups = n / TFO_GROUP;
    if (bits == 4) memset(packed, 0, (size_t)n / 2);
    for (int g = 0; g < n_groups; ++g) {
        float wmin = INFINITY, wmax = -INFINITY;
        for (int k = 0; k < TFO_GROUP; ++k) {
            float w = row[g * TFO_GROUP + k];
            if (w < wmin) wmin = w;
            if (w > wmax) wmax = w;
        }
        float scale_f, bias_f;
        if (wmax == wmin) { scale_f = 1.0f; bias_f = wmin; }
        else { scale_f = (wmax - wmin) / (float)levels; bias_f = wmin; }
        uint16_t sb = tfo_f32_to_bf16(scale_f), bb = tfo_f32_to_bf16(bias_f);
        scales[g] = sb;
        biases[g] = bb;
        float scale = tfo_bf16_to_f32(sb), bias = tfo_bf16_to_f32(bb);
        float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
        for (int k = 0; k < TFO_GROUP; ++k) {
            float w = row[g * TFO_GROUP + k];
            float t = (w - bias) * inv;
            long q = (long)roundf(t);               /* Swift .rounded(): ties away from zero */
            if (q < 0) q = 0;
            if (q > levels) q = levels;
            if (bits == 4) {
                int byte_idx = g * (TFO_GROUP / 2) + k / 2;
                uint8_t nib = (uint8_t)(q & 0x0F);
                if ((k & 1) == 0) packed[byte_idx] = (uint8_t)((packed[byte_idx] & 0xF0) | nib);
                else packed[byte_idx] = (uint8_t)((packed[byte_idx] & 0x0F) | (nib << 4));
            } else {
                packed[g * TFO_GROUP + k] = (uint8_t)q;
            }
        }
    }
}

void tfo_quantize_int4_row(const float *row, int n, uint8_t *packed, uint16_t *s, uint16_t *b) {
    quantize_affine_row(row, n, 15, 4, packed, s, b);
}

void tfo_quantize_int8_row(const float *row, int n, uint8_t *packed, uint16_t *s, uint16_t *b) {
    quantize_affine_row(row, n, 255, 8, packed, s, b);
}

/* Element j of a packed int4 row: low nibble of byte j/2 for even j, high for
 * odd j (Quantization.swift:112-114). On a little-endian host this is bits
 * 4*(j%8) .. 4*(j%8)+3 of 32-bit word j/8. */
uint32_t tfo_int4_code(const uint8_t *packed_row, size_t j) {
    uint8_t b = packed_row[j >> 1];
    return (j & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0x0F);
}

/* Quantization.swift:104-119: w = Float(nibble) * scale + bias (two roundings). */
void tfo_dequantize_int4_row(const uint8_t *packed, const uint16_t *scales, const uint16_t *biases,
                             int scale_fmt, int n, float *out) {
    for (int g = 0; g < n / TFO_GROUP; ++g) {
        float scale = tfo_decode_scale(scales[g], scale_fmt);
        float bias = tfo_decode_scale(biases[g], scale_fmt);
        for (int k = 0; k < TFO_GROUP; ++k) {
            size_t j = (size_t)g * TFO_GROUP + k;
            float prod = (float)tfo_int4_code(packed, j) * scale;
            out[j] = prod + bias;
        }
    }
}

/* ---- 2-, 3- and 4-bit rows (Quantization.swift:195-349) ---- */

/* QuantizedAffineRow.packedRowBytes (Quantization.swift:219-222). */
size_t tfo_affine_row_bytes(size_t n, int bits) { return (n * (size_t)bits + 7) / 8; }

/* Quantization.swift:295-320 (packCode): code j at bits j*bits.. of the
 * little-endian row, OR-ed in (3-bit: into the byte after as well when the
 * code straddles a byte boundary and that byte exists). */
void tfo_pack_affine_code(uint8_t *buf, size_t nbytes, uint32_t code, size_t j, int bits) {
    if (bits == 4) {
        size_t i = j / 2;
        uint8_t nib = (uint8_t)(code & 0x0F);
        buf[i] = (j & 1) == 0 ? (uint8_t)((buf[i] & 0xF0) | nib) : (uint8_t)((buf[i] & 0x0F) | (nib << 4));
    } else if (bits == 2) {
        size_t i = j / 4;
        unsigned sh = (unsigned)(j % 4) * 2;
        buf[i] = (uint8_t)((buf[i] & ~(0x03u << sh)) | ((code & 0x03u) << sh));
    } else {
        size_t bit = j * 3, i = bit / 8;
        uint32_t v = (code & 0x07u) << (bit % 8);
        buf[i] |= (uint8_t)(v & 0xFF);
        if (i + 1 < nbytes) buf[i + 1] |= (uint8_t)((v >> 8) & 0xFF);
    }
}

/* Quantization.swift:322-349 (unpackCode); bytes past the row read as 0. */
uint32_t tfo_affine_code(const uint8_t *row, size_t nbytes, size_t j, int bits) {
    if (bits == 4) return (j & 1) ? (uint32_t)(row[j / 2] >> 4) : (uint32_t)(row[j / 2] & 0x0F);
    if (bits == 2) return (uint32_t)(row[j / 4] >> ((j % 4) * 2)) & 0x03u;
    size_t bit = j * 3, i = bit / 8;
    uint32_t b0 = row[i], b1 = i + 1 < nbytes ? row[i + 1] : 0, b2 = i + 2 < nbytes ? row[i + 2] : 0;
    return ((b0 | (b1 << 8) | (b2 << 16)) >> (bit % 8)) & 0x07u;
}

/* Quantization.swift:229-273 (quantizeAffine): BF16-rounded scale/bias first,
 * codes against the rounded values, qMax = 2^bits - 1. */
void tfo_quantize_affine_row(const float *row, int n, int bits, uint8_t *packed, uint16_t *scales,
                             uint16_t *biases) {
    const int qmax = (1 << bits) - 1;
    const size_t nbytes = tfo_affine_row_bytes((size_t)n, bits);
    memset(packed, 0, nbytes);
    for (int g = 0; g < n / TFO_GROUP; ++g) {
        float wmin = INFINITY, wmax = -INFINITY;
        for (int k = 0; k < TFO_GROUP; ++k) {
            float w = row[g * TFO_GROUP + k];
            if (w < wmin) wmin = w;
            if (w > wmax) wmax = w;
        }
        float scale_f = wmax == wmin ? 1.0f : (wmax - wmin) / (float)qmax;
        uint16_t sb = tfo_f32_to_bf16(scale_f), bb = tfo_f32_to_bf16(wmin);
        scales[g] = sb;
        biases[g] = bb;
        float scale = tfo_bf16_to_f32(sb), bias = tfo_bf16_to_f32(bb);
        float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
        for (int k = 0; k < TFO_GROUP; ++k) {
            long q = (long)roundf((row[g * TFO_GROUP + k] - bias) * inv);
            if (q < 0) q = 0;
            if (q > qmax) q = qmax;
            tfo_pack_affine_code(packed, nbytes, (uint32_t)q, (size_t)g * TFO_GROUP + k, bits);
        }
    }
}

/* Quantization.swift:275-293 (dequantizeAffine): Float(code) * scale + bias. */
void tfo_dequantize_affine_row(const uint8_t *packed, const uint16_t *scales, const uint16_t *biases,
                               int scale_fmt, int bits, int n, float *out) {
    const size_t nbytes = tfo_affine_row_bytes((size_t)n, bits);
    for (int g = 0; g < n / TFO_GROUP; ++g) {
        float scale = tfo_decode_scale(scales[g], scale_fmt);
        float bias = tfo_decode_scale(biases[g], scale_fmt);
        for (int k = 0; k < TFO_GROUP; ++k) {
            size_t j = (size_t)g * TFO_GROUP + k;
            float prod = (float)tfo_affine_code(packed, nbytes, j, bits) * scale;
            out[j] = prod + bias;
        }
    }
}

/* Quantization.swift:179-191 */
void tfo_dequantize_int8_row(const uint8_t *packed, const uint16_t *scales, const uint16_t *biases,
                             int scale_fmt, int n, float *out) {
    for (int g = 0; g < n / TFO_GROUP; ++g) {
        float scale = tfo_decode_scale(scales[g], scale_fmt);
        float bias = tfo_decode_scale(biases[g], scale_fmt);
        for (int k = 0; k < TFO_GROUP; ++k) {
            size_t j = (size_t)g * TFO_GROUP + k;
            float prod = (float)packed[j] * scale;
            out[j] = prod + bias;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV references                                                           */
/* ------------------------------------------------------------------------ */

/* V/Reference/Quant/DequantInt4Gemv.swift:26-40: per row, dequantise to fp32,
 * then dot in index order (the scalar loop that pins vDSP_dotpr,
 * T/Validation/Reference/DequantInt4GEMVReferenceTests.swift:13-27). */
/* Threads the row loops below may use. Only the CPU-baseline build
 * (cpu_baseline.c, compiled with -fopenmp) acts on it: the checker build has
 * no OpenMP, so its `omp` pragmas are ignored and every loop stays serial.
 * Rows, heads, token rows and expert pairs are independent, so a split
 * changes no result (tests/test_cpu_baseline.py checks it bit for bit). */
static int tfo_threads = 1;
void tfo_set_threads(int n) { tfo_threads = n > 0 ? n : 1; }
#define TFO_ROW_CHUNK 16

static void gemv_affine_rows(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt, int bits,
                             const float *x, int r0, int r1, int n, float *y) {
    float *w = (float *)malloc(sizeof(float) * (size_t)n);
    size_t row_bytes = tfo_affine_row_bytes((size_t)n, bits), groups = (size_t)n / TFO_GROUP;
    for (int r = r0; r < r1; ++r) {
        if (bits == 4)
            tfo_dequantize_int4_row(W + (size_t)r * row_bytes, S + (size_t)r * groups,
                                    B + (size_t)r * groups, fmt, n, w);
        else
            tfo_dequantize_affine_row(W + (size_t)r * row_bytes, S + (size_t)r * groups,
                                      B + (size_t)r * groups, fmt, bits, n, w);
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) {
            float p = w[i] * x[i];
            sum = sum + p;
        }
        y[r] = sum;
    }
    free(w);
}

/* gemv_affine_rows over [0, m), in chunks of rows split over tfo_threads. */
static void gemv_affine_split(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt, int bits,
                              const float *x, int m, int n, float *y) {
#pragma omp parallel for schedule(static) num_threads(tfo_threads) if (tfo_threads > 1)
    for (int r0 = 0; r0 < m; r0 += TFO_ROW_CHUNK)
        gemv_affine_rows(W, S, B, fmt, bits, x, r0, r0 + TFO_ROW_CHUNK < m ? r0 + TFO_ROW_CHUNK : m, n, y);
}

void tfo_gemv_int4(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                   const float *x, int m, int n, float *y) {
    gemv_affine_split(W, S, B, fmt, 4, x, m, n, y);
}

/* The same GEMV over 2-, 3- or 4-bit rows of tfo_affine_row_bytes(n, bits)
 * bytes: dequantizeAffine, then the dot in index order (the b3 GEMV and
 * b2/b3 expert kernels compute this function: dequant_int4.metal:512-717,
 * moe.metal:644-1180). */
void tfo_gemv_affine(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt, int bits,
                     const float *x, int m, int n, float *y) {
    gemv_affine_split(W, S, B, fmt, bits, x, m, n, y);
}

void tfo_gemv_int4_f64(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                       const float *x, int m, int n, double *y) {
    float *w = (float *)malloc(sizeof(float) * (size_t)n);
    size_t row_bytes = (size_t)n / 2, groups = (size_t)n / TFO_GROUP;
    for (int r = 0; r < m; ++r) {
        tfo_dequantize_int4_row(W + (size_t)r * row_bytes, S + (size_t)r * groups,
                                B + (size_t)r * groups, fmt, n, w);
        double sum = 0.0;
        for (int i = 0; i < n; ++i) sum += (double)w[i] * (double)x[i];
        y[r] = sum;
    }
    free(w);
}

/* V/Reference/Quant/DequantInt8Gemv.swift:24-38 */
static void gemv_int8_rows(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                           const float *x, int r0, int r1, int n, float *y) {
    float *w = (float *)malloc(sizeof(float) * (size_t)n);
    size_t groups = (size_t)n / TFO_GROUP;
    for (int r = r0; r < r1; ++r) {
        tfo_dequantize_int8_row(W + (size_t)r * n, S + (size_t)r * groups, B + (size_t)r * groups,
                                fmt, n, w);
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) {
            float p = w[i] * x[i];
            sum = sum + p;
        }
        y[r] = sum;
    }
    free(w);
}

void tfo_gemv_int8(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                   const float *x, int m, int n, float *y) {
#pragma omp parallel for schedule(static) num_threads(tfo_threads) if (tfo_threads > 1)
    for (int r0 = 0; r0 < m; r0 += TFO_ROW_CHUNK)
        gemv_int8_rows(W, S, B, fmt, x, r0, r0 + TFO_ROW_CHUNK < m ? r0 + TFO_ROW_CHUNK : m, n, y);
}

void tfo_gemv_int8_f64(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                       const float *x, int m, int n, double *y) {
    float *w = (float *)malloc(sizeof(float) * (size_t)n);
    size_t groups = (size_t)n / TFO_GROUP;
    for (int r = 0; r < m; ++r) {
        tfo_dequantize_int8_row(W + (size_t)r * n, S + (size_t)r * groups, B + (size_t)r * groups,
                                fmt, n, w);
        double sum = 0.0;
        for (int i = 0; i < n; ++i) sum += (double)w[i] * (double)x[i];
        y[r] = sum;
    }
    free(w);
}

typedef struct {
    const uint8_t *W; const uint16_t *S, *B; int fmt; const float *x;
    int r0, r1, n; float *y;
} gemv_job;

static void *gemv_worker(void *arg) {
    gemv_job *j = (gemv_job *)arg;
    gemv_affine_rows(j->W, j->S, j->B, j->fmt, 4, j->x, j->r0, j->r1, j->n, j->y);
    return NULL;
}

void tfo_gemv_int4_mt(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                      const float *x, int m, int n, float *y, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    gemv_job jobs[256];
    int per = (m + threads - 1) / threads;
    int launched = 0;
    for (int t = 0; t < threads; ++t) {
        int r0 = t * per, r1 = r0 + per > m ? m : r0 + per;
        if (r0 >= r1) break;
        jobs[t] = (gemv_job){W, S, B, fmt, x, r0, r1, n, y};
        if (pthread_create(&tid[t], NULL, gemv_worker, &jobs[t]) != 0) {
            gemv_worker(&jobs[t]);
            tid[t] = 0;
        }
        launched = t + 1;
    }
    for (int t = 0; t < launched; ++t)
        if (tid[t]) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------------------ */
/* Router                                                                    */
/* ------------------------------------------------------------------------ */

/* T/Kernels/MoE/RouterTopKTests.swift:76-80: scaled = h ⊙ eff, then the int8
 * GEMV reference over the expert rows. */
void tfo_router_logits(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                       const float *h, const float *eff, int num_experts, int d, float *logits) {
    float *scaled = (float *)malloc(sizeof(float) * (size_t)d);
    for (int i = 0; i < d; ++i) scaled[i] = eff ? h[i] * eff[i] : h[i];
    tfo_gemv_int8(W, S, B, fmt, scaled, num_experts, d, logits);
    free(scaled);
}

/* T/Kernels/MoE/RouterTopKTests.swift:81-96: sort by (logit desc, index asc),
 * keep k, weights = exp(l - max) / Σ exp × expert_scale[idx]. */
int tfo_topk_softmax(const float *logits, int num_experts, int k, const float *expert_scale,
                     uint32_t *idx, float *weights) {
    if (k <= 0 || k > num_experts) return -1;
    /* selection by repeated scan keeps the (desc, asc-index) order exactly.
     * The reference's sort (RouterTopKTests.swift:85-87) has no defined
     * order for NaN; here NaN ranks below every number, as in the GPU
     * selector router_topk_select_k8 (S/Metal/MoE/moe.metal:152-168), which
     * never prefers a NaN score. -0 == +0, so they tie by index. */
    unsigned char *taken = (unsigned char *)calloc((size_t)num_experts, 1);
    for (int r = 0; r < k; ++r) {
        int best = -1;
        for (int e = 0; e < num_experts; ++e) {
            if (taken[e]) continue;
            /* strict: ties keep the lower index */
            if (best < 0 || (!isnan(logits[e]) && (isnan(logits[best]) || logits[e] > logits[best])))
                best = e;
        }
        taken[best] = 1;
        idx[r] = (uint32_t)best;
    }
    free(taken);
    float maximum = logits[idx[0]];
    float *ex = (float *)malloc(sizeof(float) * (size_t)k);
    float sum = 0.0f;
    for (int r = 0; r < k; ++r) { ex[r] = expf(logits[idx[r]] - maximum); }
    for (int r = 0; r < k; ++r) sum = sum + ex[r];               /* reduce(0, +) in order */
    for (int r = 0; r < k; ++r) {
        float gain = expert_scale ? expert_scale[idx[r]] : 1.0f;
        float v = ex[r] / sum;
        weights[r] = v * gain;
    }
    free(ex);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* MoE                                                                       */
/* ------------------------------------------------------------------------ */

/* V/Reference/MoE/Moe.swift:17-29:
 * inner = c * (x + k * x * x * x); y = 0.5 * x * (1 + tanh(inner)) */
float tfo_gelu_tanh(float xv) {
    const float c = 0.7978845608028654f, k3 = 0.044715f;
    float cube_term = k3 * xv;
    cube_term = cube_term * xv;
    cube_term = cube_term * xv;
    float inner_sum = xv + cube_term;
    float inner = c * inner_sum;
    float half_x = 0.5f * xv;
    float one_plus = 1.0f + tanhf(inner);
    return half_x * one_plus;
}

/* Moe.swift:33-52 on one expert blob whose gate/up/down rows hold `bits`-bit
 * codes (the b2/b3 experts of moe.metal:644-1180 compute the same FFN). */
static void ffn_affine(const uint8_t *blob, const tfo_expert_offsets *o, int fmt, int bits, const float *x,
                       int d, int f, float *out) {
    float *gate = (float *)malloc(sizeof(float) * (size_t)f);
    float *up = (float *)malloc(sizeof(float) * (size_t)f);
    float *act = (float *)malloc(sizeof(float) * (size_t)f);
    tfo_gemv_affine(blob + o->gate_w, (const uint16_t *)(blob + o->gate_s),
                    (const uint16_t *)(blob + o->gate_b), fmt, bits, x, f, d, gate);
    tfo_gemv_affine(blob + o->up_w, (const uint16_t *)(blob + o->up_s),
                    (const uint16_t *)(blob + o->up_b), fmt, bits, x, f, d, up);
    for (int i = 0; i < f; ++i) act[i] = tfo_gelu_tanh(gate[i]) * up[i];   /* vDSP_vmul */
    tfo_gemv_affine(blob + o->down_w, (const uint16_t *)(blob + o->down_s),
                    (const uint16_t *)(blob + o->down_b), fmt, bits, act, d, f, out);
    free(gate); free(up); free(act);
}

void tfo_ffn_int4(const uint8_t *blob, const tfo_expert_offsets *o, int fmt, const float *x,
                  int d, int f, float *out) {
    ffn_affine(blob, o, fmt, 4, x, d, f, out);
}

/* Moe.swift:58-88 */
void tfo_moe_routed(const uint8_t *pool, uint64_t stride, const tfo_expert_offsets *off, int fmt,
                    const float *x, const float *residual, const uint32_t *idx, const float *w,
                    int k, int d, int f, float *y) {
    tfo_moe_routed_bits(pool, stride, off, fmt, 4, x, residual, idx, w, k, d, f, y);
}

void tfo_moe_routed_bits(const uint8_t *pool, uint64_t stride, const tfo_expert_offsets *off, int fmt,
                         int bits, const float *x, const float *residual, const uint32_t *idx,
                         const float *w, int k, int d, int f, float *y) {
    float *out = (float *)malloc(sizeof(float) * (size_t)d);
    for (int i = 0; i < d; ++i) y[i] = residual ? residual[i] : 0.0f;
    for (int slot = 0; slot < k; ++slot) {
        ffn_affine(pool + (uint64_t)idx[slot] * stride, off, fmt, bits, x, d, f, out);
        for (int i = 0; i < d; ++i) {
            float scaled = out[i] * w[slot];      /* vDSP_vsmul */
            y[i] = y[i] + scaled;                 /* vDSP_vadd */
        }
    }
    free(out);
}

/* The shared expert: gate/up by the GEMV reference of `bits` (4: DequantInt4GemvRef,
 * 8: DequantInt8GemvRef), act = Float(Float16(Float(gelu) * u)) with the GELU
 * in double, then the down GEMV over act (T/Kernels/MoE/SharedExpertInt4Tests.swift:21-28,
 * SharedExpertInt8Tests.swift:57-68). round_gu: gate and up are first rounded
 * to fp16, as the reference's GPU sequence stores them (SharedExpertInt4's
 * fp16 scratchGate/scratchUp, SharedExpertInt4.swift:67-80 + utility.metal:7-18;
 * shared_int8_gate_up_act_simd, dequant_int8.metal:150-152). */
void tfo_shared_expert(const uint8_t *gW, const uint16_t *gS, const uint16_t *gB,
                       const uint8_t *uW, const uint16_t *uS, const uint16_t *uB,
                       const uint8_t *dW, const uint16_t *dS, const uint16_t *dB,
                       int fmt, int bits, int round_gu, const float *x, int d, int f, float *y) {
    float *g = (float *)malloc(sizeof(float) * (size_t)f);
    float *u = (float *)malloc(sizeof(float) * (size_t)f);
    float *act = (float *)malloc(sizeof(float) * (size_t)f);
    if (bits == 8) {
        tfo_gemv_int8(gW, gS, gB, fmt, x, f, d, g);
        tfo_gemv_int8(uW, uS, uB, fmt, x, f, d, u);
    } else {
        tfo_gemv_int4(gW, gS, gB, fmt, x, f, d, g);
        tfo_gemv_int4(uW, uS, uB, fmt, x, f, d, u);
    }
    for (int i = 0; i < f; ++i) {
        float gv = round_gu ? tfo_f16_to_f32(tfo_f32_to_f16(g[i])) : g[i];
        float uv = round_gu ? tfo_f16_to_f32(tfo_f32_to_f16(u[i])) : u[i];
        float cube = gv * gv;
        cube = cube * gv;
        float k3c = 0.044715f * cube;
        float inner_f = gv + k3c;
        double inner = 0.7978845608028654 * (double)inner_f;
        double gelu = 0.5 * (double)gv * (1.0 + tanh(inner));
        float prod = (float)gelu * uv;
        act[i] = tfo_f16_to_f32(tfo_f32_to_f16(prod));
    }
    if (bits == 8) tfo_gemv_int8(dW, dS, dB, fmt, act, d, f, y);
    else tfo_gemv_int4(dW, dS, dB, fmt, act, d, f, y);
    free(g); free(u); free(act);
}

/* T/Kernels/MoE/SharedExpertInt4Tests.swift:21-28 */
void tfo_shared_expert_int4(const uint8_t *gW, const uint16_t *gS, const uint16_t *gB,
                            const uint8_t *uW, const uint16_t *uS, const uint16_t *uB,
                            const uint8_t *dW, const uint16_t *dS, const uint16_t *dB,
                            int fmt, const float *x, int d, int f, float *y) {
    tfo_shared_expert(gW, gS, gB, uW, uS, uB, dW, dS, dB, fmt, 4, 0, x, d, f, y);
}

/* T/Kernels/MoE/SharedExpertInt8Tests.swift:57-68 */
void tfo_shared_expert_int8(const uint8_t *gW, const uint16_t *gS, const uint16_t *gB,
                            const uint8_t *uW, const uint16_t *uS, const uint16_t *uB,
                            const uint8_t *dW, const uint16_t *dS, const uint16_t *dB,
                            int fmt, const float *x, int d, int f, float *y) {
    tfo_shared_expert(gW, gS, gB, uW, uS, uB, dW, dS, dB, fmt, 8, 0, x, d, f, y);
}

/* ------------------------------------------------------------------------ */
/* Prefill grouping                                                          */
/* ------------------------------------------------------------------------ */

static const uint64_t *g_sort_keys;   /* comparator context (single-threaded use) */

/* PrefillMoEGrouping.swift:145-154: (sortKey[expert]?, expert, token, rank) ascending. */
static int pair_cmp(const void *pa, const void *pb) {
    const tfo_pair *a = (const tfo_pair *)pa, *b = (const tfo_pair *)pb;
    if (g_sort_keys) {
        uint64_t ka = g_sort_keys[a->expert], kb = g_sort_keys[b->expert];
        if (ka != kb) return ka < kb ? -1 : 1;
    }
    if (a->expert != b->expert) return a->expert < b->expert ? -1 : 1;
    if (a->token != b->token) return a->token < b->token ? -1 : 1;
    if (a->rank != b->rank) return a->rank < b->rank ? -1 : 1;
    return 0;
}

/* PrefillMoEGrouping.swift:91-192 */
int tfo_group_pairs(const tfo_pair *pairs, int64_t n_pairs, int64_t query_count, int64_t top_k,
                    int64_t num_experts, int64_t tile_expert_count,
                    const uint64_t *sort_keys, int64_t n_sort_keys,
                    tfo_pair *sorted, uint32_t *offsets, uint32_t *counts,
                    tfo_group *groups, int64_t *n_groups, tfo_tile *tiles, int64_t *n_tiles,
                    int64_t err[2]) {
    err[0] = err[1] = 0;
    if (query_count < 0) { err[0] = query_count; return TFO_GROUP_INVALID_QUERY_COUNT; }
    if (top_k <= 0) { err[0] = top_k; return TFO_GROUP_INVALID_TOPK; }
    if (num_experts <= 0) { err[0] = num_experts; return TFO_GROUP_INVALID_NUM_EXPERTS; }
    if (tile_expert_count < 1 || tile_expert_count > 16) {
        err[0] = tile_expert_count; return TFO_GROUP_INVALID_TILE_EXPERT_COUNT;
    }
    if (sort_keys && n_sort_keys != num_experts) {
        err[0] = num_experts; err[1] = n_sort_keys; return TFO_GROUP_SORT_KEY_COUNT_MISMATCH;
    }
    int64_t expected = query_count * top_k;
    if (n_pairs != expected) { err[0] = expected; err[1] = n_pairs; return TFO_GROUP_PAIR_COUNT_MISMATCH; }

    unsigned char *seen = (unsigned char *)calloc((size_t)(expected > 0 ? expected : 1), 1);
    for (int64_t i = 0; i < n_pairs; ++i) {
        const tfo_pair *p = &pairs[i];
        if ((int64_t)p->token >= query_count) { free(seen); err[0] = p->token; return TFO_GROUP_TOKEN_OUT_OF_RANGE; }
        if ((int64_t)p->rank >= top_k) { free(seen); err[0] = p->rank; return TFO_GROUP_RANK_OUT_OF_RANGE; }
        if ((int64_t)p->expert >= num_experts) { free(seen); err[0] = p->expert; return TFO_GROUP_EXPERT_OUT_OF_RANGE; }
        int64_t key = (int64_t)p->token * top_k + p->rank;
        if (seen[key]) { free(seen); err[0] = p->token; err[1] = p->rank; return TFO_GROUP_DUPLICATE_TOKEN_RANK; }
        seen[key] = 1;
    }
    free(seen);

    memcpy(sorted, pairs, sizeof(tfo_pair) * (size_t)n_pairs);
    g_sort_keys = sort_keys;
    qsort(sorted, (size_t)n_pairs, sizeof(tfo_pair), pair_cmp);
    g_sort_keys = NULL;

    for (int64_t e = 0; e < num_experts; ++e) { offsets[e] = 0xFFFFFFFFu; counts[e] = 0; }
    int64_t ng = 0;
    int64_t i = 0;
    while (i < n_pairs) {
        uint32_t expert = sorted[i].expert;
        int64_t start = i;
        while (i < n_pairs && sorted[i].expert == expert) ++i;
        offsets[expert] = (uint32_t)start;
        counts[expert] = (uint32_t)(i - start);
        groups[ng].expert = expert;
        groups[ng].pair_start = (uint32_t)start;
        groups[ng].pair_count = (uint32_t)(i - start);
        ++ng;
    }
    int64_t nt = 0;
    for (int64_t gs = 0; gs < ng;) {
        int64_t ge = gs + tile_expert_count < ng ? gs + tile_expert_count : ng;
        uint32_t ps = groups[gs].pair_start;
        uint32_t pe = groups[ge - 1].pair_start + groups[ge - 1].pair_count;
        tiles[nt].group_start = (uint32_t)gs;
        tiles[nt].group_count = (uint32_t)(ge - gs);
        tiles[nt].pair_start = ps;
        tiles[nt].pair_count = pe - ps;
        ++nt;
        gs = ge;
    }
    *n_groups = ng;
    *n_tiles = nt;
    return TFO_GROUP_OK;
}

int tfo_prefill_router(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                       const float *hidden, int hidden_stride, const float *eff,
                       const float *expert_scale, int T, int num_experts, int d, int k,
                       uint32_t *idx, float *weights) {
    float *logits = (float *)malloc(sizeof(float) * (size_t)num_experts);
    int rc = 0;
    for (int t = 0; t < T && rc == 0; ++t) {
        tfo_router_logits(W, S, B, fmt, hidden + (size_t)t * hidden_stride, eff, num_experts, d,
                          logits);
        rc = tfo_topk_softmax(logits, num_experts, k, expert_scale, idx + (size_t)t * k,
                              weights + (size_t)t * k);
    }
    free(logits);
    return rc;
}

/* cpuInt4Dot (PrefillGroupedRoutedMoETests.swift:281-303): acc += (q*s + b) * x. */
static float int4_dot_blob(const uint8_t *blob, uint32_t w_off, uint32_t s_off, uint32_t b_off,
                           int fmt, int bits, int row, int n, const float *x) {
    int groups = n / TFO_GROUP;
    size_t rb = tfo_affine_row_bytes((size_t)n, bits);
    const uint8_t *w_row = blob + w_off + (size_t)row * rb;
    const uint16_t *s_row = (const uint16_t *)(blob + s_off) + (size_t)row * groups;
    const uint16_t *b_row = (const uint16_t *)(blob + b_off) + (size_t)row * groups;
    float acc = 0.0f;
    for (int g = 0; g < groups; ++g) {
        float scale = tfo_decode_scale(s_row[g], fmt), bias = tfo_decode_scale(b_row[g], fmt);
        for (int k = 0; k < TFO_GROUP; ++k) {
            int col = g * TFO_GROUP + k;
            float q = (float)tfo_affine_code(w_row, rb, (size_t)col, bits);
            float w = q * scale;
            w = w + bias;
            float p = w * x[col];
            acc = acc + p;
        }
    }
    return acc;
}

/* PrefillGroupedRoutedMoETests.swift:229-279 */
void tfo_grouped_route_partials(const tfo_pair *sorted, int64_t n_pairs,
                                const uint16_t *hidden_f16, int hidden_stride,
                                const uint8_t *pool, uint64_t stride,
                                const tfo_expert_offsets *o, int fmt,
                                int top_k, int d, int f, uint16_t *partials) {
    tfo_grouped_route_partials_bits(sorted, n_pairs, hidden_f16, hidden_stride, pool, stride, o, fmt, 4,
                                    top_k, d, f, partials);
}

/* The same over experts of `bits`-bit rows (the b2/b3 grouped kernels,
 * prefill.metal:1223-1450, compute this per pair). */
void tfo_grouped_route_partials_bits(const tfo_pair *sorted, int64_t n_pairs,
                                     const uint16_t *hidden_f16, int hidden_stride,
                                     const uint8_t *pool, uint64_t stride,
                                     const tfo_expert_offsets *o, int fmt, int bits,
                                     int top_k, int d, int f, uint16_t *partials) {
#pragma omp parallel num_threads(tfo_threads) if (tfo_threads > 1)
    {
    float *x = (float *)malloc(sizeof(float) * (size_t)d);
    float *act = (float *)malloc(sizeof(float) * (size_t)f);
#pragma omp for schedule(dynamic, 4)
    for (int64_t p = 0; p < n_pairs; ++p) {
        const tfo_pair *pr = &sorted[p];
        const uint8_t *blob = pool + (uint64_t)pr->expert * stride;
        for (int i = 0; i < d; ++i)
            x[i] = tfo_f16_to_f32(hidden_f16[(size_t)pr->token * hidden_stride + i]);
        for (int r = 0; r < f; ++r) {
            float gate = int4_dot_blob(blob, o->gate_w, o->gate_s, o->gate_b, fmt, bits, r, d, x);
            float up = int4_dot_blob(blob, o->up_w, o->up_s, o->up_b, fmt, bits, r, d, x);
            float a = tfo_gelu_tanh(gate) * up;
            act[r] = tfo_f16_to_f32(tfo_f32_to_f16(a));
        }
        size_t out_base = ((size_t)pr->token * top_k + pr->rank) * d;
        for (int r = 0; r < d; ++r) {
            float v = int4_dot_blob(blob, o->down_w, o->down_s, o->down_b, fmt, bits, r, f, act);
            partials[out_base + r] = tfo_f32_to_f16(v);
        }
    }
    free(x); free(act);
    }
}

/* PrefillMoETests.swift:46-58 */
void tfo_reduce_token_major(const uint16_t *partials, const uint16_t *weights, int rows, int top_k,
                            int d, uint16_t *h2) {
    for (int t = 0; t < rows; ++t) {
        for (int c = 0; c < d; ++c) {
            float acc = 0.0f;
            for (int r = 0; r < top_k; ++r) {
                size_t pi = ((size_t)t * top_k + r) * d + c;
                float p = tfo_f16_to_f32(weights[t * top_k + r]) * tfo_f16_to_f32(partials[pi]);
                acc = acc + p;
            }
            h2[(size_t)t * d + c] = tfo_f32_to_f16(acc);
        }
    }
}

/* MPPPrefillInt4QMMTests.swift:80-105: weight = q*s + b (two roundings),
 * accumulator.addProduct(weight, x) (fused). */
void tfo_gemm_int4(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt,
                   const float *X, int M, int N, int K, float *Y, int row0, int row1) {
    tfo_gemm_affine(W, S, B, fmt, 4, X, M, N, K, Y, row0, row1);
}

/* tfo_gemm_int4 over `bits`-bit rows: the 3-bit prefill QMM
 * (prefill.metal:711-757) computes the same sum. */
void tfo_gemm_affine(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt, int bits,
                     const float *X, int M, int N, int K, float *Y, int row0, int row1) {
    int groups = K / TFO_GROUP;
    size_t row_bytes = tfo_affine_row_bytes((size_t)K, bits);
    if (row0 < 0) row0 = 0;
    if (row1 > M) row1 = M;
#pragma omp parallel for schedule(dynamic, 1) num_threads(tfo_threads) if (tfo_threads > 1)
    for (int t = row0; t < row1; ++t) {
        const float *xr = X + (size_t)t * K;
        for (int n = 0; n < N; ++n) {
            const uint8_t *wr = W + (size_t)n * row_bytes;
            float acc = 0.0f;
            for (int g = 0; g < groups; ++g) {
                float scale = tfo_decode_scale(S[(size_t)n * groups + g], fmt);
                float bias = tfo_decode_scale(B[(size_t)n * groups + g], fmt);
                for (int lk = 0; lk < TFO_GROUP; ++lk) {
                    int col = g * TFO_GROUP + lk;
                    float w = (float)tfo_affine_code(wr, row_bytes, (size_t)col, bits) * scale;
                    w = w + bias;
                    acc = fmaf(w, xr[col], acc);
                }
            }
            Y[(size_t)t * N + n] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Decode layer                                                              */
/* ------------------------------------------------------------------------ */

/* RmsNorm.swift:14-44 (vDSP_svesq, vDSP_vmul then vDSP_vsmul). */
void tfo_rmsnorm(const float *x, const float *w, int n, float eps, float *y) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    const float inv = 1.0f / sqrtf((float)(ss / (double)n) + eps);
    for (int i = 0; i < n; ++i) {
        float xw = w ? x[i] * w[i] : x[i];
        y[i] = xw * inv;
    }
}

/* logit.metal:706-716 (finite rows only), 758-763 / 743-746 (larger value,
 * then lower index), 784 (no finite value -> token 0). */
uint32_t tfo_greedy_argmax(const float *z, int n) {
    uint32_t best_i = 0xFFFFFFFFu;
    float best_v = -INFINITY;
    for (int i = 0; i < n; ++i) {
        if (!isfinite(z[i])) continue;
        if (best_i == 0xFFFFFFFFu || z[i] > best_v) {
            best_v = z[i];
            best_i = (uint32_t)i;
        }
    }
    return best_i == 0xFFFFFFFFu ? 0u : best_i;
}

/* LMHeadChainInt4.swift:105-134: RMSNorm into a half buffer, then the
 * int4 rows and the greedy reduction. */
uint32_t tfo_lm_head_greedy(const uint16_t *hidden_f16, const uint16_t *norm_w_f16, const uint8_t *W,
                            const uint16_t *S, const uint16_t *B, int fmt, int d, int vocab,
                            float eps, float *z) {
    float *h = (float *)calloc((size_t)d, sizeof(float));
    float *w = (float *)calloc((size_t)d, sizeof(float));
    float *x = (float *)calloc((size_t)d, sizeof(float));
    float *zz = z ? z : (float *)malloc(sizeof(float) * (size_t)vocab);
    for (int i = 0; i < d; ++i) {
        h[i] = tfo_f16_to_f32(hidden_f16[i]);
        w[i] = norm_w_f16 ? tfo_f16_to_f32(norm_w_f16[i]) : 1.0f;
    }
    tfo_rmsnorm(h, norm_w_f16 ? w : NULL, d, eps, x);
    for (int i = 0; i < d; ++i) x[i] = tfo_f16_to_f32(tfo_f32_to_f16(x[i]));
    tfo_gemv_int4(W, S, B, fmt, x, vocab, d, zz);
    const uint32_t token = tfo_greedy_argmax(zz, vocab);
    if (!z) free(zz);
    free(h);
    free(w);
    free(x);
    return token;
}

/* RoPE.swift:70-110 (applyNeox). */
void tfo_rope_neox(float *x, int num_heads, int head_dim, int rotated_pairs, int position,
                   float theta) {
    const int half = head_dim / 2;
    for (int i = 0; i < rotated_pairs; ++i) {
        const double ang = (double)position * pow((double)theta, -2.0 * (double)i / (double)head_dim);
        const float c = (float)cos(ang), sn = (float)sin(ang);
        for (int h = 0; h < num_heads; ++h) {
            float *b = x + (size_t)h * head_dim;
            const float x0 = b[i], x1 = b[half + i];
            b[i] = x0 * c - x1 * sn;
            b[half + i] = x0 * sn + x1 * c;
        }
    }
}

/* Attention.swift:14-104. */
void tfo_attention(const float *q, const float *k, const float *v, int hd, int nq, int nkv,
                   int seq_len, int window, float scale, float *out) {
    const int group = nq / nkv;
    const int start = (window > 0 && seq_len > window) ? seq_len - window : 0;
    const int n = seq_len - start;
#pragma omp parallel for schedule(static, 1) num_threads(tfo_threads) if (tfo_threads > 1)
    for (int qh = 0; qh < nq; ++qh) {
        double *p = (double *)malloc(sizeof(double) * (size_t)n);
        const int kvh = qh / group;
        const float *qv = q + (size_t)qh * hd;
        double mx = -INFINITY;
        for (int j = 0; j < n; ++j) {
            const float *kv = k + ((size_t)(start + j) * nkv + kvh) * hd;
            double dot = 0.0;
            for (int e = 0; e < hd; ++e) dot += (double)qv[e] * (double)kv[e];
            p[j] = dot * (double)scale;
            if (p[j] > mx) mx = p[j];
        }
        double sum = 0.0;
        for (int j = 0; j < n; ++j) {
            p[j] = exp(p[j] - mx);
            sum += p[j];
        }
        for (int e = 0; e < hd; ++e) {
            double acc = 0.0;
            for (int j = 0; j < n; ++j)
                acc += p[j] * (double)v[((size_t)(start + j) * nkv + kvh) * hd + e];
            out[(size_t)qh * hd + e] = (float)(acc / sum);
        }
        free(p);
    }
}

static float r16(float x) { return tfo_f16_to_f32(tfo_f32_to_f16(x)); }

static float *f16_to_f32_vec(const uint16_t *src, size_t n) {
    float *o = (float *)calloc(n ? n : 1, sizeof(float));
    for (size_t i = 0; i < n; ++i) o[i] = tfo_f16_to_f32(src[i]);
    return o;
}

static void round_vec(float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = r16(x[i]);
}

static void store_f16(uint16_t *dst, const float *x, size_t n) {
    if (!dst) return;
    for (size_t i = 0; i < n; ++i) dst[i] = tfo_f32_to_f16(x[i]);
}

/* rmsnorm of an fp32 vector with fp16 weights (NULL: no scale), rounded to fp16. */
static void norm16(const float *x, const uint16_t *w16, int n, float eps, float *y) {
    float *w = w16 ? f16_to_f32_vec(w16, (size_t)n) : NULL;
    tfo_rmsnorm(x, w, n, eps, y);
    round_vec(y, (size_t)n);
    free(w);
}

void tfo_decode_layer(const tfo_layer_weights *w, const tfo_layer_shape *s,
                      const uint16_t *hidden16, uint16_t *k_cache, uint16_t *v_cache, int position,
                      uint16_t *out16, uint32_t *idx_out, float *w_out, tfo_layer_trace *trace) {
    const int d = s->d, hd = s->hd, qd = s->nq * s->hd, kvd = s->nkv * s->hd;
    const int seq = position + 1;
    const float eps = s->eps;
    float *hidden = f16_to_f32_vec(hidden16, (size_t)d);
    float *normed = (float *)malloc(sizeof(float) * (size_t)d);
    float *q = (float *)malloc(sizeof(float) * (size_t)qd);
    float *kn = (float *)malloc(sizeof(float) * (size_t)kvd);
    float *vn = (float *)malloc(sizeof(float) * (size_t)kvd);

    /* gInputNorm + gQKV (RealForwardRunner.swift:2273-2300) */
    norm16(hidden, w->input_norm, d, eps, normed);
    tfo_gemv_int4(w->q.w, w->q.s, w->q.b, TFO_FMT_F16, normed, qd, d, q);
    tfo_gemv_int4(w->k.w, w->k.s, w->k.b, TFO_FMT_F16, normed, kvd, d, kn);
    /* v_proj exists only on the sliding-window layers; the full-attention
     * layers run k_proj as the v projection (:2252-2255), so V is the no-scale
     * norm of the raw k projection. */
    if (w->v.w)
        tfo_gemv_int4(w->v.w, w->v.s, w->v.b, TFO_FMT_F16, normed, kvd, d, vn);
    else
        memcpy(vn, kn, sizeof(float) * (size_t)kvd);
    round_vec(q, (size_t)qd);
    round_vec(kn, (size_t)kvd);
    round_vec(vn, (size_t)kvd);

    /* gQKVEpilogue (:2302-2322; fused.metal:86-180) */
    for (int h = 0; h < s->nq; ++h) norm16(q + (size_t)h * hd, w->q_norm, hd, eps, q + (size_t)h * hd);
    for (int h = 0; h < s->nkv; ++h) {
        norm16(kn + (size_t)h * hd, w->k_norm, hd, eps, kn + (size_t)h * hd);
        norm16(vn + (size_t)h * hd, NULL, hd, eps, vn + (size_t)h * hd);
    }
    tfo_rope_neox(q, s->nq, hd, s->rotated_pairs, position, s->theta);
    tfo_rope_neox(kn, s->nkv, hd, s->rotated_pairs, position, s->theta);
    round_vec(q, (size_t)qd);
    round_vec(kn, (size_t)kvd);
    store_f16(k_cache + (size_t)position * kvd, kn, (size_t)kvd);
    store_f16(v_cache + (size_t)position * kvd, vn, (size_t)kvd);
    if (trace) store_f16(trace->q, q, (size_t)qd);

    /* gAttention (:2324-2362) */
    float *K = f16_to_f32_vec(k_cache, (size_t)seq * kvd);
    float *V = f16_to_f32_vec(v_cache, (size_t)seq * kvd);
    float *attn = (float *)malloc(sizeof(float) * (size_t)qd);
    tfo_attention(q, K, V, hd, s->nq, s->nkv, seq, s->window, s->scale, attn);
    round_vec(attn, (size_t)qd);
    if (trace) store_f16(trace->attn, attn, (size_t)qd);
    free(K);
    free(V);

    /* gOProj + gPostAttnSetup (:2363-2386; fused.metal:199-268) */
    float *o = (float *)malloc(sizeof(float) * (size_t)d);
    float *an = (float *)malloc(sizeof(float) * (size_t)d);
    float *h = (float *)malloc(sizeof(float) * (size_t)d);
    tfo_gemv_int4(w->o.w, w->o.s, w->o.b, TFO_FMT_F16, attn, d, qd, o);
    round_vec(o, (size_t)d);
    norm16(o, w->post_attention_norm, d, eps, an);
    for (int i = 0; i < d; ++i) h[i] = r16(hidden[i] + an[i]);
    float *dense_x = (float *)malloc(sizeof(float) * (size_t)d);
    float *routed_x = (float *)malloc(sizeof(float) * (size_t)d);
    float *router_x = (float *)malloc(sizeof(float) * (size_t)d);
    norm16(h, w->pre_ffn_norm, d, eps, dense_x);
    norm16(h, w->pre_ffn2_norm, d, eps, routed_x);
    norm16(h, NULL, d, eps, router_x);
    if (trace) {
        store_f16(trace->o, o, (size_t)d);
        store_f16(trace->h, h, (size_t)d);
    }

    /* gRouter (:2388-2400): logits on router_x ⊙ eff, top-k softmax × gain */
    const int E = w->num_experts, k = s->k;
    float *eff = w->router_eff ? f16_to_f32_vec(w->router_eff, (size_t)d) : NULL;
    float *gain = w->router_gain ? f16_to_f32_vec(w->router_gain, (size_t)E) : NULL;
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    uint32_t idx[64];
    float rw[64];
    tfo_router_logits(w->router_w, w->router_s, w->router_b, TFO_FMT_F16, router_x, eff, E, d, logits);
    tfo_topk_softmax(logits, E, k, gain, idx, rw);
    for (int i = 0; i < k; ++i) {
        rw[i] = r16(rw[i]);
        if (idx_out) idx_out[i] = idx[i];
        if (w_out) w_out[i] = rw[i];
    }

    /* gSharedFFN + gSharedNorm (:2418-2440) */
    float *h1 = (float *)malloc(sizeof(float) * (size_t)d);
    tfo_shared_expert(w->shared_gate.w, w->shared_gate.s, w->shared_gate.b, w->shared_up.w, w->shared_up.s,
                      w->shared_up.b, w->shared_down.w, w->shared_down.s, w->shared_down.b, TFO_FMT_F16,
                      w->shared_bits == 8 ? 8 : 4, 0, dense_x, d, s->fs, h1);
    round_vec(h1, (size_t)d);
    /* routed phases (:2849-2862), zero residual */
    float *h2 = (float *)malloc(sizeof(float) * (size_t)d);
    tfo_moe_routed_bits(w->pool, w->stride, &w->off, TFO_FMT_F16, w->expert_bits ? w->expert_bits : 4, routed_x,
                        NULL, idx, rw, k, d, s->f, h2);
    round_vec(h2, (size_t)d);
    if (trace) {
        store_f16(trace->h1, h1, (size_t)d);
        store_f16(trace->h2, h2, (size_t)d);
    }

    /* gTail (fused.metal:270-375) */
    float *t = (float *)malloc(sizeof(float) * (size_t)d);
    float *h12 = (float *)malloc(sizeof(float) * (size_t)d);
    norm16(h1, w->post_ffn1_norm, d, eps, h12);
    norm16(h2, w->post_ffn2_norm, d, eps, t);
    for (int i = 0; i < d; ++i) h12[i] = r16(h12[i] + t[i]);
    norm16(h12, w->post_ffn_norm, d, eps, t);
    const float sc = r16(w->layer_scalar);
    for (int i = 0; i < d; ++i) out16[i] = tfo_f32_to_f16(r16(h[i] + t[i]) * sc);

    free(hidden); free(normed); free(q); free(kn); free(vn); free(attn); free(o); free(an); free(h);
    free(dense_x); free(routed_x); free(router_x); free(eff); free(gain); free(logits); free(h1);
    free(h2); free(t); free(h12);
}

/* ------------------------------------------------------------------------ */
/* Tolerance helpers (V/Tolerance/RelError.swift:7-27)                       */
/* ------------------------------------------------------------------------ */

float tfo_rel_error(const float *actual, const float *reference, size_t n) {
    float max_abs = 0.0f, ref_norm = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float d = fabsf(actual[i] - reference[i]);
        if (d > max_abs || d != d) max_abs = d;
        float r = fabsf(reference[i]);
        if (r > ref_norm) ref_norm = r;
    }
    return max_abs / (ref_norm > 1e-6f ? ref_norm : 1e-6f);
}

float tfo_max_abs_diff(const float *a, const float *b, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float d = fabsf(a[i] - b[i]);
        if (d > m || d != d) m = d;
    }
    return m;
}
