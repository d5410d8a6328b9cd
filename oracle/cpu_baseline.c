/*
 * cpu_baseline.c — the reference's CPU path for BASELINE configs 0 and 1,
 * row-partitioned over host threads, for the CPU baseline that bench.py
 * times beside the GPU. TEST AND MEASUREMENT INFRASTRUCTURE ONLY: built into
 * oracle/libtfq_cpu_baseline.so (-O3 -march=native on the host that runs it,
 * -ffp-contract=off kept), never linked into the product.
 *
 * Every output row is computed by the oracle's own row function
 * (tfo_gemv_affine / tfo_gemv_int8 on that row; DequantInt4GemvRef.apply,
 * V/Reference/Quant/DequantInt4Gemv.swift:12-42, DequantInt8GemvRef.apply,
 * DequantInt8Gemv.swift:12-40), so the results equal the serial oracle's
 * bit for bit at any thread count; threads only split the rows
 * (the "all host cores" form of the reference path). The MoE token follows
 * RouterTopKTests.reference (T/Kernels/MoE/RouterTopKTests.swift:72-97) and
 * MoeRef.applyStreamedRouted (V/Reference/MoE/Moe.swift:58-88).
 */
#include <math.h>
#include <omp.h>
#include <stdlib.h>

#include "tfq_oracle.h"

/* y[r] for r < m of an affine g64 matrix (bits 2/3/4, or 8 = int8 rows). */
static void gemv_rows_mt(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt, int bits,
                         const float *x, int m, int n, float *y, int threads) {
    const size_t rb = bits == 8 ? (size_t)n : tfo_affine_row_bytes((size_t)n, bits);
    const size_t groups = (size_t)n / TFO_GROUP;
    /* a few rows per task: the per-call scratch of the row function is small */
    const int chunk = 16;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int r0 = 0; r0 < m; r0 += chunk) {
        const int rows = r0 + chunk <= m ? chunk : m - r0;
        if (bits == 8)
            tfo_gemv_int8(W + r0 * rb, S + r0 * groups, B + r0 * groups, fmt, x, rows, n, y + r0);
        else
            tfo_gemv_affine(W + r0 * rb, S + r0 * groups, B + r0 * groups, fmt, bits, x, rows, n, y + r0);
    }
}

/* BASELINE config 0: the int4 g64 GEMV. */
void tfb_gemv_int4(const uint8_t *W, const uint16_t *S, const uint16_t *B, int fmt, const float *x, int m,
                   int n, float *y, int threads) {
    gemv_rows_mt(W, S, B, fmt, 4, x, m, n, y, threads);
}

/* BASELINE config 1: one decode token through the routed MoE block — the
 * int8 router over h (effective scale 1), top-k softmax, then each selected
 * expert's FFN (gate/up rows, GeGLU, down rows) added in slot order. idx/w
 * receive the routing; y the block output (residual NULL = zeros). */
void tfb_moe_decode_token(const uint8_t *rW, const uint16_t *rS, const uint16_t *rB, int num_experts,
                          const uint8_t *pool, uint64_t stride, const tfo_expert_offsets *o, int fmt,
                          const float *h, const float *residual, int d, int f, int k, uint32_t *idx, float *w,
                          float *y, int threads) {
    float *logits = (float *)malloc(sizeof(float) * (size_t)num_experts);
    float *gate = (float *)malloc(sizeof(float) * (size_t)f);
    float *up = (float *)malloc(sizeof(float) * (size_t)f);
    float *act = (float *)malloc(sizeof(float) * (size_t)f);
    float *out = (float *)malloc(sizeof(float) * (size_t)d);
    gemv_rows_mt(rW, rS, rB, fmt, 8, h, num_experts, d, logits, threads);
    tfo_topk_softmax(logits, num_experts, k, NULL, idx, w);
    for (int i = 0; i < d; ++i) y[i] = residual ? residual[i] : 0.0f;
    for (int slot = 0; slot < k; ++slot) {
        const uint8_t *blob = pool + (uint64_t)idx[slot] * stride;
        gemv_rows_mt(blob + o->gate_w, (const uint16_t *)(blob + o->gate_s), (const uint16_t *)(blob + o->gate_b),
                     fmt, 4, h, f, d, gate, threads);
        gemv_rows_mt(blob + o->up_w, (const uint16_t *)(blob + o->up_s), (const uint16_t *)(blob + o->up_b), fmt,
                     4, h, f, d, up, threads);
        for (int i = 0; i < f; ++i) act[i] = tfo_gelu_tanh(gate[i]) * up[i];
        gemv_rows_mt(blob + o->down_w, (const uint16_t *)(blob + o->down_s), (const uint16_t *)(blob + o->down_b),
                     fmt, 4, act, d, f, out, threads);
        for (int i = 0; i < d; ++i) {
            float scaled = out[i] * w[slot];
            y[i] = y[i] + scaled;
        }
    }
    free(logits); free(gate); free(up); free(act); free(out);
}
