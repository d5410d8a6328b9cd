/*
 * tfq_oracle.h — CPU restatement of the reference's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libtfq, the HIP kernels,
 * the edgeexpert_amd package) links, loads or calls this library. It is the
 * checker: tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py use it to verify and to time the CPU path.
 *
 * Every function follows one reference function; the file:line it restates is
 * cited beside it (paths relative to the reference checkout):
 *   S/ = Sources/TurboFieldfare/
 *   V/ = Sources/TurboFieldfareValidation/Support/
 *   T/ = Tests/TurboFieldfare/Core/
 *
 * Scale/bias words: the reference stores BF16 scale and bias per group of 64
 * (S/Infrastructure/ModelIO/Quantization.swift:32-45); the MI355X library
 * stores fp16. Every dequantising function therefore takes `scale_fmt`
 * (TFO_FMT_F16 or TFO_FMT_BF16) and decodes the 16-bit words accordingly; the
 * arithmetic after decoding is the reference's.
 *
 * Floating point: this file is compiled with -ffp-contract=off so that
 * `a * b + c` rounds twice, exactly as Swift evaluates it; where the
 * reference calls a fused multiply-add (Swift `addProduct`, Metal `fma`)
 * the restatement calls fmaf explicitly.
 */
#ifndef TFQ_ORACLE_H
#define TFQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TFO_FMT_F16 = 0, TFO_FMT_BF16 = 1 };
enum { TFO_GROUP = 64 };

/* ---- PRNG (V/PRNG/SplitMix64.swift:11-23, V/PRNG/SeedTree.swift:12-19) ---- */
uint64_t tfo_splitmix64_next(uint64_t *state);
float tfo_splitmix64_uniform(uint64_t *state, float lo, float hi);
uint64_t tfo_seedtree_key(uint64_t root, const char *label);

/* ---- 16-bit float conversions ---- */
uint16_t tfo_f32_to_bf16(float x);            /* Quantization.swift:16-23 */
float tfo_bf16_to_f32(uint16_t bits);         /* Quantization.swift:25-28 */
uint16_t tfo_f32_to_f16(float x);             /* IEEE binary16, round-half-even (Swift Float16(_:)) */
float tfo_f16_to_f32(uint16_t bits);
float tfo_decode_scale(uint16_t bits, int scale_fmt);

/* ---- affine format (Quantization.swift:50-191) ---- */
void tfo_quantize_int4_row(const float *row, int n, uint8_t *packed,
                           uint16_t *scales_bf16, uint16_t *biases_bf16);
void tfo_quantize_int8_row(const float *row, int n, uint8_t *packed,
                           uint16_t *scales_bf16, uint16_t *biases_bf16);
void tfo_dequantize_int4_row(const uint8_t *packed, const uint16_t *scales,
                             const uint16_t *biases, int scale_fmt, int n, float *out);
void tfo_dequantize_int8_row(const uint8_t *packed, const uint16_t *scales,
                             const uint16_t *biases, int scale_fmt, int n, float *out);
uint32_t tfo_int4_code(const uint8_t *packed_row, size_t j);

/* ---- 2-, 3- and 4-bit rows (Quantization.swift:195-349) ---- */
size_t tfo_affine_row_bytes(size_t n, int bits);
void tfo_pack_affine_code(uint8_t *buf, size_t nbytes, uint32_t code, size_t j, int bits);
uint32_t tfo_affine_code(const uint8_t *row, size_t nbytes, size_t j, int bits);
void tfo_quantize_affine_row(const float *row, int n, int bits, uint8_t *packed,
                             uint16_t *scales_bf16, uint16_t *biases_bf16);
void tfo_dequantize_affine_row(const uint8_t *packed, const uint16_t *scales, const uint16_t *biases,
                               int scale_fmt, int bits, int n, float *out);

/* ---- GEMV: dequantise row to fp32, then fp32 dot in index order ----
 * V/Reference/Quant/DequantInt4Gemv.swift:12-42 and DequantInt8Gemv.swift:12-40
 * (vDSP_dotpr, pinned to a scalar index-order loop within 1e-5 by
 * T/Validation/Reference/DequantInt4GEMVReferenceTests.swift:38-53).
 * W rows are contiguous: row r starts at W + r*n/2 (int4) or W + r*n (int8);
 * scales/biases rows at S + r*n/64. The _f64 variants accumulate in double
 * (the "truth" used to bound the fp32 paths). */
void tfo_gemv_int4(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                   const float *x, int m, int n, float *y);
void tfo_gemv_int4_f64(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                       const float *x, int m, int n, double *y);
void tfo_gemv_int8(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                   const float *x, int m, int n, float *y);
void tfo_gemv_int8_f64(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                       const float *x, int m, int n, double *y);
/* tfo_gemv_int4 over 2-, 3- or 4-bit rows: row r starts at
 * W + r*tfo_affine_row_bytes(n, bits). */
void tfo_gemv_affine(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt, int bits,
                     const float *x, int m, int n, float *y);
/* Row-partitioned multithreaded variant of tfo_gemv_int4 (same per-row arithmetic). */
/* Threads of the row loops in the CPU-baseline build (no effect in the
 * checker build, which has no OpenMP); results do not depend on it. */
void tfo_set_threads(int n);

void tfo_gemv_int4_mt(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                      const float *x, int m, int n, float *y, int threads);

/* ---- router (T/Kernels/MoE/RouterTopKTests.swift:72-97) ----
 * logits = int8-GEMV(W, h ⊙ eff); eff == NULL means all ones. */
void tfo_router_logits(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                       const float *h, const float *eff, int num_experts, int d, float *logits);
/* sort (score desc, index asc), keep k, softmax over the k, × expert_scale
 * (NULL = ones). Returns 0, or -1 when k > num_experts or k <= 0. */
int tfo_topk_softmax(const float *logits, int num_experts, int k, const float *expert_scale,
                     uint32_t *idx, float *weights);

/* ---- MoE (V/Reference/MoE/Moe.swift:16-88) ---- */
float tfo_gelu_tanh(float x);                                 /* Moe.swift:21-29 */

typedef struct {
    uint32_t gate_w, gate_s, gate_b;
    uint32_t up_w, up_s, up_b;
    uint32_t down_w, down_s, down_b;
} tfo_expert_offsets;                                         /* S/Kernels/MoE/MoE.swift:4-29 */

/* runFFN (Moe.swift:33-52) for one expert blob: out = down(gelu(gate·x) ⊙ (up·x)). */
void tfo_ffn_int4(const uint8_t *blob, const tfo_expert_offsets *off, int scale_fmt,
                  const float *x, int d, int f, float *out);
/* applyStreamedRouted (Moe.swift:58-88): y = residual + Σ_slot w[slot]·ffn(expert idx[slot]).
 * Expert e's blob is pool + e*stride. residual == NULL means zeros. */
void tfo_moe_routed(const uint8_t *pool, uint64_t stride, const tfo_expert_offsets *off,
                    int scale_fmt, const float *x, const float *residual,
                    const uint32_t *idx, const float *w, int k, int d, int f, float *y);
/* tfo_moe_routed over experts whose rows hold `bits`-bit codes (2, 3, 4). */
void tfo_moe_routed_bits(const uint8_t *pool, uint64_t stride, const tfo_expert_offsets *off,
                         int scale_fmt, int bits, const float *x, const float *residual,
                         const uint32_t *idx, const float *w, int k, int d, int f, float *y);
/* Shared expert reference (T/Kernels/MoE/SharedExpertInt4Tests.swift:21-28):
 * gate/up by the GEMV reference, act rounded to fp16, down by the GEMV reference.
 * The GELU here is evaluated in double as that test does. */
void tfo_shared_expert_int4(const uint8_t *gW, const uint16_t *gS, const uint16_t *gB,
                            const uint8_t *uW, const uint16_t *uS, const uint16_t *uB,
                            const uint8_t *dW, const uint16_t *dS, const uint16_t *dB,
                            int scale_fmt, const float *x, int d, int f, float *y);
/* The shared expert at `bits` 4 or 8 (the two above are round_gu = 0);
 * round_gu = 1 rounds gate and up to fp16 before the activation, as the
 * reference's GPU sequence stores them (SharedExpertInt4.swift:67-80,
 * dequant_int8.metal:150-152). */
void tfo_shared_expert(const uint8_t *gW, const uint16_t *gS, const uint16_t *gB,
                       const uint8_t *uW, const uint16_t *uS, const uint16_t *uB,
                       const uint8_t *dW, const uint16_t *dS, const uint16_t *dB,
                       int scale_fmt, int bits, int round_gu, const float *x, int d, int f, float *y);
/* T/Kernels/MoE/SharedExpertInt8Tests.swift:57-68 (int8 gate/up/down) */
void tfo_shared_expert_int8(const uint8_t *gW, const uint16_t *gS, const uint16_t *gB,
                            const uint8_t *uW, const uint16_t *uS, const uint16_t *uB,
                            const uint8_t *dW, const uint16_t *dS, const uint16_t *dB,
                            int scale_fmt, const float *x, int d, int f, float *y);

/* ---- prefill grouping (S/Kernels/Prefill/MoE/PrefillMoEGrouping.swift:91-192) ---- */
typedef struct { uint32_t token, expert, rank, weight_bits; } tfo_pair;   /* PrefillRouter.swift:5-28 */
typedef struct { uint32_t expert, pair_start, pair_count; } tfo_group;   /* PrefillMoEGrouping.swift:3-14 */
typedef struct { uint32_t group_start, group_count, pair_start, pair_count; } tfo_tile; /* :16-29 */

enum {
    TFO_GROUP_OK = 0,
    TFO_GROUP_INVALID_QUERY_COUNT = 1,
    TFO_GROUP_INVALID_TOPK = 2,
    TFO_GROUP_INVALID_NUM_EXPERTS = 3,
    TFO_GROUP_INVALID_TILE_EXPERT_COUNT = 4,
    TFO_GROUP_PAIR_COUNT_MISMATCH = 5,
    TFO_GROUP_TOKEN_OUT_OF_RANGE = 6,
    TFO_GROUP_RANK_OUT_OF_RANGE = 7,
    TFO_GROUP_EXPERT_OUT_OF_RANGE = 8,
    TFO_GROUP_DUPLICATE_TOKEN_RANK = 9,
    TFO_GROUP_SORT_KEY_COUNT_MISMATCH = 10,
};

/* Returns a TFO_GROUP_* code; on error err[0], err[1] carry the values the
 * Swift error case carries. sort_keys may be NULL; n_sort_keys is its length.
 * Outputs: sorted[n_pairs], offsets[num_experts], counts[num_experts],
 * groups[<= num_experts], tiles[<= num_experts]. */
int tfo_group_pairs(const tfo_pair *pairs, int64_t n_pairs, int64_t query_count, int64_t top_k,
                    int64_t num_experts, int64_t tile_expert_count,
                    const uint64_t *sort_keys, int64_t n_sort_keys,
                    tfo_pair *sorted, uint32_t *offsets, uint32_t *counts,
                    tfo_group *groups, int64_t *n_groups, tfo_tile *tiles, int64_t *n_tiles,
                    int64_t err[2]);

/* Per-token block router (S/Metal/Prefill/prefill.metal:478-573 semantics,
 * restated with the decode router reference per token): idx/w are [T][k]. */
int tfo_prefill_router(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                       const float *hidden, int hidden_stride, const float *eff,
                       const float *expert_scale, int T, int num_experts, int d, int k,
                       uint32_t *idx, float *weights);

/* cpuSyntheticRoutePartials (T/Kernels/Prefill/PrefillGroupedRoutedMoETests.swift:229-303):
 * for each sorted pair, act = fp16(gelu(gate)·up), partial = fp16(down·act),
 * written at partials[(token*top_k + rank)*d + row]. hidden is fp16 bits. */
void tfo_grouped_route_partials(const tfo_pair *sorted, int64_t n_pairs,
                                const uint16_t *hidden_f16, int hidden_stride,
                                const uint8_t *pool, uint64_t stride,
                                const tfo_expert_offsets *off, int scale_fmt,
                                int top_k, int d, int f, uint16_t *partials_f16);
/* tfo_grouped_route_partials over experts of `bits`-bit rows (2, 3, 4). */
void tfo_grouped_route_partials_bits(const tfo_pair *sorted, int64_t n_pairs,
                                     const uint16_t *hidden_f16, int hidden_stride,
                                     const uint8_t *pool, uint64_t stride,
                                     const tfo_expert_offsets *off, int scale_fmt, int bits,
                                     int top_k, int d, int f, uint16_t *partials);

/* cpuReduce (T/Kernels/Prefill/PrefillMoETests.swift:46-58). */
void tfo_reduce_token_major(const uint16_t *partials_f16, const uint16_t *weights_f16,
                            int rows, int top_k, int d, uint16_t *h2_f16);

/* MPP GEMM cpuReference (T/Kernels/TensorCore/MPPPrefillInt4QMMTests.swift:80-105):
 * Y[t][n] = Σ_k fma(q·s + b, X[t][k]) over k in index order (fp32, unrounded).
 * Rows of Y in [row0, row1) are computed (a bounded sample for timing). */
void tfo_gemm_int4(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt,
                   const float *X, int M, int N, int K, float *Y, int row0, int row1);
/* tfo_gemm_int4 over `bits`-bit rows (2, 3, 4). */
void tfo_gemm_affine(const uint8_t *W, const uint16_t *S, const uint16_t *B, int scale_fmt, int bits,
                     const float *X, int M, int N, int K, float *Y, int row0, int row1);

/* ---- decode layer (config 4) ----
 * RmsNormRef.apply (V/Reference/Primitives/RmsNorm.swift:14-44):
 *   y[i] = x[i] * w[i] * 1/sqrt(Σx²/n + eps); w == NULL: no scale (the
 *   rmsnorm_no_scale form of S/Metal/Fusions/fused.metal:86-180). */
void tfo_rmsnorm(const float *x, const float *w, int n, float eps, float *y);
/* ---- greedy int4 LM head (S/Metal/Sampling/logit.metal:688-787,
 * S/Kernels/Fusions/LMHeadChainInt4.swift:62-135) ----
 * tfo_greedy_argmax: the index of the largest finite z[i], the lowest index
 * among equal values (logit.metal:713-716,758-763); 0 when no z is finite
 * (logit.metal:784). tfo_lm_head_greedy: normed = f16(rmsnorm(hidden,
 * norm_w)) (the reference's half xNormed buffer; norm_w NULL: no scale),
 * z = tfo_gemv_int4 rows
 * over it, token = tfo_greedy_argmax(z); z (may be NULL) receives the
 * vocab logits. */
uint32_t tfo_greedy_argmax(const float *z, int n);
uint32_t tfo_lm_head_greedy(const uint16_t *hidden_f16, const uint16_t *norm_w_f16, const uint8_t *W,
                            const uint16_t *S, const uint16_t *B, int scale_fmt, int d, int vocab,
                            float eps, float *z);
/* RopeRef.applyNeox (V/Reference/Attention/RoPE.swift:70-110), in place over
 * num_heads heads: pairs (i, i + head_dim/2), i < rotated_pairs, rotated by
 * position * theta^(-2i/head_dim). The angle and its cos/sin are evaluated
 * in double (the reference's vForce tables carry fp32 angle error at long
 * positions). */
void tfo_rope_neox(float *x, int num_heads, int head_dim, int rotated_pairs, int position,
                   float theta);
/* AttentionRef.apply (V/Reference/Attention/Attention.swift:14-104):
 * q [nq][hd], k/v [seq_len][nkv][hd] (fp32), out [nq][hd]; keys
 * [max(0, seq_len - window), seq_len) (window 0: all). Dot products and the
 * output sums accumulate in double; softmax is the stable form. */
void tfo_attention(const float *q, const float *k, const float *v, int head_dim, int nq, int nkv,
                   int seq_len, int window, float scale, float *out);

typedef struct {
    const uint8_t *w;
    const uint16_t *s, *b;
} tfo_q4;

/* Gemma 4 decoder-layer weights (fp16 bits for every norm weight). */
typedef struct {
    const uint16_t *input_norm;
    tfo_q4 q, k, v, o;
    const uint16_t *q_norm, *k_norm;
    const uint16_t *post_attention_norm, *pre_ffn_norm, *pre_ffn2_norm;
    const uint8_t *router_w;
    const uint16_t *router_s, *router_b, *router_eff, *router_gain;  /* eff/gain may be NULL */
    int num_experts;
    const uint8_t *pool;
    uint64_t stride;
    tfo_expert_offsets off;
    tfo_q4 shared_gate, shared_up, shared_down;
    const uint16_t *post_ffn1_norm, *post_ffn2_norm, *post_ffn_norm;
    float layer_scalar;
    int expert_bits;    /* code width of the routed experts: 2, 3 or 4 (0 reads as 4) */
    int shared_bits;    /* shared expert: 4 (int4, also 0) or 8 (int8 rows of d bytes), Model.swift:59 */
} tfo_layer_weights;

typedef struct {
    int d, nq, nkv, hd, rotated_pairs, window, f, fs, k;
    float eps, theta, scale;
} tfo_layer_shape;

/* Optional intermediate outputs (each may be NULL), fp16 bits. */
typedef struct {
    uint16_t *q;        /* [nq*hd] after the epilogue */
    uint16_t *attn;     /* [nq*hd] attention output */
    uint16_t *o;        /* [d] o projection */
    uint16_t *h;        /* [d] post-attention residual stream */
    uint16_t *h1;       /* [d] shared-expert output */
    uint16_t *h2;       /* [d] routed output */
} tfo_layer_trace;

/* One decoder layer for the token at `position`, composed from the
 * references above in the per-layer order of RealForwardRunner
 * (S/Runtime/Inference/RealForwardRunner.swift:2273-2862) with an fp16
 * rounding wherever that sequence stores a buffer:
 *   normed = f16(rmsnorm(hidden, input_norm)); q,k,v = f16(GEMV(·, normed))
 *   q,k = f16(rope(f16(rmsnorm_head(·, q_norm/k_norm)))); v = f16(rmsnorm_head(v))
 *   (k, v stored into cache slot `position`)
 *   attn = f16(attention(q, K[0..position], V[0..position]))
 *   o = f16(GEMV(o_proj, attn)); h = f16(hidden + f16(rmsnorm(o, post_attention_norm)))
 *   router on f16(rmsnorm(h)) (no scale), weights rounded to fp16
 *   h1 = f16(shared(f16(rmsnorm(h, pre_ffn_norm)))) (the CPU references' shared
 *        expert, gate/up in fp32), int4 or int8 rows by shared_bits
 *   h2 = f16(Σ w·ffn(f16(rmsnorm(h, pre_ffn2_norm))))
 *   h12 = f16(f16(rmsnorm(h1, post_ffn1)) + f16(rmsnorm(h2, post_ffn2)))
 *   out = f16(f16(h + f16(rmsnorm(h12, post_ffn))) * f16(layer_scalar))
 * (fused.metal:86-375 for the fusion boundaries). Caches are fp16 bits
 * [capacity][nkv][hd]. idx/w (may be NULL) receive the routing. */
void tfo_decode_layer(const tfo_layer_weights *w, const tfo_layer_shape *s,
                      const uint16_t *hidden, uint16_t *k_cache, uint16_t *v_cache, int position,
                      uint16_t *out, uint32_t *idx, float *weights, tfo_layer_trace *trace);

/* RelError.compute (V/Tolerance/RelError.swift:7-16). */
float tfo_rel_error(const float *actual, const float *reference, size_t n);
float tfo_max_abs_diff(const float *a, const float *b, size_t n);

#ifdef __cplusplus
}
#endif
#endif
