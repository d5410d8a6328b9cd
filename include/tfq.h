/*
 * tfq.h — C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * Drop-in replacement for the Metal quantized-matmul entry points of the
 * TurboFieldfare / edgeexpert runtime. Each entry point below names the
 * reference wrapper it replaces (paths relative to the reference checkout,
 * S/ = Sources/TurboFieldfare/).
 *
 * Conventions (shared by every entry point)
 *  - Weight format: MLX affine, group 64 along the reduction axis. int4 rows
 *    pack 2 codes per byte (low nibble = even element), i.e. 8 codes per
 *    little-endian uint32 word along K; int8 rows hold one code per byte.
 *    Scale and bias are IEEE fp16, one pair per group: w = q*scale + bias.
 *    (The reference stores BF16; BF16 -> fp16 is exact for |v| in
 *    [2^-14, 65504], see tfq_convert_bf16_to_f16.)
 *  - Axis names follow the reference wrappers: for a GEMV `m` is the number
 *    of output rows and `n` the reduction length (DequantInt4GEMV.swift:95-96);
 *    for a GEMM `t`/`m` counts tokens, `n` outputs, `k` the reduction.
 *  - All pointers are device pointers (hipMalloc'd), all work is enqueued
 *    asynchronously on `stream` (a hipStream_t; NULL = the null stream).
 *    The caller owns every buffer; nothing is allocated per call.
 *  - Every call returns a status. Shape, alignment and null-pointer contract
 *    violations return TFQ_E_INVAL (the reference traps with `precondition`);
 *    shapes no kernel is compiled for return TFQ_E_UNSUPPORTED; a failing
 *    HIP call returns TFQ_E_HIP and its code is kept for tfq_last_hip_error().
 *    Nothing aborts the process.
 *  - A context is immutable after tfq_create and may be shared by threads
 *    that use distinct streams: every call runs on the caller's stream alone.
 *    Calls that take a `workspace` must not run concurrently with another
 *    call using the same workspace.
 *  - ABI versions (TFQ_ABI_VERSION, tfq_abi_version()): a binding built
 *    against one version must check the library's at load time. Version 2
 *    widened the grouping state of tfq_moe_group / tfq_moe_grouped from 1 to
 *    TFQ_MOE_GROUP_STATE_WORDS words and added tfq_decode_layer_weights
 *    .shared_bits; version 3 added the staged k/v segment at the end of the
 *    tfq_decode_layer workspace (tfq_decode_layer_workspace_bytes grew),
 *    head_dim 512 and a NULL v_proj (V from the k projection); version 4
 *    moved the tfq_decode_layer workspace's o, h1, h2 segments to its
 *    start and added tfq_decode_layers.
 */
#ifndef TFQ_H
#define TFQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TFQ_OK 0
#define TFQ_E_INVAL 1
#define TFQ_E_UNSUPPORTED 2
#define TFQ_E_HIP 3
#define TFQ_E_NOT_LOADED 4
#define TFQ_E_IO 5          /* a checkpoint file is missing, unreadable or short (tfq_loader.h) */

#define TFQ_GROUP_SIZE 64

/* Version of this header's structs and contracts; tfq_abi_version() returns
 * the library's. No reference counterpart (the Swift wrappers and their
 * shaders ship in one build). */
#define TFQ_ABI_VERSION 4
int tfq_abi_version(void);

typedef struct tfq_ctx tfq_ctx;

/* Loads the gfx950 code objects (tfq_*.co, one per kernel translation unit)
 * and resolves every kernel (hipModuleLoad + hipModuleGetFunction) on the
 * current device. code_object_path: the directory holding them, or a file in
 * that directory; NULL = the directory holding libtfq.so. Replaces
 * MetalContext pipeline creation (S/Infrastructure/Metal/MetalContext.swift:104-201). */
int tfq_create(tfq_ctx **out, const char *code_object_path);
void tfq_destroy(tfq_ctx *ctx);
const char *tfq_status_string(int status);
/* hipError_t of the last failing HIP call on this thread (0 if none). */
int tfq_last_hip_error(void);
/* Human-readable reason of the last non-OK status on this thread. */
const char *tfq_last_error_message(void);

/* ---------------------------------------------------------------- decode -- */

/* y[m] = W[m][n] · x[n]; int4 g64 weights, fp16 x/y, fp32 accumulate.
 * Replaces DequantInt4GEMV.encode and .encodeTgx
 * (S/Kernels/Quant/DequantInt4GEMV.swift:84-180).
 * Contract: n % 64 == 0, n <= 8192, m >= 1, weights 16-byte aligned,
 * scales/biases/x/y 2-byte aligned. A 16-byte aligned x runs the kernel form
 * whose staging is fixed at compile time (faster); a 2-byte aligned one the
 * form that reads it at run time. */
int tfq_gemv_q4g64(tfq_ctx *ctx, void *stream, const void *weights, const uint16_t *scales,
                   const uint16_t *biases, const uint16_t *x, uint16_t *y, uint32_t m,
                   uint32_t n);

/* One int4 matrix (weights, scales, biases). */
typedef struct {
    const void *weights;
    const uint16_t *scales;
    const uint16_t *biases;
} tfq_q4_matrix;

/* q, k and v projections of one token in one launch over the concatenated
 * rows mq + 2*mkv. Replaces FusedQKVGEMV.encode
 * (S/Kernels/Fusions/FusedQKVGEMV.swift:92-156). Same contract as
 * tfq_gemv_q4g64 for each matrix. */
int tfq_gemv_q4g64_qkv(tfq_ctx *ctx, void *stream, const tfq_q4_matrix *q,
                       const tfq_q4_matrix *k, const tfq_q4_matrix *v, const uint16_t *x,
                       uint16_t *yq, uint16_t *yk, uint16_t *yv, uint32_t mq, uint32_t mkv,
                       uint32_t n);

/* tfq_gemv_q4g64 at `bits` = 3 or 4 bits per code (rows of n*bits/8 bytes,
 * codes packed from the least significant bit, Quantization.swift:195-201).
 * Replaces DequantInt4GEMV.encode(..., bits:) with its 3-bit kernels
 * (DequantInt4GEMV.swift:140-180, dequant_int4.metal:512-717). Other bit
 * widths: TFQ_E_INVAL (the reference's precondition, :149-150). */
int tfq_gemv_qg64(tfq_ctx *ctx, void *stream, const void *weights, const uint16_t *scales,
                  const uint16_t *biases, const uint16_t *x, uint16_t *y, uint32_t m, uint32_t n,
                  uint32_t bits);

/* tfq_gemv_q4g64_qkv at `bits` = 3 or 4. Replaces FusedQKVGEMV.encode(...,
 * bits:) (FusedQKVGEMV.swift:100-156). */
int tfq_gemv_qg64_qkv(tfq_ctx *ctx, void *stream, const tfq_q4_matrix *q, const tfq_q4_matrix *k,
                      const tfq_q4_matrix *v, const uint16_t *x, uint16_t *yq, uint16_t *yk,
                      uint16_t *yv, uint32_t mq, uint32_t mkv, uint32_t n, uint32_t bits);

/* y[m] = W8[m][n] · x[n]; int8 g64 weights. Replaces DequantInt8GEMV.encode
 * (S/Kernels/Quant/DequantInt8GEMV.swift:50-81).
 * Contract: n % 64 == 0, n <= 4096, weights 16-byte aligned. A 16-byte
 * aligned x runs the form whose staging is fixed at compile time. */
int tfq_gemv_q8g64(tfq_ctx *ctx, void *stream, const uint8_t *weights, const uint16_t *scales,
                   const uint16_t *biases, const uint16_t *x, uint16_t *y, uint32_t m,
                   uint32_t n);

/* Bytes of workspace tfq_router_topk needs (holds the fp32 logits when
 * out_logits_f32 is NULL). */
#define TFQ_ROUTER_WORKSPACE_BYTES 4096u

/* Bytes of workspace tfq_lm_head_greedy needs (per-block argmax summaries). */
#define TFQ_LM_HEAD_WORKSPACE_BYTES 65536u

/* Greedy decode head: out_token[0] = the vocab row with the largest finite
 * z = W·f16(rmsnorm(hidden, norm_weight)) (z in fp32; W int4 g64
 * [vocab][d]), the lowest row among equal z (-0 equals +0), 0 when no z is
 * finite. norm_weight may be NULL (no scale). Two launches on `stream`: the
 * rows with the RMSNorm folded into their activation staging and a
 * per-block argmax, then a one-block reduce. Replaces
 * LMHeadChainInt4.encodeGreedyDecode
 * (S/Kernels/Fusions/LMHeadChainInt4.swift:62-135; kernels
 * S/Metal/Sampling/logit.metal:688-787; its separate RMSNorm launch is
 * folded in). Contract: d % 64 == 0, d <= 8192, vocab >= 1, eps > 0,
 * weights 16-byte aligned, out_token 4-byte aligned, workspace
 * TFQ_LM_HEAD_WORKSPACE_BYTES bytes, 8-byte aligned. A 16-byte aligned
 * hidden (and norm_weight) with d <= 4096 runs the rows form whose RMSNorm
 * staging is fixed at compile time (faster; the same token). */
int tfq_lm_head_greedy(tfq_ctx *ctx, void *stream, const uint16_t *hidden,
                       const uint16_t *norm_weight, const void *weights, const uint16_t *scales,
                       const uint16_t *biases, uint32_t *out_token, uint32_t d, uint32_t vocab,
                       float eps, void *workspace);

/* Router GEMV, then top-k + softmax over the k + per-expert gain (two
 * launches on `stream`: a many-block int8 GEMV and a one-wavefront select).
 * logits[e] = Σ_g s·Σ q·(h⊙eff) + b·Σ(h⊙eff) (fp32); indices sorted by
 * logit descending, ties to the lower expert index; weights[i] =
 * fp16(softmax_i × per_expert_scale[idx_i]). effective_scale /
 * per_expert_scale may be NULL (= all ones). Replaces MoE.encodeRouterGemma4
 * (S/Kernels/MoE/MoE.swift:147-197).
 * Contract: d % 64 == 0, d <= 4096, 1 <= num_experts <= 256,
 * 1 <= top_k <= 64 (the reference decode path requires top_k == 8),
 * weights 16-byte aligned. out_logits_f32 (may be NULL) receives the fp32
 * logits; out_weights_f32 (may be NULL) the unrounded weights. */
int tfq_router_topk(tfq_ctx *ctx, void *stream, const uint8_t *weights, const uint16_t *scales,
                    const uint16_t *biases, const uint16_t *hidden,
                    const uint16_t *effective_scale, const uint16_t *per_expert_scale,
                    uint32_t *out_indices, uint16_t *out_weights, float *out_weights_f32,
                    float *out_logits_f32, uint32_t num_experts, uint32_t d, uint32_t top_k,
                    void *workspace);

/* The router GEMV alone: logits[e] (fp32) as in tfq_router_topk
 * (router_gemv_gemma4_r4, S/Metal/MoE/moe.metal:78-133). Same contract. */
int tfq_router_logits(tfq_ctx *ctx, void *stream, const uint8_t *weights, const uint16_t *scales,
                      const uint16_t *biases, const uint16_t *hidden, const uint16_t *effective_scale,
                      float *logits, uint32_t num_experts, uint32_t d);

/* Sub-tensor byte offsets inside one routed-expert blob
 * (MoEExpertOffsets, S/Kernels/MoE/MoE.swift:4-29). */
typedef struct {
    uint32_t gate_w, gate_s, gate_b;
    uint32_t up_w, up_s, up_b;
    uint32_t down_w, down_s, down_b;
} tfq_expert_offsets;

/* All routed experts of one layer, resident in HBM: expert e's blob starts
 * at base + e*stride. Replaces the argument buffer of per-slot blob
 * pointers (S/Kernels/MoE/MoE.swift:398-409): the address is computed on the
 * device from the router's index buffer, so no host round trip is needed.
 * weight_bits: code width of every gate/up/down row, 2, 3 or 4 (0 means 4,
 * the default of the reference's `bits:` argument, MoE.swift:244,281,324);
 * a row of n codes takes n*bits/8 bytes, codes packed from the least
 * significant bit (Quantization.swift:195-201). The decode
 * and grouped prefill entry points run every width.
 * Contract: base, stride and the *_w offsets 16-byte aligned; *_s and *_b
 * offsets 2-byte aligned. */
typedef struct {
    const void *base;
    uint64_t stride;
    uint32_t num_experts;
    tfq_expert_offsets offsets;
    uint32_t weight_bits;
} tfq_expert_pool;

/* Phase 1: acts[slot][f] = fp16(gelu_tanh(gate_e[f]·x) * (up_e[f]·x)), e =
 * indices[slot], fp32 accumulate; acts is fp16 [top_k][f] (moe.metal:368).
 * An out-of-range expert index yields NaN activations instead of a fault.
 * Replaces MoE.encodeRoutedPersistentPhase1U16Load (MoE.swift:234-266).
 * Contract: d % 64 == 0, d <= 8192, f % 64 == 0, 1 <= top_k <= 8. */
int tfq_moe_phase1(tfq_ctx *ctx, void *stream, const tfq_expert_pool *pool,
                   const uint32_t *indices, const uint16_t *x, uint16_t *acts, uint32_t d,
                   uint32_t f, uint32_t top_k);

/* Phase 1 over a subset of slots (active_slots: device uint32 [active_count]).
 * Replaces MoE.encodeRoutedPersistentPhase1SubsetU16Load (MoE.swift:268-310). */
int tfq_moe_phase1_subset(tfq_ctx *ctx, void *stream, const tfq_expert_pool *pool,
                          const uint32_t *indices, const uint16_t *x, uint16_t *acts,
                          const uint32_t *active_slots, uint32_t active_count, uint32_t d,
                          uint32_t f, uint32_t top_k);

/* Phase 1 with the router's selection folded in: every block selects the
 * top_k experts from `logits` exactly as tfq_router_topk does (identical
 * results in every block) and block 0 writes out_indices / out_weights
 * (fp16) / out_weights_f32 (may be NULL). One launch replaces
 * router_topk_select_k8 + Phase1U16Load (S/Metal/MoE/moe.metal:135-185,
 * S/Kernels/MoE/MoE.swift:147-266). Contract: as tfq_moe_phase1;
 * num_experts == pool->num_experts <= 256. */
int tfq_moe_phase1_routed(tfq_ctx *ctx, void *stream, const tfq_expert_pool *pool,
                          const float *logits, const uint16_t *per_expert_scale,
                          uint32_t num_experts, uint32_t *out_indices, uint16_t *out_weights,
                          float *out_weights_f32, const uint16_t *x, uint16_t *acts, uint32_t d,
                          uint32_t f, uint32_t top_k);

/* Phase 2: y[d] = fp16(residual[d] + Σ_{slot=0..top_k-1} w[slot]·(down_e[d]·acts[slot])),
 * slots summed in fixed order. routing_weights fp16 [top_k]; residual may be
 * NULL (zeros). Replaces MoE.encodeRoutedPersistentPhase2Reduce
 * (MoE.swift:312-362). Contract: f % 64 == 0, f <= 1024, top_k == 8 or
 * top_k <= 8. */
int tfq_moe_phase2(tfq_ctx *ctx, void *stream, const tfq_expert_pool *pool,
                   const uint32_t *indices, const uint16_t *acts, const uint16_t *routing_weights,
                   const uint16_t *residual, uint16_t *y, uint32_t d, uint32_t f,
                   uint32_t top_k);

/* Phase 1 then phase 2 (acts_scratch: fp16 [top_k][f] device buffer). */
int tfq_moe_decode(tfq_ctx *ctx, void *stream, const tfq_expert_pool *pool,
                   const uint32_t *indices, const uint16_t *routing_weights, const uint16_t *x,
                   const uint16_t *residual, uint16_t *y, uint32_t d, uint32_t f,
                   uint32_t top_k, uint16_t *acts_scratch);

/* int8 router of one MoE layer (weights [num_experts][d], fp16 scale/bias per
 * 64). effective_scale [d] / per_expert_scale [num_experts] may be NULL. */
typedef struct {
    const uint8_t *weights;
    const uint16_t *scales;
    const uint16_t *biases;
    const uint16_t *effective_scale;
    const uint16_t *per_expert_scale;
    uint32_t num_experts;
} tfq_router;

/* The whole routed decode block of one token, all on the device, in three
 * launches: router GEMV (logits into the workspace), phase 1 with the top-k
 * selection folded in (every block selects from the logits; block 0
 * publishes out_indices / out_weights), phase 2. Replaces the decode
 * sequence encodeRouterGemma4 -> CPU readback of the indices -> expert fetch
 * -> Phase1U16Load -> Phase2Reduce (S/Runtime/Inference/
 * RealForwardRunner.swift:2390-2401, 2491-2521, 2822-2864); the indices never
 * leave HBM. out_indices [top_k] / out_weights fp16 [top_k] receive the
 * routing; acts_scratch is fp16 [top_k][f]; workspace is
 * TFQ_ROUTER_WORKSPACE_BYTES. Contracts as for the individual calls. */
int tfq_moe_decode_token(tfq_ctx *ctx, void *stream, const tfq_router *router,
                         const tfq_expert_pool *pool, const uint16_t *x,
                         const uint16_t *residual, uint16_t *y, uint32_t d, uint32_t f,
                         uint32_t top_k, uint32_t *out_indices, uint16_t *out_weights,
                         uint16_t *acts_scratch, void *workspace);

/* Bytes of the device scratch array of tfq_moe_decode_token_noalloc (one
 * per GPU, held until the process ends). */
#define TFQ_NOALLOC_SCRATCH_BYTES (16384u + TFQ_ROUTER_WORKSPACE_BYTES)

/* tfq_moe_decode_token with no scratch arguments and no allocation: the
 * routed activations and the router logits live in a fixed device array
 * inside libtfq (TFQ_NOALLOC_SCRATCH_BYTES, one copy per GPU, resolved once
 * per context at tfq_create). This entry point has no counterpart in the
 * reference; it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It calls no hipMalloc/hipFree. Limit: top_k * f * 2 <= 16384
 * bytes (every shape the decode phases accept: f <= 1024, top_k <= 8);
 * larger shapes return TFQ_E_INVAL. Every call on one GPU shares that GPU's
 * array, through every context: calls that overlap on one GPU (concurrent
 * streams or threads) race. Nothing in the array needs to start at zero
 * (each call writes what it reads), and the last call's contents remain.
 * Contracts otherwise as tfq_moe_decode_token. */
int tfq_moe_decode_token_noalloc(tfq_ctx *ctx, void *stream, const tfq_router *router,
                                 const tfq_expert_pool *pool, const uint16_t *x,
                                 const uint16_t *residual, uint16_t *y, uint32_t d, uint32_t f,
                                 uint32_t top_k, uint32_t *out_indices, uint16_t *out_weights);

/* Shared expert, int4 form: act[i] = fp16(gelu_tanh(gate[i]·x) * (up[i]·x))
 * with gate/up kept in fp32 (one fused launch), then y = fp16(down·act).
 * gate/up are [f][d], down is [d][f]; act_scratch: fp16 [f].
 * Replaces SharedExpertInt4.encode (S/Kernels/MoE/SharedExpertInt4.swift:30-94),
 * whose GPU sequence rounds gate and up to fp16 before the activation (its
 * CPU reference does not; the rounding moves the output ~8e-4 from it).
 * Contract: d, f multiples of 64 and <= 8192. A 16-byte aligned x (d <=
 * 4096) runs the gate/up form whose staging is fixed at compile time. */
int tfq_shared_expert_q4(tfq_ctx *ctx, void *stream, const tfq_q4_matrix *gate,
                         const tfq_q4_matrix *up, const tfq_q4_matrix *down, const uint16_t *x,
                         uint16_t *y, uint32_t d, uint32_t f, uint16_t *act_scratch);

/* One int8 g64 matrix: rows of n bytes (one code per byte), fp16 scale/bias
 * per 64 codes (the layout of tfq_q4_matrix with 8-bit codes). */
typedef tfq_q4_matrix tfq_q8_matrix;

/* Shared expert, int8 form (the reference's default width,
 * S/Runtime/Inference/Model.swift:59): act[i] = fp16(gelu_tanh(g)·u) with
 * g = gate[i]·x, u = up[i]·x in fp32 in one fused launch (the reference
 * kernel rounds g and u to fp16 first, dequant_int8.metal:150-152, which its
 * CPU reference does not; that rounding moves the output ~4e-4 from it),
 * then the int8 down GEMV y = fp16(down·act). gate/up [f][d], down [d][f]; act_scratch
 * fp16 [f]. Replaces SharedExpertInt8.encode
 * (S/Kernels/MoE/SharedExpertInt8.swift:90-130; kernel
 * shared_int8_gate_up_act_simd, S/Metal/Quant/dequant_int8.metal:99-154).
 * Contract: d, f multiples of 64 and <= 4096; gate/up weights 16-byte aligned.
 * A 16-byte aligned x runs the gate/up form whose staging is fixed at
 * compile time. */
int tfq_shared_expert_q8(tfq_ctx *ctx, void *stream, const tfq_q8_matrix *gate,
                         const tfq_q8_matrix *up, const tfq_q8_matrix *down, const uint16_t *x,
                         uint16_t *y, uint32_t d, uint32_t f, uint16_t *act_scratch);

/* -------------------------------------------------------- decode layer -- */

/* Workspace bytes of tfq_attention_decode for `seq_len` positions. */
size_t tfq_attention_workspace_bytes(uint32_t head_dim, uint32_t num_q_heads, uint32_t seq_len,
                                     uint32_t window);

/* Single-token GQA attention over an fp16 KV cache:
 * out[h] = Σ_j softmax_j(scale · q[h]·K[j][h/G]) V[j][h/G] over the visible
 * keys j in [max(0, seq_len - window), seq_len) (window 0: all), G =
 * num_q_heads / num_kv_heads. q, out fp16 [num_q_heads][head_dim]; caches
 * fp16 [capacity][num_kv_heads][head_dim]. fp32 scores and accumulation, one
 * fp16 rounding of the output. Replaces Attention.encodeFull /
 * Attention.encodeSWA (S/Kernels/Attention/Attention.swift:238-370).
 * Also replaces attention_decode_gqa_full_partial + attention_decode_combine
 * (S/Metal/Attention/attention.metal:454-615), the full-attention layers'
 * kernel (head_dim 512).
 * Contract: head_dim 128 or 256 with G in {1, 2, 4}, or head_dim 512 with G
 * in {1, 2, 4, 8}; seq_len in 1...65536; q, caches and workspace 16-byte
 * aligned. */
int tfq_attention_decode(tfq_ctx *ctx, void *stream, const uint16_t *q, const uint16_t *k_cache,
                         const uint16_t *v_cache, uint16_t *out, uint32_t head_dim,
                         uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t seq_len,
                         uint32_t window, float scale, void *workspace, size_t workspace_bytes);

/* Weights of one Gemma 4 decoder layer (all device pointers; norm weights
 * fp16, converted from the checkpoint's BF16 with tfq_convert_bf16_to_f16). */
typedef struct {
    const uint16_t *input_norm;          /* [d] input_layernorm */
    tfq_q4_matrix q_proj, k_proj, v_proj; /* [nq*hd][d], [nkv*hd][d], [nkv*hd][d];
                                            v_proj.weights NULL: no v projection, V is
                                            the k projection (the full-attention layers,
                                            RealForwardRunner.swift:2252-2255) */
    const uint16_t *q_norm, *k_norm;     /* [head_dim] per-head q/k RMSNorm */
    tfq_q4_matrix o_proj;                /* [d][nq*hd] */
    const uint16_t *post_attention_norm; /* [d] */
    const uint16_t *pre_ffn_norm;        /* [d] shared-expert input (pre_feedforward_layernorm) */
    const uint16_t *pre_ffn2_norm;       /* [d] routed-expert input (pre_feedforward_layernorm_2) */
    tfq_router router;                   /* input: no-scale RMSNorm of the residual stream */
    tfq_expert_pool experts;
    tfq_q4_matrix shared_gate, shared_up, shared_down; /* [fs][d], [fs][d], [d][fs] */
    const uint16_t *post_ffn1_norm;      /* [d] shared-expert output norm */
    const uint16_t *post_ffn2_norm;      /* [d] routed output norm */
    const uint16_t *post_ffn_norm;       /* [d] */
    float layer_scalar;
    uint32_t shared_bits;                /* shared expert rows: 4 (int4, also 0) or 8 (int8,
                                            shared_gate/up/down as tfq_q8_matrix) */
} tfq_decode_layer_weights;

typedef struct {
    uint32_t d, num_q_heads, num_kv_heads, head_dim;
    uint32_t rotated_pairs;              /* NeoX RoPE pairs (head_dim/2: full rotation) */
    uint32_t window;                     /* 0: full causal attention */
    uint32_t expert_f, shared_f, top_k;
    float eps, rope_theta, attn_scale;   /* Gemma 4: eps 1e-6, scale 1.0 */
} tfq_decode_layer_shape;

/* Workspace bytes of tfq_decode_layer for positions < max_seq_len. */
size_t tfq_decode_layer_workspace_bytes(const tfq_decode_layer_shape *shape, uint32_t max_seq_len);

/* One decoder layer for the token at `position` (keys 0..position visible):
 *   q,k,v = QKV(rmsnorm(hidden, input_norm)); k, v written to cache slot `position`
 *   q,k <- rope(rmsnorm_head(.., q_norm/k_norm)); v <- rmsnorm_head(v) (no scale)
 *   a = o_proj(attention(q, K, V));  h = hidden + rmsnorm(a, post_attention_norm)
 *   router on rmsnorm(h) (no scale) -> top_k experts and weights
 *   h1 = shared(rmsnorm(h, pre_ffn_norm));  h2 = Σ w·expert(rmsnorm(h, pre_ffn2_norm))
 *   out = (h + rmsnorm(rmsnorm(h1, post_ffn1) + rmsnorm(h2, post_ffn2), post_ffn)) * layer_scalar
 * with fp16 rounding wherever the reference stores a buffer. Every launch
 * runs on `stream`, in order (the call can be captured into a graph); with
 * 4-bit routed experts and shared_f <= 4096 the shared expert's (int4 or
 * int8) gate/up/act and down run inside the routed phase-1 and phase-2
 * launches, its input normed from the h and r(h) the router stores.
 * hidden_out may alias hidden_in. out_indices/out_weights (may be NULL)
 * receive the routing. Replaces the per-layer decode sequence of
 * RealForwardRunner (S/Runtime/Inference/RealForwardRunner.swift:2265-2862:
 * gInputNorm, gQKV, gQKVEpilogue, gAttention, gOProj, gPostAttnSetup,
 * gRouter, gSharedFFN + gSharedNorm, routed phases 1/2, gTail).
 * Full-attention layers (Gemma 4: every sixth layer, head_dim 512, 2 kv
 * heads, rope theta 1e6, rotated_pairs = head_dim * partial_rotary / 2 = 64)
 * pass their shape and a NULL v_proj: V = rmsnorm_head(k projection) (no
 * scale), K = rope(rmsnorm_head(k projection, k_norm)).
 * Contract: d multiple of 64, <= 4096; hidden vectors and norm weights
 * 16-byte aligned; attention as tfq_attention_decode; experts as
 * tfq_moe_decode; workspace 256-byte aligned. */
int tfq_decode_layer(tfq_ctx *ctx, void *stream, const tfq_decode_layer_weights *weights,
                     const tfq_decode_layer_shape *shape, const uint16_t *hidden_in,
                     uint16_t *hidden_out, uint16_t *k_cache, uint16_t *v_cache, uint32_t position,
                     uint32_t *out_indices, uint16_t *out_weights, void *workspace,
                     size_t workspace_bytes);

/* Workspace bytes of tfq_decode_layers for positions < max_seq_len. */
size_t tfq_decode_layers_workspace_bytes(const tfq_decode_layer_shape *shapes, uint32_t n_layers,
                                         uint32_t max_seq_len);

/* n_layers consecutive decoder layers for the token at `position` (the
 * reference's per-token loop over layers, RealForwardRunner.swift:2239-2862):
 * layer i's input is hidden_in for i = 0, else layer i-1's output, and
 * hiddens [n_layers][d] receives every layer's output (row n_layers-1 is the
 * token's final hidden state). Each layer computes exactly what
 * tfq_decode_layer computes, but the tail of layer i (its output) is formed
 * inside layer i+1's first launch, the QKV GEMV, while it stages its input,
 * so the chain takes n_layers - 1 launches fewer. weights / shapes [n_layers]
 * (sliding and full-attention layers may alternate; d and eps are shared);
 * k_caches / v_caches: host arrays of n_layers device pointers. One
 * workspace of tfq_decode_layers_workspace_bytes serves all layers (calls
 * that share it must not overlap). Contract as tfq_decode_layer, for every
 * layer. No reference counterpart as one call: the reference encodes the
 * same kernels layer by layer. */
int tfq_decode_layers(tfq_ctx *ctx, void *stream, uint32_t n_layers,
                      const tfq_decode_layer_weights *weights, const tfq_decode_layer_shape *shapes,
                      const uint16_t *hidden_in, uint16_t *hiddens, uint16_t *const *k_caches,
                      uint16_t *const *v_caches, uint32_t position, void *workspace,
                      size_t workspace_bytes);

/* ---------------------------------------------------------------- prefill -- */

#define TFQ_DTYPE_F16 0
#define TFQ_DTYPE_BF16 1

/* Y[t][n] = Σ_k X[t][k]·W[n][k] for t < m tokens, n < n outputs, k < k:
 * W int4 g64 [n][k] (fp16 scale/bias [n][k/64]), X [m][k] and Y [m][n] in
 * `dtype` (fp16 or bf16), fp32 accumulate on the matrix cores. Weights are
 * dequantised in registers to fp16 (q*s + b, one rounding) and multiplied
 * with fp16 activations; bf16 activations are converted to fp16 on the way
 * (round to nearest even: exact for |x| in [2^-14, 65504]; smaller values
 * keep fewer bits and larger ones become +-inf, as in the reference's fp16
 * activation path; callers that need to know can run
 * tfq_convert_bf16_to_f16 with its inexact counter on X). The kernel is
 * chosen by token count, as PrefillProjectionDispatchPolicy does
 * (S/Runtime/Inference/RealForwardRunner.swift:217-230, 1411-1492): the
 * decode GEMV for one token, a few-token weight stream below the measured
 * crossover of the shape, the 64-token MFMA tile above it. The GEMV forms
 * s·Σq·x + b·Σx in fp32 from the unrounded q·s, the two MFMA kernels
 * multiply fp16(q·s + b) weights: the paths differ by those roundings and
 * the summation order, each within the north-star bar of the CPU reference.
 * Replaces PrefillInt4QMM.encode
 * (S/Kernels/Prefill/Primitives/PrefillPrimitives.swift:82-122) and
 * MPPPrefillInt4QMM.encode (S/Kernels/TensorCore/MPPPrefillInt4QMM.swift:34-78).
 * Contract: k % 64 == 0, k <= 8192, n >= 1, m >= 1; W and X 16-byte aligned. */
int tfq_gemm_q4g64(tfq_ctx *ctx, void *stream, const void *weights, const uint16_t *scales,
                   const uint16_t *biases, const uint16_t *x, uint16_t *y, uint32_t m, uint32_t n,
                   uint32_t k, int dtype);

/* Kernel choices of the prefill GEMM (tfq_gemm_qg64_path). */
#define TFQ_GEMM_PATH_AUTO 0      /* by token count and shape, as tfq_gemm_q4g64 / tfq_gemm_qg64 do */
#define TFQ_GEMM_PATH_TILE 1      /* the 64-token x 256-output MFMA projection tile */
#define TFQ_GEMM_PATH_SKINNY 2    /* few-token weight stream: 16 rows x 16 tokens per wave, K split in 8 */
#define TFQ_GEMM_PATH_SKINNY32 3  /* the same with 32 rows per wave */
#define TFQ_GEMM_PATH_GEMV 4      /* the decode GEMV once per token (the reference's repeated
                                     GEMV below 32 tokens, RealForwardRunner.swift:1460-1491) */

/* tfq_gemm_q4g64 at `bits` = 3 or 4 bits per code (rows of k*bits/8 bytes,
 * codes packed from the least significant bit). Replaces
 * PrefillInt4QMM.encode(..., bits: 3) (PrefillPrimitives.swift:82-122 with
 * prefill_dequant_int4_qmm_f16_block_b3, prefill.metal:711-757); other
 * widths: TFQ_E_INVAL (the reference's precondition, :94-95). */
int tfq_gemm_qg64(tfq_ctx *ctx, void *stream, const void *weights, const uint16_t *scales,
                  const uint16_t *biases, const uint16_t *x, uint16_t *y, uint32_t m, uint32_t n,
                  uint32_t k, int dtype, uint32_t bits);

/* tfq_gemm_qg64 with the kernel named by `path` (TFQ_GEMM_PATH_*) instead of
 * the built-in choice: for measuring the crossover and for tests that hold
 * both kernels to the same reference. Same contract; results of the two
 * kernels differ only by fp32 summation order. */
int tfq_gemm_qg64_path(tfq_ctx *ctx, void *stream, const void *weights, const uint16_t *scales,
                       const uint16_t *biases, const uint16_t *x, uint16_t *y, uint32_t m, uint32_t n,
                       uint32_t k, int dtype, uint32_t bits, int path);

/* Workspace bytes of tfq_prefill_shared_expert. */
size_t tfq_prefill_shared_expert_workspace_bytes(uint32_t weight_bits, uint32_t tokens, uint32_t f);

/* The shared expert over a block of `tokens` rows: y + t*y_stride =
 * shared(x + t*x_stride) for t < tokens (strides in halves). int8 weights
 * run the decode kernels over all rows in one launch each, so each row is
 * bit-identical to tfq_shared_expert_q8. int4 weights run the prefill GEMM:
 * gate and up are stored to the workspace in fp16 before gelu_mul (the
 * rounding of the reference's GPU sequence, SharedExpertInt4.swift:30-94),
 * then down; tfq_shared_expert_q4 keeps gate/up in fp32 instead, so the two
 * int4 forms differ by those roundings (~8e-4 of max|y| at the config-4
 * shapes). The GEMM kernel follows the token count. Replaces
 * PrefillSharedExpert.encodeBlock
 * (S/Kernels/Prefill/MoE/PrefillSharedExpert.swift:11-60), which encodes the
 * decode form once per row. Contract: as the decode forms; x_stride >= d and
 * y_stride >= d (a multiple of 8 for int4, with x 16-byte aligned);
 * workspace 256-byte aligned, tfq_prefill_shared_expert_workspace_bytes
 * long; tokens == 0 does nothing. */
int tfq_prefill_shared_expert(tfq_ctx *ctx, void *stream, uint32_t weight_bits,
                              const tfq_q4_matrix *gate, const tfq_q4_matrix *up,
                              const tfq_q4_matrix *down, const uint16_t *x, uint32_t x_stride,
                              uint16_t *y, uint32_t y_stride, uint32_t tokens, uint32_t d, uint32_t f,
                              void *workspace, size_t workspace_bytes);

/* (token, expert, rank, fp16 routing weight bits in the low half) — the
 * 16-byte PrefillTokenExpertPair (S/Kernels/Prefill/MoE/PrefillRouter.swift:5-28). */
typedef struct {
    uint32_t token;
    uint32_t expert;
    uint32_t rank;
    uint32_t weight_bits;
} tfq_pair;

/* One 128-row MFMA tile of one expert: sorted pairs [start, start+count). */
typedef struct {
    uint32_t expert;
    uint32_t start;
    uint32_t count;
    uint32_t reserved;
} tfq_tile;

/* Upper bound of the tile count for T*top_k pairs over num_experts experts. */
#define TFQ_MOE_MAX_TILES(T, top_k, num_experts)                                   \
    (((T) * (top_k) + 127u) / 128u +                                               \
     ((num_experts) < (T) * (top_k) ? (num_experts) : (T) * (top_k)))

/* Router for a chunk of T tokens: hidden [T] rows of hidden_stride fp16
 * elements -> indices [T][top_k] and fp16 weights [T][top_k] (fp32 copy to
 * out_weights_f32 if non-NULL). logits_scratch: fp32 [T][num_experts].
 * Same arithmetic per token as tfq_router_topk. Replaces
 * PrefillRouter.encodeGemma4Block (S/Kernels/Prefill/MoE/PrefillRouter.swift:37-89).
 * Contract: T >= 1, hidden_stride >= d, d % 64 == 0, d <= 4096,
 * 1 <= num_experts <= 256, 1 <= top_k <= min(64, num_experts). */
int tfq_prefill_router(tfq_ctx *ctx, void *stream, const tfq_router *router,
                       const uint16_t *hidden, uint32_t hidden_stride, uint32_t T, uint32_t d,
                       uint32_t top_k, uint32_t *out_indices, uint16_t *out_weights,
                       float *out_weights_f32, float *logits_scratch);

/* Status written by tfq_moe_group (values of PrefillMoEGroupingError the
 * device can detect; same numbering as tfq_group_pairs_host). */
#define TFQ_GROUP_OK 0
#define TFQ_GROUP_INVALID_QUERY_COUNT 1
#define TFQ_GROUP_INVALID_TOPK 2
#define TFQ_GROUP_INVALID_NUM_EXPERTS 3
#define TFQ_GROUP_INVALID_TILE_EXPERT_COUNT 4
#define TFQ_GROUP_PAIR_COUNT_MISMATCH 5
#define TFQ_GROUP_TOKEN_OUT_OF_RANGE 6
#define TFQ_GROUP_RANK_OUT_OF_RANGE 7
#define TFQ_GROUP_EXPERT_OUT_OF_RANGE 8
#define TFQ_GROUP_DUPLICATE_TOKEN_RANK 9
#define TFQ_GROUP_SORT_KEY_COUNT_MISMATCH 10

/* Words of the device grouping state (the n_tiles argument of tfq_moe_group
 * and tfq_moe_grouped): [0] the tile count, [1..2] the work counters of the
 * grouped launches, [3] reserved. */
#define TFQ_MOE_GROUP_STATE_WORDS 4

/* Device grouping of the token-major pairs (token t, rank r) -> expert
 * indices[t*top_k + r] with weight weights[t*top_k + r]: a stable counting
 * sort giving the order (expert, token, rank) of PrefillMoEGrouping
 * .groupTokenExpertPairs (S/Kernels/Prefill/MoE/PrefillMoEGrouping.swift:91-192,
 * no sort keys). offsets/counts [num_experts] (offset 0xFFFFFFFF for an empty
 * expert), tiles [TFQ_MOE_MAX_TILES], n_tiles [TFQ_MOE_GROUP_STATE_WORDS]
 * (the tile count, then counters zeroed here) and *status on the device. An
 * out-of-range expert index groups nothing and sets *status =
 * TFQ_GROUP_EXPERT_OUT_OF_RANGE. Contract: 1 <= T*top_k <= 8192,
 * 1 <= num_experts <= 256. */
int tfq_moe_group(tfq_ctx *ctx, void *stream, const uint32_t *indices, const uint16_t *weights,
                  uint32_t T, uint32_t top_k, uint32_t num_experts, tfq_pair *sorted,
                  uint32_t *offsets, uint32_t *counts, tfq_tile *tiles, uint32_t *n_tiles,
                  uint32_t *status);

/* A group of equal-expert pairs and a tile of <= tile_expert_count groups, as
 * returned by the host grouping (PrefillMoEGroup / PrefillMoETile,
 * PrefillMoEGrouping.swift:3-29). */
typedef struct { uint32_t expert, pair_start, pair_count; } tfq_group;
typedef struct { uint32_t group_start, group_count, pair_start, pair_count; } tfq_group_tile;

/* Host-side grouping with the reference's exact contract, validation order
 * and error cases (PrefillMoEGrouping.groupTokenExpertPairs,
 * PrefillMoEGrouping.swift:91-192): returns TFQ_GROUP_*; err[0..1] carry the
 * values of the Swift error case. sort_keys may be NULL. Output arrays:
 * sorted [n_pairs], offsets/counts/groups/tiles [num_experts]. */
int tfq_group_pairs_host(const tfq_pair *pairs, int64_t n_pairs, int64_t query_count,
                         int64_t top_k, int64_t num_experts, int64_t tile_expert_count,
                         const uint64_t *sort_keys, int64_t n_sort_keys, tfq_pair *sorted,
                         uint32_t *offsets, uint32_t *counts, tfq_group *groups,
                         int64_t *n_groups, tfq_group_tile *tiles, int64_t *n_tiles,
                         int64_t err[2]);

/* Grouped routed experts over the sorted pairs: for every tile, gate/up on
 * the MFMA cores with act = fp16(gelu(gate)·up) into act_scratch
 * [T*top_k][f] (row = sorted position), then down with each row written to
 * route_partials[(token*top_k + rank)*d ...] (fp16 [T*top_k][d]); rows of
 * (token, rank) slots without a pair are left untouched. max_tiles is the
 * launch bound (TFQ_MOE_MAX_TILES, at most 320 = 8192/128 + 256,
 * TFQ_E_UNSUPPORTED beyond); the device tile count n_tiles[0] decides. The
 * launches take their work units from the counters n_tiles[1..2], which must
 * be zero on entry (tfq_moe_group zeroes them; a state built by other means
 * must too, or blocks skip work units and rows stay unwritten), and leave
 * them zero, so calls on one grouping state must not overlap. Replaces
 * PrefillGroupedRoutedMoE.encodeStreamedBatched
 * (S/Kernels/Prefill/MoE/PrefillGroupedRoutedMoE.swift:446-527), and its
 * 2/3-bit forms (prefill.metal:1304-1450) when pool->weight_bits is 2 or 3.
 * Contract: d, f multiples of 64 and at most 8192 (TFQ_E_UNSUPPORTED
 * beyond); hidden rows, act_scratch and route_partials 16-byte aligned.
 * Pools whose scale/bias offsets are 16-byte aligned (d <= 3072 for gate/up,
 * f <= 1024 for down) run launches that stage each unit's scale/bias table
 * through registers (faster; the same bits). */
int tfq_moe_grouped(tfq_ctx *ctx, void *stream, const tfq_expert_pool *pool,
                    const tfq_pair *sorted, const tfq_tile *tiles, uint32_t *n_tiles,
                    uint32_t max_tiles, const uint16_t *hidden, uint32_t hidden_stride,
                    uint32_t d, uint32_t f, uint32_t top_k, uint16_t *act_scratch,
                    uint16_t *route_partials);

/* h2[t][d] = fp16(Σ_r fma(w[t][r], partials[(t*top_k + r)*d + ...])) in rank
 * order. Replaces PrefillMoE.encodeReduceTokenMajor
 * (S/Kernels/Prefill/MoE/PrefillMoE.swift:11-38). */
int tfq_moe_combine(tfq_ctx *ctx, void *stream, const uint16_t *route_partials,
                    const uint16_t *route_weights, uint16_t *h2, uint32_t T, uint32_t top_k,
                    uint32_t d);

/* Workspace bytes of tfq_moe_prefill. */
size_t tfq_moe_prefill_workspace_bytes(uint32_t T, uint32_t top_k, uint32_t num_experts,
                                       uint32_t d, uint32_t f);

/* Routed MoE of a prefill chunk, all on the device: tfq_prefill_router ->
 * tfq_moe_group -> tfq_moe_grouped -> tfq_moe_combine. out_indices /
 * out_weights [T][top_k] receive the routing; h2 [T][d] fp16. */
int tfq_moe_prefill(tfq_ctx *ctx, void *stream, const tfq_router *router,
                    const tfq_expert_pool *pool, const uint16_t *hidden,
                    uint32_t hidden_stride, uint32_t T, uint32_t d, uint32_t f, uint32_t top_k,
                    uint16_t *h2, uint32_t *out_indices, uint16_t *out_weights, void *workspace,
                    size_t workspace_bytes);

/* ----------------------------------------------------------------- loader -- */

/* fp16 <- BF16, elementwise on the device. Values outside the exactly
 * representable fp16 range are still converted (round to nearest even /
 * saturate to inf) and counted: *inexact_count_dev (device uint32, may be
 * NULL) is incremented once per inexact element. src and dst may be the
 * same buffer. Converts the reference's BF16 scales/biases
 * (S/Infrastructure/ModelIO/Quantization.swift:32-45). */
int tfq_convert_bf16_to_f16(tfq_ctx *ctx, void *stream, const uint16_t *src, uint16_t *dst,
                            uint64_t count, uint32_t *inexact_count_dev);

/* ------------------------------------------------------------ measurement -- */

/* Pure read of `bytes` (16-byte aligned) with 128-bit coalesced loads, one
 * pass, xor-reduced into sink[0..blocks) (device uint32, sink_blocks
 * entries; the launch uses at most that many blocks). The HBM read ceiling
 * the GEMVs are compared with; replaces bw_ceiling_read
 * (S/Metal/Quant/dequant_int4.metal:487-502). */
int tfq_read_ceiling(tfq_ctx *ctx, void *stream, const void *src, uint64_t bytes, uint32_t *sink,
                     uint32_t sink_blocks);

#ifdef __cplusplus
}
#endif
#endif /* TFQ_H */
