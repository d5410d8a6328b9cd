// abi_types.h — kernel-argument structs shared by the device code and the
// host launcher (plain C layout; passed by value through hipModuleLaunchKernel).
#pragma once
#include <stdint.h>

namespace tfq {

// One int4 matrix and its fp16 output, as seen by a multi-matrix launch;
// r (may be null) is an fp16 residual added to the fp32 result before the
// output is rounded: y = fp16(r + W·x).
struct Q4Mat {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint16_t* y;
    const uint16_t* r;
    uint32_t rows;
    uint32_t pad_;
};

// One int8 g64 matrix (rows of n bytes, fp16 scale/bias per 64 codes).
struct Q8Mat {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
};

// How a kernel forms its fp16 activation vector a from x while staging it
// to LDS (r(v) = 1/sqrt(mean(v^2) + eps), every intermediate rounded to fp16
// where a separate kernel would have stored it):
//   kStageCopy      a = x
//   kStageNorm      a = fp16(x * w * r(x))                (w == null: no scale)
//   kStagePostAttn  h = fp16(x + fp16(attn * attn_w * r(attn)));
//                   a = fp16(h * w * r(h))                (w == null: no scale)
// kStagePostAttn is the decode layer's post-attention residual + pre-FFN (or
// router) norm, recomputed by every block that consumes it. With export_h
// set, block 0 of the launch also stores h (fp16) to export_h and r(h)
// (fp32) to *export_inv, so a later kernel can form a = fp16(h * w * r(h))
// for another w without the reductions:
//   kStageResidual  a = h (the post-attention residual stream, no norm)
//   kStageScaled    a = fp16(x * w * inv[0])              (w == null: no scale;
//                   x = an exported h, inv its exported r(h))
//   kStageBf16      a = fp16(x) for a bf16 x (round to nearest even, as the
//                   prefill GEMM converts its activations); the GEMV then
//                   stores its rows as bf16 too (the prefill GEMM's one-token path)
//   kStageTail      out = the previous decoder layer's tail (layer_tail in
//                   attention.hpp) from x = that layer's input hidden, attn =
//                   its o projection (attn_w its post_attention_norm), h1 /
//                   h2 with their output norms h1_w / h2_w, ffn_w and scalar;
//                   block 0 stores out (the layer's output) to export_h; then
//                   a = fp16(out * w * r(out)) (the next layer's input norm)
enum StageMode : uint32_t { kStageCopy = 0, kStageNorm = 1, kStagePostAttn = 2, kStageResidual = 3,
                            kStageScaled = 4, kStageBf16 = 5, kStageTail = 6 };

struct NormArg {
    const uint16_t* w;
    const uint16_t* attn;
    const uint16_t* attn_w;
    float eps;
    uint32_t mode;
    const float* inv;          // kStageScaled: r(h)
    uint16_t* export_h;        // kStagePostAttn: h and r(h) from block 0 (nullable); kStageTail: out
    float* export_inv;
    const uint16_t* h1;        // kStageTail: shared-expert output and post_feedforward_layernorm_1
    const uint16_t* h1_w;
    const uint16_t* h2;        // kStageTail: routed output and post_feedforward_layernorm_2
    const uint16_t* h2_w;
    const uint16_t* ffn_w;     // kStageTail: post_feedforward_layernorm
    float scalar;              // kStageTail: layer scalar
};

// Dynamic LDS of the int4 GEMV-family kernels for an activation vector of n
// halves (n a multiple of 32): the staged fp16 vector (2n bytes), its paired
// copy in the order the int4 dot consumes it (2n bytes) and four fp32 words
// of sums per 32-element chunk (16 bytes each).
constexpr uint32_t xpairs_lds_bytes(uint32_t n) { return 4u * n + 16u * (n >> 5); }

// Keys per split-K attention block (attention.hpp) and the most chunks the
// combine merges (its weight table in LDS): 65536 visible keys.
constexpr uint32_t kAttnChunk = 64;
constexpr uint32_t kAttnMaxChunks = 65536 / kAttnChunk;
// The combine's block: 256 threads over 64 head dims (grid: query heads x
// head_dim / 64).
constexpr uint32_t kAttnCombineDims = 64;
constexpr uint32_t kAttnCombineThreads = 256;

// Gemma 4 q/k/v epilogue applied inside the decode attention kernel
// (fused_qkv_epilogue, S/Metal/Fusions/fused.metal:86-180): per-head RMSNorm
// of q and k with the shared head-dim weights, NeoX RoPE of the first
// rotated_pairs pairs at the new token's position, no-scale RMSNorm of v.
// q_norm == null disables it (plain attention). k_raw / v_raw: the new
// token's raw k and v rows [num_kv_heads][head_dim] when they are staged
// outside the caches (required when a kv head's query heads are split over
// blocks, which then all read them; v_raw == k_raw for the full-attention
// layers that take V from the k projection); null: read from the cache slot.
struct AttnEpilogue {
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    float eps;
    float theta;
    uint32_t rotated_pairs;
    uint32_t pad_;
    double log2_theta;      // log2(theta), set by the launcher
    const uint16_t* k_raw;
    const uint16_t* v_raw;
};

// Up to three matrices sharing x and n (plain GEMV: 1; fused QKV: 3).
struct Q4Multi {
    Q4Mat m[3];
    uint32_t nmat;
    uint32_t total_rows;
    NormArg norm;
};

// Sub-tensor byte offsets inside one routed-expert blob (MoEExpertOffsets).
struct ExpertOffsets {
    uint32_t gate_w, gate_s, gate_b;
    uint32_t up_w, up_s, up_b;
    uint32_t down_w, down_s, down_b;
};

// A layer's routed experts resident in HBM: blob(e) = base + e*stride.
struct ExpertPool {
    const uint8_t* base;
    uint64_t stride;
    uint32_t num_experts;
    uint32_t pad_;
    ExpertOffsets off;
};

// PrefillTokenExpertPair (S/Kernels/Prefill/MoE/PrefillRouter.swift:5-28).
struct Pair {
    uint32_t token;
    uint32_t expert;
    uint32_t rank;
    uint32_t weight_bits;
};

// One 128-row MFMA tile of one expert's run in the sorted pair list.
struct Tile {
    uint32_t expert;
    uint32_t start;
    uint32_t count;
    uint32_t pad_;
};

// Shape of one grouped launch (moe_prefill.hpp): the tile list's bound and
// the row blocks per entry of the two roles; the grid is the resident
// blocks, which walk the work list.
struct GroupedLaunch {
    uint32_t max_tiles;
    uint32_t wx;      // row blocks of the wide role
    uint32_t sx;      // row blocks of the stream
};

}  // namespace tfq
