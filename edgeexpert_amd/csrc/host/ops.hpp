// ops.hpp — C++ operator classes mirroring the reference's Swift kernel
// wrappers (S/Kernels/**): same class names, same argument meaning, one
// `encode` per reference `encode`. Where the Swift wrapper traps on a
// precondition these return TFQ_E_INVAL; where it would silently skip they
// return an error too. A stream replaces the command buffer; device
// pointers replace (MTLBuffer, offset) pairs.
#pragma once

#include <algorithm>
#include <cmath>

#include "../kernels/abi_types.h"
#include "module.hpp"

namespace tfq {

constexpr uint32_t kBlock = 256;          // 4 wavefronts per block for every GEMV-family kernel
constexpr uint32_t kMaxN = 8192;          // longest reduction with x resident in LDS
constexpr uint32_t kFixedStageMaxN = 4096; // longest x of the fixed-mode GEMV staging: 8 halves x 2 chunks x 256 threads
constexpr uint32_t kRowsInFlight = 1;     // rows per segment in flight (entry_points.hpp kRowsInFlight)
constexpr uint32_t kProjBM = 64;           // projection GEMM tile: tokens (gemm.hpp kProjBM)
constexpr uint32_t kProjBN = 256;          // outputs (gemm.hpp kProjBN)
constexpr uint32_t kProjThreads = 256;     // threads (gemm.hpp kProjThreads)
constexpr uint32_t kProjGemmThreads = 512; // threads of the prefill GEMM's tile (gemm.hpp kProjGemmThreads)
constexpr uint32_t kProjMaxK = 8192;       // longest reduction (gemm.hpp kProjMaxK)
constexpr uint32_t kUnitThreads = 256;          // grouped MoE units (moe_prefill.hpp)
constexpr uint32_t kUnitStride = 128 + 8;       // halves per LDS activation row of a unit
constexpr uint32_t kGroupMaxTiles = 8192 / 128 + 256;  // tiles the device planner takes (moe_prefill.hpp)
// the pipelined tile of the prefill GEMM (gemm.hpp proj_pl_lds_bytes)
constexpr uint32_t proj_pl_lds_bytes(uint32_t k) { return 3u * kProjBM * 72u * 2u + 4u * kProjBN * (k / 64u); }
static_assert(proj_pl_lds_bytes(kProjMaxK) <= 160u * 1024u, "pipelined tile exceeds the LDS of a CU");

// Grid of a row-loop kernel (blocks of kBlock threads, `lds` dynamic LDS
// bytes): one block per rows_per_block rows, but no more blocks than the GPU
// holds resident at once; the blocks then loop over the rows. A grid beyond
// that adds a partial second round of blocks, each re-staging x, and leaves
// most CUs idle while it drains.
inline uint32_t grid_for_rows(const Module& m, hipFunction_t f, uint32_t lds, uint64_t rows,
                              uint32_t rows_per_block, uint32_t block = kBlock) {
    uint64_t g = (rows + rows_per_block - 1) / rows_per_block;
    if (g < 1) g = 1;
    if (!f) return (uint32_t)(g < 1024 ? g : 1024);     // launch() reports the missing kernel
    const uint32_t cap = m.resident_blocks(f, block, lds);
    return (uint32_t)(g > cap ? cap : g);
}

// Validates how a kernel stages its activation vector (NormArg, abi_types.h).
inline int check_stage(const NormArg& na) {
    switch (na.mode) {
    case kStageCopy:
        return TFQ_OK;
    case kStageNorm:
        break;
    case kStageScaled:
        if (!na.inv) return fail(TFQ_E_INVAL, "scaled staging needs the exported r(h)");
        return TFQ_OK;
    case kStageBf16:
        return TFQ_OK;
    case kStageTail:
        if (!na.attn || !na.attn_w || !na.h1 || !na.h1_w || !na.h2 || !na.h2_w || !na.ffn_w)
            return fail(TFQ_E_INVAL, "tail staging needs o, h1, h2 and their norm weights");
        break;
    case kStagePostAttn:
    case kStageResidual:
        if (!na.attn || !na.attn_w)
            return fail(TFQ_E_INVAL, "post-attention staging needs the attention output and its norm weight");
        if (na.export_h && (na.mode != kStagePostAttn || !na.export_inv))
            return fail(TFQ_E_INVAL, "exporting h needs post-attention staging and a place for r(h)");
        break;
    default:
        return fail(TFQ_E_INVAL, "unknown staging mode %u", na.mode);
    }
    if (!(na.eps > 0.0f)) return fail(TFQ_E_INVAL, "RMSNorm eps must be positive");
    return TFQ_OK;
}

inline NormArg stage_copy() { return NormArg{nullptr, nullptr, nullptr, 0.0f, kStageCopy, nullptr, nullptr, nullptr}; }

// Kernel-name infix of the GEMV-family form that stages x as `na` says:
// "" for a plain copy, "norm_" for the forms that normalise while staging,
// "tail_" for the int4 GEMV that forms the previous layer's tail.
inline const char* form_prefix(const NormArg& na) {
    return na.mode == kStageCopy ? "" : na.mode == kStageTail ? "tail_" : "norm_";
}

// S/Kernels/Quant/DequantInt4GEMV.swift:5-181 (encode and encodeTgx share one kernel here:
// x always lives in LDS) and S/Kernels/Fusions/FusedQKVGEMV.swift:4-157.
class DequantInt4GEMV {
public:
    explicit DequantInt4GEMV(const Module& m) : m_(m) {}

    // DequantInt4GEMV.encode (DequantInt4GEMV.swift:84-127, bits: 3 or 4 as
    // at :145-157). residual (may be null): y = fp16(residual + W·x); stage:
    // how x is staged.
    int encode(void* stream, const void* weights, const uint16_t* scales, const uint16_t* biases,
               const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n,
               const uint16_t* residual = nullptr, const NormArg& stage = stage_copy(),
               uint32_t bits = 4) const {
        Q4Multi mats{};
        mats.m[0] = {static_cast<const uint8_t*>(weights), scales, biases, y, residual, m, 0};
        mats.nmat = 1;
        mats.total_rows = m;
        mats.norm = stage;
        return launch_multi(stream, mats, x, n, bits);
    }

    // FusedQKVGEMV.encode (FusedQKVGEMV.swift:92-156): rows mq + 2*mkv in one launch.
    int encode_qkv(void* stream, const tfq_q4_matrix& q, const tfq_q4_matrix& k,
                   const tfq_q4_matrix& v, const uint16_t* x, uint16_t* yq, uint16_t* yk,
                   uint16_t* yv, uint32_t mq, uint32_t mkv, uint32_t n,
                   const NormArg& stage = stage_copy(), uint32_t bits = 4) const {
        Q4Multi mats{};
        mats.m[0] = {static_cast<const uint8_t*>(q.weights), q.scales, q.biases, yq, nullptr, mq, 0};
        mats.m[1] = {static_cast<const uint8_t*>(k.weights), k.scales, k.biases, yk, nullptr, mkv, 0};
        mats.m[2] = {static_cast<const uint8_t*>(v.weights), v.scales, v.biases, yv, nullptr, mkv, 0};
        mats.nmat = 3;
        mats.total_rows = mq + 2 * mkv;
        mats.norm = stage;
        return launch_multi(stream, mats, x, n, bits);
    }

    // q and k only (the full-attention layers, whose V is formed from k).
    int encode_qk(void* stream, const tfq_q4_matrix& q, const tfq_q4_matrix& k, const uint16_t* x,
                  uint16_t* yq, uint16_t* yk, uint32_t mq, uint32_t mkv, uint32_t n,
                  const NormArg& stage = stage_copy(), uint32_t bits = 4) const {
        Q4Multi mats{};
        mats.m[0] = {static_cast<const uint8_t*>(q.weights), q.scales, q.biases, yq, nullptr, mq, 0};
        mats.m[1] = {static_cast<const uint8_t*>(k.weights), k.scales, k.biases, yk, nullptr, mkv, 0};
        mats.nmat = 2;
        mats.total_rows = mq + mkv;
        mats.norm = stage;
        return launch_multi(stream, mats, x, n, bits);
    }

private:
    int launch_multi(void* stream, Q4Multi& mats, const uint16_t* x, uint32_t n, uint32_t bits) const {
        // the reference's attention kernels exist at 3 and 4 bits (DequantInt4GEMV.swift:149-150)
        if (bits != 3 && bits != 4) return fail(TFQ_E_INVAL, "unsupported attention weight bits %u", bits);
        if (n == 0 || n % TFQ_GROUP_SIZE != 0)
            return fail(TFQ_E_INVAL, "n=%u must be a positive multiple of 64", n);
        if (n > kMaxN) return fail(TFQ_E_UNSUPPORTED, "n=%u exceeds %u", n, kMaxN);
        if (!x || !aligned(x, 2)) return fail(TFQ_E_INVAL, "x must be non-null and 2-byte aligned");
        if (int rc = check_stage(mats.norm)) return rc;
        for (uint32_t i = 0; i < mats.nmat; ++i) {
            const Q4Mat& q = mats.m[i];
            if (q.rows == 0) return fail(TFQ_E_INVAL, "matrix %u has zero rows", i);
            if (!q.w || !q.s || !q.b || !q.y)
                return fail(TFQ_E_INVAL, "matrix %u has a null pointer", i);
            // 128-bit weight loads (the reference needs only 2-byte alignment, DequantInt4GEMV.swift:97-102).
            if (!aligned(q.w, 16)) return fail(TFQ_E_INVAL, "weights of matrix %u are not 16-byte aligned", i);
            if (!aligned(q.s, 2) || !aligned(q.b, 2) || !aligned(q.y, 2) || !aligned(q.r, 2))
                return fail(TFQ_E_INVAL, "scales/biases/y of matrix %u are not 2-byte aligned", i);
        }
        const SegShape sh = seg_shape_fit(n / 32, 2);
        // The plain and _rms forms fix the staging mode at compile time and
        // take only 16-byte aligned inputs of n <= kFixedStageMaxN; other
        // calls go to the _norm form, which reads the mode. The tail form is
        // always fixed: its inputs must qualify.
        const NormArg& na = mats.norm;
        const bool vec = aligned(x, 16) && n <= kFixedStageMaxN;
        const char* form = "norm_";
        if (na.mode == kStageTail) {
            for (const void* p : {(const void*)x, (const void*)na.w, (const void*)na.attn, (const void*)na.attn_w,
                                  (const void*)na.h1, (const void*)na.h1_w, (const void*)na.h2, (const void*)na.h2_w,
                                  (const void*)na.ffn_w, (const void*)na.export_h})
                if (!p || !aligned(p, 16)) return fail(TFQ_E_INVAL, "tail staging needs 16-byte aligned vectors");
            form = "tail_";
        } else if (na.mode == kStageCopy && vec) {
            form = "";
        } else if (na.mode == kStageCopy && bits == 4 && aligned(x, 16) && n <= 2 * kFixedStageMaxN) {
            form = "wide_";
        } else if (na.mode == kStageNorm && vec && aligned(na.w, 16)) {
            form = "rms_";
        }
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_q%u_gemv_%ss%u_p%u", bits, form, sh.seg, sh.p);
        // the tail form runs 1024-thread blocks (entry_points.hpp kTailGemvThreads)
        const uint32_t block = na.mode == kStageTail ? 1024u : kBlock;
        const uint32_t rows_per_block = (block / 64) * (64 / sh.seg) * kRowsInFlight;
        uint32_t nn = n;
        void* args[] = {&mats, &x, &nn};
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = xpairs_lds_bytes(n);
        return launch(fn, grid_for_rows(m_, fn, lds, mats.total_rows, rows_per_block, block), block, lds, stream,
                      args, name);
    }

    const Module& m_;
};

// S/Kernels/Quant/DequantInt8GEMV.swift:16-82.
class DequantInt8GEMV {
public:
    explicit DequantInt8GEMV(const Module& m) : m_(m) {}

    // tokens > 1: the same GEMV for `tokens` inputs x + t·x_stride into
    // y + t·y_stride (one launch; blockIdx.y is the token).
    int encode(void* stream, const uint8_t* weights, const uint16_t* scales, const uint16_t* biases,
               const uint16_t* x, uint16_t* y, uint32_t m, uint32_t n, uint32_t tokens = 1,
               uint32_t x_stride = 0, uint32_t y_stride = 0) const {
        if (n == 0 || n % TFQ_GROUP_SIZE != 0)
            return fail(TFQ_E_INVAL, "n=%u must be a positive multiple of 64", n);
        if (n > 4096) return fail(TFQ_E_UNSUPPORTED, "int8 GEMV n=%u exceeds 4096", n);
        if (m == 0) return fail(TFQ_E_INVAL, "m must be positive");
        if (tokens == 0 || tokens > 65535) return fail(TFQ_E_INVAL, "token count %u must be in 1...65535", tokens);
        if (!weights || !scales || !biases || !x || !y)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(weights, 16)) return fail(TFQ_E_INVAL, "weights are not 16-byte aligned");
        if (!aligned(scales, 2) || !aligned(biases, 2) || !aligned(x, 2) || !aligned(y, 2))
            return fail(TFQ_E_INVAL, "fp16 operands must be 2-byte aligned");
        const SegShape sh = seg_shape(n / 16, 4);
        // 16-byte aligned rows of x: the form with the copy staging fixed at
        // compile time (n <= 4096 is checked above)
        const bool fixed = aligned(x, 16) && (tokens == 1 || x_stride % 8 == 0);
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_q8_gemv_%ss%u_p%u", fixed ? "c_" : "", sh.seg, sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg) * kRowsInFlight;
        void* args[] = {&weights, &scales, &biases, &x, &x_stride, &y, &y_stride, &m, &n};
        hipFunction_t fn = m_.get(name);
        if (!fn) return fail(TFQ_E_NOT_LOADED, "kernel %s is not in the code object", name);
        return hip_check(hipModuleLaunchKernel(fn, grid_for_rows(m_, fn, n * 6, m, rows_per_block), tokens, 1,
                                               kBlock, 1, 1, n * 6, (hipStream_t)stream, args, nullptr),
                         name);
    }

private:
    const Module& m_;
};

// S/Kernels/Fusions/LMHeadChainInt4.swift:62-135 (encodeGreedyDecode): the
// reference's RMSNorm launch is folded into the rows' activation staging;
// then the int4 rows with a per-block argmax (logit.metal:688-737) and a
// one-block reduce to the token (logit.metal:740-787).
class LMHeadGreedyInt4 {
public:
    explicit LMHeadGreedyInt4(const Module& m) : m_(m) {}

    int encode(void* stream, const uint16_t* hidden, const uint16_t* norm_weight, const void* weights,
               const uint16_t* scales, const uint16_t* biases, uint32_t* out_token, uint32_t d, uint32_t vocab,
               float eps, void* workspace, size_t workspace_bytes) const {
        if (d == 0 || d % TFQ_GROUP_SIZE != 0)
            return fail(TFQ_E_INVAL, "d=%u must be a positive multiple of 64", d);
        if (d > kMaxN) return fail(TFQ_E_UNSUPPORTED, "d=%u exceeds %u", d, kMaxN);
        if (vocab == 0) return fail(TFQ_E_INVAL, "vocab must be positive");
        if (!(eps > 0.0f)) return fail(TFQ_E_INVAL, "RMSNorm eps must be positive");
        if (!hidden || !weights || !scales || !biases || !out_token || !workspace)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(weights, 16)) return fail(TFQ_E_INVAL, "weights are not 16-byte aligned");
        if (!aligned(hidden, 2) || !aligned(norm_weight, 2) || !aligned(scales, 2) || !aligned(biases, 2))
            return fail(TFQ_E_INVAL, "hidden/norm/scales/biases are not 2-byte aligned");
        if (!aligned(out_token, 4) || !aligned(workspace, 8))
            return fail(TFQ_E_INVAL, "out_token must be 4-byte and workspace 8-byte aligned");
        if (workspace_bytes < 8) return fail(TFQ_E_INVAL, "workspace too small");
        Q4Multi mats{};
        mats.m[0] = {static_cast<const uint8_t*>(weights), scales, biases, nullptr, nullptr, vocab, 0};
        mats.nmat = 1;
        mats.total_rows = vocab;
        mats.norm = NormArg{norm_weight, nullptr, nullptr, eps, kStageNorm};
        const SegShape sh = seg_shape_fit(d / 32, 2);
        // 16-byte aligned hidden state and norm weight: the form with the
        // RMSNorm staging fixed at compile time
        const bool fixed = aligned(hidden, 16) && aligned(norm_weight, 16) && d <= kFixedStageMaxN;
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_lm_head_greedy_%ss%u_p%u", fixed ? "rms_" : "", sh.seg, sh.p);
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = xpairs_lds_bytes(d);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg) * kRowsInFlight;
        uint32_t grid = grid_for_rows(m_, fn, lds, vocab, rows_per_block);
        const uint64_t max_blocks = workspace_bytes / 8;
        if (grid > max_blocks) grid = (uint32_t)max_blocks;      // the row loop covers the rest
        uint64_t* summaries = static_cast<uint64_t*>(workspace);
        uint32_t dd = d;
        void* args[] = {&mats, &hidden, &dd, &summaries};
        int rc = launch(fn, grid, kBlock, lds, stream, args, name);
        if (rc) return rc;
        void* rargs[] = {&summaries, &grid, &out_token};
        return launch(m_.get("tfq_lm_head_reduce"), 1, kBlock, 0, stream, rargs, "tfq_lm_head_reduce");
    }

private:
    const Module& m_;
};

// Code width of a pool's rows: weight_bits, 0 meaning 4 (the `bits: Int = 4`
// default of S/Kernels/MoE/MoE.swift:244).
inline uint32_t pool_bits(const tfq_expert_pool& pool) { return pool.weight_bits ? pool.weight_bits : 4u; }

// Shared pool checks / conversion for the MoE operators.
inline int check_expert_pool(const tfq_expert_pool& pool, uint32_t d, uint32_t f) {
    const uint32_t bits = pool_bits(pool);
    if (bits < 2 || bits > 4)     // MoE.swift:365-375: 4, or the 2/3-bit variants
        return fail(TFQ_E_INVAL, "unsupported routed expert weight bits %u", pool.weight_bits);
    if (d == 0 || d % TFQ_GROUP_SIZE != 0 || f == 0 || f % TFQ_GROUP_SIZE != 0)
        return fail(TFQ_E_INVAL, "d=%u and f=%u must be positive multiples of 64", d, f);
    if (!pool.base || pool.num_experts == 0) return fail(TFQ_E_INVAL, "empty expert pool");
    const tfq_expert_offsets& o = pool.offsets;
    if (!aligned(pool.base, 16) || pool.stride % 16 != 0 || o.gate_w % 16 || o.up_w % 16 ||
        o.down_w % 16)
        return fail(TFQ_E_INVAL, "pool base, stride and weight offsets must be 16-byte aligned");
    if ((o.gate_s | o.gate_b | o.up_s | o.up_b | o.down_s | o.down_b) & 1u)
        return fail(TFQ_E_INVAL, "scale/bias offsets must be 2-byte aligned");
    // every sub-tensor must lie inside one blob
    const uint64_t wbytes = (uint64_t)f * d / 8 * bits, sbytes = (uint64_t)f * (d / 64) * 2;
    const uint64_t ends[9] = {o.gate_w + wbytes, o.gate_s + sbytes, o.gate_b + sbytes,
                              o.up_w + wbytes,   o.up_s + sbytes,   o.up_b + sbytes,
                              o.down_w + wbytes, o.down_s + (uint64_t)d * (f / 64) * 2,
                              o.down_b + (uint64_t)d * (f / 64) * 2};
    for (uint64_t e : ends)
        if (e > pool.stride) return fail(TFQ_E_INVAL, "expert sub-tensor exceeds the pool stride");
    return TFQ_OK;
}

inline ExpertPool kernel_pool(const tfq_expert_pool& p) {
    ExpertPool k{};
    k.base = static_cast<const uint8_t*>(p.base);
    k.stride = p.stride;
    k.num_experts = p.num_experts;
    const tfq_expert_offsets& o = p.offsets;
    k.off = {o.gate_w, o.gate_s, o.gate_b, o.up_w, o.up_s, o.up_b, o.down_w, o.down_s, o.down_b};
    return k;
}

// S/Kernels/MoE/MoE.swift:31-414: router + routed decode phases.
class MoE {
public:
    explicit MoE(const Module& m) : m_(m) {}

    // MoE.encodeRouterGemma4 (MoE.swift:147-197): the logits GEMV (many
    // blocks), then a one-block selection; stream order is the only sync.
    int encode_router_gemma4(void* stream, const uint8_t* weights, const uint16_t* scales,
                             const uint16_t* biases, const uint16_t* hidden,
                             const uint16_t* effective_scale, const uint16_t* per_expert_scale,
                             uint32_t* out_indices, uint16_t* out_weights, float* out_weights_f32,
                             float* out_logits, uint32_t num_experts, uint32_t d, uint32_t top_k,
                             void* workspace, const NormArg& stage = stage_copy()) const {
        float* logits = nullptr;
        int rc = encode_router_logits(stream, weights, scales, biases, hidden, effective_scale, out_logits,
                                      num_experts, d, top_k, workspace, stage, &logits);
        if (rc) return rc;
        if (!out_indices || !out_weights) return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(out_indices, 4)) return fail(TFQ_E_INVAL, "indices are not 4-byte aligned");
        void* sargs[] = {&logits, &per_expert_scale, &out_indices, &out_weights, &out_weights_f32,
                         &num_experts, &top_k};
        return launch(m_.get("tfq_router_select"), 1, 256, 0, stream, sargs, "tfq_router_select");
    }

    // The router GEMV alone (the selection then runs inside phase 1); the
    // logits land in out_logits, or the workspace when it is null.
    int encode_router_logits(void* stream, const uint8_t* weights, const uint16_t* scales,
                             const uint16_t* biases, const uint16_t* hidden,
                             const uint16_t* effective_scale, float* out_logits, uint32_t num_experts,
                             uint32_t d, uint32_t top_k, void* workspace, const NormArg& stage,
                             float** logits_used) const {
        if (d == 0 || d % TFQ_GROUP_SIZE != 0)
            return fail(TFQ_E_INVAL, "d=%u must be a positive multiple of 64", d);
        if (d > 4096) return fail(TFQ_E_UNSUPPORTED, "router d=%u exceeds 4096", d);
        if (num_experts == 0 || num_experts > 256)
            return fail(TFQ_E_INVAL, "numExperts=%u must be in 1...256", num_experts);
        if (top_k == 0 || top_k > 64 || top_k > num_experts)
            return fail(TFQ_E_INVAL, "topK=%u must be in 1...min(64, numExperts)", top_k);
        if (!weights || !scales || !biases || !hidden || !workspace)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(weights, 16)) return fail(TFQ_E_INVAL, "weights are not 16-byte aligned");
        if (!aligned(workspace, 16)) return fail(TFQ_E_INVAL, "workspace is not 16-byte aligned");
        if (int rc = check_stage(stage)) return rc;
        float* logits = out_logits ? out_logits : static_cast<float*>(workspace);
        *logits_used = logits;
        const SegShape sh = seg_shape(d / 16, 4);
        // aligned inputs in the copy or post-attention mode take the form with
        // the staging mode fixed at compile time (d <= 4096 is checked above)
        bool vec = aligned(hidden, 16) && aligned(effective_scale, 16);
        const char* form = "";
        if (stage.mode == kStageCopy && vec) {
            form = "c_";
        } else if (stage.mode == kStagePostAttn) {
            for (const void* p : {(const void*)stage.w, (const void*)stage.attn, (const void*)stage.attn_w,
                                  (const void*)stage.export_h})
                vec = vec && aligned(p, 16);
            if (vec) form = "pa_";
        }
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_router_logits_%ss%u_p%u", form, sh.seg, sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg);
        const uint32_t grid = (num_experts + rows_per_block - 1) / rows_per_block;
        NormArg na = stage;
        void* args[] = {&weights, &scales, &biases, &hidden, &effective_scale, &logits, &num_experts, &d, &na};
        return launch(m_.get(name), grid, kBlock, d * 6, stream, args, name);
    }

    // encodeRoutedPersistentPhase1U16Load / ...SubsetU16Load (MoE.swift:234-310).
    int encode_phase1(void* stream, const tfq_expert_pool& pool, const uint32_t* indices,
                      const uint16_t* x, uint16_t* acts, const uint32_t* active_slots,
                      uint32_t active_count, uint32_t d, uint32_t f, uint32_t top_k,
                      const NormArg& stage = stage_copy()) const {
        int rc = check_pool(pool, d, f, top_k);
        if (rc) return rc;
        if ((rc = check_stage(stage))) return rc;
        if (d > kMaxN) return fail(TFQ_E_UNSUPPORTED, "d=%u exceeds %u", d, kMaxN);
        if (!indices || !x || !acts) return fail(TFQ_E_INVAL, "null pointer argument");
        if (active_count == 0) return TFQ_OK;               // nothing to do (MoE.swift:283)
        if (active_slots == nullptr && active_count != top_k)
            return fail(TFQ_E_INVAL, "full phase 1 covers exactly topK slots");
        if (active_count > top_k) return fail(TFQ_E_INVAL, "activeCount > topK");
        ExpertPool kp = kernel_pool(pool);
        const SegShape sh = seg_shape_fit(d / 32, 2);
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_moe_phase1_%s%ss%u_p%u", bits_infix(pool), form_prefix(stage),
                      sh.seg, sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg) * kRowsInFlight;
        NormArg na = stage;
        void* args[] = {&kp, &indices, &active_slots, &active_count, &top_k, &x, &acts, &d, &f, &na};
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = xpairs_lds_bytes(d);
        return launch(fn, grid_for_rows(m_, fn, lds, (uint64_t)active_count * f, rows_per_block), kBlock,
                      lds, stream, args, name);
    }

    // Phase 1 that also performs the router's selection from `logits`
    // (every block selects; block 0 writes out_indices / out_weights /
    // out_weights_f32 for phase 2 and the caller).
    int encode_phase1_routed(void* stream, const tfq_expert_pool& pool, const float* logits,
                             const uint16_t* per_expert_scale, uint32_t num_experts, uint32_t* out_indices,
                             uint16_t* out_weights, float* out_weights_f32, const uint16_t* x,
                             uint16_t* acts, uint32_t d, uint32_t f, uint32_t top_k,
                             const NormArg& stage = stage_copy()) const {
        int rc = check_pool(pool, d, f, top_k);
        if (rc) return rc;
        if ((rc = check_stage(stage))) return rc;
        if (d > kMaxN) return fail(TFQ_E_UNSUPPORTED, "d=%u exceeds %u", d, kMaxN);
        if (!logits || !out_indices || !out_weights || !x || !acts)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (num_experts != pool.num_experts)
            return fail(TFQ_E_INVAL, "router has %u experts, pool %u", num_experts, pool.num_experts);
        if (num_experts > 256 || top_k > num_experts)
            return fail(TFQ_E_INVAL, "numExperts must be <= 256 and >= topK");
        ExpertPool kp = kernel_pool(pool);
        const SegShape sh = seg_shape_fit(d / 32, 2);
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_moe_phase1_routed_%s%ss%u_p%u", bits_infix(pool),
                      form_prefix(stage), sh.seg, sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg) * kRowsInFlight;
        NormArg na = stage;
        void* args[] = {&kp,   &logits, &per_expert_scale, &num_experts, &top_k, &out_indices, &out_weights,
                        &out_weights_f32, &x, &acts, &d, &f, &na};
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = xpairs_lds_bytes(d);
        return launch(fn, grid_for_rows(m_, fn, lds, (uint64_t)top_k * f, rows_per_block), kBlock, lds,
                      stream, args, name);
    }

    // encodeRoutedPersistentPhase2Reduce (MoE.swift:312-362).
    int encode_phase2(void* stream, const tfq_expert_pool& pool, const uint32_t* indices,
                      const uint16_t* acts, const uint16_t* routing_weights, const uint16_t* residual,
                      uint16_t* y, uint32_t d, uint32_t f, uint32_t top_k) const {
        int rc = check_pool(pool, d, f, top_k);
        if (rc) return rc;
        if (f > 1024) return fail(TFQ_E_UNSUPPORTED, "phase 2 f=%u exceeds 1024", f);
        if (!indices || !acts || !routing_weights || !y)
            return fail(TFQ_E_INVAL, "null pointer argument");
        ExpertPool kp = kernel_pool(pool);
        const uint32_t p = ((f / 32) + 7) / 8;
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_moe_phase2_%sp%u", bits_infix(pool), p);
        void* args[] = {&kp, &indices, &acts, &routing_weights, &residual, &y, &d, &f, &top_k};
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = xpairs_lds_bytes(top_k * f);
        return launch(fn, grid_for_rows(m_, fn, lds, d, (kBlock / 64) * kRowsInFlight), kBlock, lds, stream,
                      args, name);
    }

    // The decoder layer's phase 1 with the shared expert's gate/up/act in the
    // same launch (moe_phase1_routed_shared / _shared8): x = h (kStageScaled),
    // the routed input normed with stage.w, the shared one with
    // shared_norm_w; the shared expert's act lands in shared_act.
    // shared_bits 4 or 8; 4-bit pools only.
    int encode_phase1_shared(void* stream, const tfq_expert_pool& pool, const float* logits,
                             const uint16_t* per_expert_scale, uint32_t num_experts, uint32_t* out_indices,
                             uint16_t* out_weights, const uint16_t* x, uint16_t* acts, uint32_t d, uint32_t f,
                             uint32_t top_k, const NormArg& stage, const tfq_q4_matrix& gate,
                             const tfq_q4_matrix& up, const uint16_t* shared_norm_w, uint16_t* shared_act,
                             uint32_t fs, uint32_t shared_bits) const {
        int rc = check_pool(pool, d, f, top_k);
        if (rc) return rc;
        if ((rc = check_stage(stage))) return rc;
        if (pool_bits(pool) != 4) return fail(TFQ_E_UNSUPPORTED, "the fused shared form takes 4-bit experts");
        if (stage.mode != kStageScaled) return fail(TFQ_E_INVAL, "the fused shared form stages h scaled by r(h)");
        if (shared_bits != 4 && shared_bits != 8)
            return fail(TFQ_E_INVAL, "SharedExpert unsupported weight bits: %u", shared_bits);
        // both parts stage h with the scaled mode fixed at compile time:
        // 16-byte aligned vectors, d <= kFixedStageMaxN
        if (d > kFixedStageMaxN) return fail(TFQ_E_UNSUPPORTED, "d=%u exceeds %u", d, kFixedStageMaxN);
        for (const void* p : {(const void*)x, (const void*)stage.w, (const void*)shared_norm_w, (const void*)stage.inv})
            if (!aligned(p, 16)) return fail(TFQ_E_INVAL, "h, r(h) and the norm weights must be 16-byte aligned");
        if (fs == 0 || fs % 64) return fail(TFQ_E_INVAL, "shared f=%u must be a positive multiple of 64", fs);
        if (!logits || !out_indices || !out_weights || !x || !acts || !shared_act || !gate.weights || !up.weights ||
            !gate.scales || !gate.biases || !up.scales || !up.biases)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(gate.weights, 16) || !aligned(up.weights, 16))
            return fail(TFQ_E_INVAL, "gate/up weights must be 16-byte aligned");
        if (num_experts != pool.num_experts)
            return fail(TFQ_E_INVAL, "router has %u experts, pool %u", num_experts, pool.num_experts);
        if (num_experts > 256 || top_k > num_experts)
            return fail(TFQ_E_INVAL, "numExperts must be <= 256 and >= topK");
        ExpertPool kp = kernel_pool(pool);
        const SegShape sh = seg_shape_fit(d / 32, 2);
        const SegShape s8 = seg_shape(d / 16, 4);
        char name[64];
        if (shared_bits == 8)
            std::snprintf(name, sizeof(name), "tfq_moe_phase1_shared8_s%u_p%u_q%u_%u", sh.seg, sh.p, s8.seg, s8.p);
        else
            std::snprintf(name, sizeof(name), "tfq_moe_phase1_shared_s%u_p%u", sh.seg, sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg) * kRowsInFlight;
        const uint32_t shared_rows_per_block =
            (kBlock / 64) * (64 / (shared_bits == 8 ? s8.seg : sh.seg)) * kRowsInFlight;
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = std::max(xpairs_lds_bytes(d), shared_bits == 8 ? d * 6 : 0u);
        // each part's grid as it would be launched alone
        uint32_t shared_blocks = grid_for_rows(m_, fn, lds, fs, shared_rows_per_block);
        const uint32_t routed_blocks = grid_for_rows(m_, fn, lds, (uint64_t)top_k * f, rows_per_block);
        float* no_wf = nullptr;
        NormArg na = stage;
        Q4Mat g4 = {static_cast<const uint8_t*>(gate.weights), gate.scales, gate.biases, nullptr, nullptr, fs, 0};
        Q4Mat u4 = {static_cast<const uint8_t*>(up.weights), up.scales, up.biases, nullptr, nullptr, fs, 0};
        Q8Mat g8 = {static_cast<const uint8_t*>(gate.weights), gate.scales, gate.biases};
        Q8Mat u8 = {static_cast<const uint8_t*>(up.weights), up.scales, up.biases};
        void* gp = shared_bits == 8 ? (void*)&g8 : (void*)&g4;
        void* upp = shared_bits == 8 ? (void*)&u8 : (void*)&u4;
        void* args[] = {&kp,    &logits, &per_expert_scale, &num_experts, &top_k, &out_indices, &out_weights,
                        &no_wf, &x,      &acts,             &d,           &f,     &na,          gp,
                        upp,    &shared_norm_w, &shared_act, &fs,         &shared_blocks};
        return launch(fn, shared_blocks + routed_blocks, kBlock, lds, stream, args, name);
    }

    // Phase 2 (no residual) with the shared expert's down GEMV (rows of fs
    // codes, fs <= 4096) into shared_y in the same launch (moe_phase2_shared /
    // _shared8). shared_bits 4 or 8; 4-bit pools only.
    int encode_phase2_shared(void* stream, const tfq_expert_pool& pool, const uint32_t* indices,
                             const uint16_t* acts, const uint16_t* routing_weights, uint16_t* y, uint32_t d,
                             uint32_t f, uint32_t top_k, const tfq_q4_matrix& down, const uint16_t* shared_act,
                             uint16_t* shared_y, uint32_t fs, uint32_t shared_bits) const {
        int rc = check_pool(pool, d, f, top_k);
        if (rc) return rc;
        if (pool_bits(pool) != 4) return fail(TFQ_E_UNSUPPORTED, "the fused shared form takes 4-bit experts");
        if (shared_bits != 4 && shared_bits != 8)
            return fail(TFQ_E_INVAL, "SharedExpert unsupported weight bits: %u", shared_bits);
        if (f > 1024) return fail(TFQ_E_UNSUPPORTED, "phase 2 f=%u exceeds 1024", f);
        if (fs == 0 || fs % 64 || fs > 4096)
            return fail(TFQ_E_UNSUPPORTED, "shared f=%u must be a multiple of 64 up to 4096", fs);
        if (!indices || !acts || !routing_weights || !y || !shared_act || !shared_y || !down.weights ||
            !down.scales || !down.biases)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(down.weights, 16)) return fail(TFQ_E_INVAL, "down weights must be 16-byte aligned");
        // both parts stage their acts with the fixed-mode copy (16-byte loads)
        if (!aligned(shared_act, 16) || !aligned(acts, 16))
            return fail(TFQ_E_INVAL, "acts must be 16-byte aligned");
        ExpertPool kp = kernel_pool(pool);
        const uint32_t p2 = ((f / 32) + 7) / 8;
        const SegShape s8 = seg_shape(fs / 16, 4);
        char name[64];
        if (shared_bits == 8)
            std::snprintf(name, sizeof(name), "tfq_moe_phase2_shared8_p%u_q%u_%u", p2, s8.seg, s8.p);
        else
            std::snprintf(name, sizeof(name), "tfq_moe_phase2_shared_p%u_sp%u", p2, ((fs / 32) + 31) / 32);
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = std::max(xpairs_lds_bytes(top_k * f), shared_bits == 8 ? fs * 6 : xpairs_lds_bytes(fs));
        const uint32_t shared_rows_per_block = (kBlock / 64) * (shared_bits == 8 ? 64 / s8.seg : 2) * kRowsInFlight;
        uint32_t shared_blocks = grid_for_rows(m_, fn, lds, d, shared_rows_per_block);
        const uint32_t routed_blocks = grid_for_rows(m_, fn, lds, d, (kBlock / 64) * kRowsInFlight);
        Q4Mat dn4 = {static_cast<const uint8_t*>(down.weights), down.scales, down.biases, nullptr, nullptr, d, 0};
        Q8Mat dn8 = {static_cast<const uint8_t*>(down.weights), down.scales, down.biases};
        void* dp = shared_bits == 8 ? (void*)&dn8 : (void*)&dn4;
        void* args[] = {&kp, &indices, &acts, &routing_weights, &y, &d, &f, &top_k, dp, &shared_act, &shared_y,
                        &fs, &shared_blocks};
        return launch(fn, shared_blocks + routed_blocks, kBlock, lds, stream, args, name);
    }

private:
    // Kernel-name infix of the pool's code width: "" (4 bits), "b2_", "b3_".
    static const char* bits_infix(const tfq_expert_pool& pool) {
        const uint32_t b = pool_bits(pool);
        return b == 2 ? "b2_" : b == 3 ? "b3_" : "";
    }

    int check_pool(const tfq_expert_pool& pool, uint32_t d, uint32_t f, uint32_t top_k) const {
        if (top_k == 0 || top_k > 8) return fail(TFQ_E_INVAL, "topK=%u must be in 1...8", top_k);
        return check_expert_pool(pool, d, f);
    }

    const Module& m_;
};

// S/Kernels/MoE/SharedExpertInt4.swift:21-95.
class SharedExpertInt4 {
public:
    explicit SharedExpertInt4(const Module& m) : m_(m), gemv_(m) {}

    int encode(void* stream, const uint16_t* x, const tfq_q4_matrix& gate, const tfq_q4_matrix& up,
               const tfq_q4_matrix& down, uint16_t* y, uint32_t d, uint32_t f,
               uint16_t* act_scratch, const NormArg& stage = stage_copy()) const {
        if (d == 0 || f == 0 || d % 64 || f % 64)
            return fail(TFQ_E_INVAL, "dimension mismatch: d=%u f=%u must be multiples of 64", d, f);
        if (d > kMaxN || f > kMaxN) return fail(TFQ_E_UNSUPPORTED, "d/f exceed %u", kMaxN);
        if (!x || !y || !act_scratch || !gate.weights || !up.weights || !down.weights ||
            !gate.scales || !gate.biases || !up.scales || !up.biases)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(gate.weights, 16) || !aligned(up.weights, 16))
            return fail(TFQ_E_INVAL, "gate/up weights must be 16-byte aligned");
        if (int rc = check_stage(stage)) return rc;
        Q4Mat g = {static_cast<const uint8_t*>(gate.weights), gate.scales, gate.biases, nullptr, nullptr, f, 0};
        Q4Mat u = {static_cast<const uint8_t*>(up.weights), up.scales, up.biases, nullptr, nullptr, f, 0};
        NormArg na = stage;
        const SegShape sh = seg_shape_fit(d / 32, 2);
        // an aligned x in the copy mode: the form whose staging is fixed at
        // compile time
        const char* form = na.mode == kStageCopy && aligned(x, 16) && d <= kFixedStageMaxN ? "c_" : form_prefix(na);
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_gate_up_act_%ss%u_p%u", form, sh.seg, sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg) * kRowsInFlight;
        void* args[] = {&g, &u, &x, &act_scratch, &d, &f, &na};
        hipFunction_t fn = m_.get(name);
        const uint32_t lds = xpairs_lds_bytes(d);
        int rc = launch(fn, grid_for_rows(m_, fn, lds, f, rows_per_block), kBlock, lds, stream, args, name);
        if (rc) return rc;
        return gemv_.encode(stream, down.weights, down.scales, down.biases, act_scratch, y, d, f);
    }

private:
    const Module& m_;
    DequantInt4GEMV gemv_;
};

// S/Kernels/MoE/SharedExpertInt8.swift:55-210: the fused int8 gate/up/act
// (shared_int8_gate_up_act_simd; gate and up kept in fp32 up to the
// activation) and the int8 down GEMV. tokens > 1 runs the same for a block
// of inputs x + t·x_stride into y + t·y_stride, act_scratch [tokens][f].
class SharedExpertInt8 {
public:
    explicit SharedExpertInt8(const Module& m) : m_(m), gemv_(m) {}

    int encode(void* stream, const uint16_t* x, const tfq_q4_matrix& gate, const tfq_q4_matrix& up,
               const tfq_q4_matrix& down, uint16_t* y, uint32_t d, uint32_t f, uint16_t* act_scratch,
               const NormArg& stage = stage_copy(), uint32_t tokens = 1, uint32_t x_stride = 0,
               uint32_t y_stride = 0) const {
        if (d == 0 || f == 0 || d % 64 || f % 64)
            return fail(TFQ_E_INVAL, "SharedExpertInt8 dimension mismatch: d=%u f=%u must be multiples of 64", d, f);
        if (d > 4096 || f > 4096) return fail(TFQ_E_UNSUPPORTED, "int8 shared expert d/f exceed 4096");
        if (tokens == 0 || tokens > 65535) return fail(TFQ_E_INVAL, "token count %u must be in 1...65535", tokens);
        if (!x || !y || !act_scratch || !gate.weights || !up.weights || !down.weights || !gate.scales ||
            !gate.biases || !up.scales || !up.biases || !down.scales || !down.biases)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(gate.weights, 16) || !aligned(up.weights, 16))
            return fail(TFQ_E_INVAL, "gate/up weights must be 16-byte aligned");
        if (tokens > 1 && (x_stride < d || y_stride < d))
            return fail(TFQ_E_INVAL, "x/y strides must be at least d");
        if (int rc = check_stage(stage)) return rc;
        Q8Mat g = {static_cast<const uint8_t*>(gate.weights), gate.scales, gate.biases};
        Q8Mat u = {static_cast<const uint8_t*>(up.weights), up.scales, up.biases};
        NormArg na = stage;
        const SegShape sh = seg_shape(d / 16, 4);
        char name[64];
        // 16-byte aligned rows of x in the copy mode: the form whose staging is
        // fixed at compile time (d <= 4096 is checked above)
        const bool fixed = na.mode == kStageCopy && aligned(x, 16) && (tokens == 1 || x_stride % 8 == 0);
        std::snprintf(name, sizeof(name), "tfq_q8_gate_up_act_%ss%u_p%u", fixed ? "c_" : form_prefix(na), sh.seg,
                      sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg) * kRowsInFlight;
        void* args[] = {&g, &u, &x, &x_stride, &act_scratch, &d, &f, &na};
        hipFunction_t fn = m_.get(name);
        if (!fn) return fail(TFQ_E_NOT_LOADED, "kernel %s is not in the code object", name);
        const uint32_t lds = d * 6;
        int rc = hip_check(hipModuleLaunchKernel(fn, grid_for_rows(m_, fn, lds, f, rows_per_block), tokens, 1,
                                                 kBlock, 1, 1, lds, (hipStream_t)stream, args, nullptr),
                           name);
        if (rc) return rc;
        return gemv_.encode(stream, static_cast<const uint8_t*>(down.weights), down.scales, down.biases,
                            act_scratch, y, d, f, tokens, f, tokens > 1 ? y_stride : 0);
    }

private:
    const Module& m_;
    DequantInt8GEMV gemv_;
};

inline int launch2(const Module& m, const char* name, uint32_t gx, uint32_t gy, uint32_t block,
                   uint32_t lds, void* stream, void** args) {
    hipFunction_t f = m.get(name);
    if (!f) return fail(TFQ_E_NOT_LOADED, "kernel %s is not in the code object", name);
    return hip_check(hipModuleLaunchKernel(f, gx, gy, 1, block, 1, 1, lds, (hipStream_t)stream, args,
                                           nullptr),
                     name);
}

constexpr uint32_t kSkinnyTok = 16;         // tokens per skinny block row (gemm_skinny.hpp kSkinnyTok)
constexpr uint32_t kSkinnyThreads = 512;    // (gemm_skinny.hpp kSkinnyThreads)

// The prefill projection's kernel choice by token count, the role of
// PrefillProjectionDispatchPolicy (S/Runtime/Inference/RealForwardRunner.swift:
// 217-230, 1411-1492: repeated GEMV below 32 tokens, QMM / MPP above). Here
// one token takes the decode GEMV; the other kernels are the few-token weight stream (gemm_skinny.hpp: every
// weight dequantised once per 16 tokens, 8 K-slices per block, N/16 or N/32
// blocks) and the 64-token projection tile (gemm.hpp: N/256 blocks per
// token tile). Both multiply the same fp16 weights, so the choice changes
// time, not results beyond fp32 summation order. The skinny form is used up
// to the largest token count at which it measured faster on MI355X for that
// output count (K = 2816; see skinny_max_tokens).
struct GemmPlan {
    int path;        // TFQ_GEMM_PATH_TILE, _SKINNY (16 rows per wave) or _SKINNY32 (32)
};

// Largest token count at which the weight stream beat the tile on MI355X
// (bf16 activations, K = 2816, back-to-back launches; the tile takes ~28 us
// at any token count up to 448 at these shapes, the stream grows by one
// weight pass per 16 tokens): N = 2048: 320, 2816: 192, 4096: 160, 8192: 80.
// Other N follow the measured ~1/N trend. The crossover is taken to be
// independent of K: both kernels' times scale with K.
inline uint32_t skinny_max_tokens(uint32_t n, uint32_t k) {
    (void)k;
    if (n <= 2048) return 320;
    if (n <= 2816) return 192;
    if (n <= 4096) return 160;
    if (n <= 8192) return 80;
    const uint32_t t = 655360u / n / 16u * 16u;
    return t < 16 ? 16 : t;
}

inline GemmPlan plan_gemm(uint32_t t, uint32_t n, uint32_t k) {
    // one token: the decode GEMV (N 2048: 3.9 against 4.4 us for the weight
    // stream, N 8192: 5.8 against 6.4 us, cold weights); from two tokens on
    // the stream reads the weights once for up to 16 tokens and wins (N 8192,
    // two tokens: 6.5 against 11.2 us for two GEMVs)
    if (t == 1) return {TFQ_GEMM_PATH_GEMV};
    if (t > skinny_max_tokens(n, k)) return {TFQ_GEMM_PATH_TILE};
    // 16 rows per wave keeps more blocks for narrow matrices and few tokens;
    // 32 rows per wave halves the activation reads and wins elsewhere
    const bool rows16 = (t <= 16 && n < 8192) || (t <= 32 && n <= 2048);
    return {rows16 ? TFQ_GEMM_PATH_SKINNY : TFQ_GEMM_PATH_SKINNY32};
}

// S/Kernels/Prefill/Primitives/PrefillPrimitives.swift:73-123 (PrefillInt4QMM) and
// S/Kernels/TensorCore/MPPPrefillInt4QMM.swift:4-83, with the GEMV-vs-QMM
// choice of RealForwardRunner.swift:217-230 made inside (plan_gemm).
class PrefillInt4QMM {
public:
    explicit PrefillInt4QMM(const Module& m) : m_(m) {}

    // bits: 4, or 3 (PrefillPrimitives.swift:91-99; prefill.metal:711-757).
    // path: TFQ_GEMM_PATH_AUTO (plan_gemm) or a forced kernel.
    // ldx / ldy: halves between token rows of x / y (0: k / n).
    int encode(void* stream, const void* weights, const uint16_t* scales, const uint16_t* biases,
               const uint16_t* x, uint16_t* y, uint32_t t, uint32_t n, uint32_t k, int dtype,
               uint32_t bits = 4, int path = TFQ_GEMM_PATH_AUTO, uint32_t ldx = 0, uint32_t ldy = 0) const {
        if (ldx == 0) ldx = k;
        if (ldy == 0) ldy = n;
        if (bits != 3 && bits != 4) return fail(TFQ_E_INVAL, "unsupported attention weight bits %u", bits);
        if (k == 0 || k % TFQ_GROUP_SIZE != 0)
            return fail(TFQ_E_INVAL, "k=%u must be a positive multiple of 64", k);
        if (n == 0) return fail(TFQ_E_INVAL, "output count must be positive");
        if (t == 0) return fail(TFQ_E_INVAL, "token count must be positive");
        if (dtype != TFQ_DTYPE_F16 && dtype != TFQ_DTYPE_BF16)
            return fail(TFQ_E_INVAL, "dtype %d is neither fp16 nor bf16", dtype);
        if (!weights || !scales || !biases || !x || !y) return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(weights, 16) || !aligned(x, 16))
            return fail(TFQ_E_INVAL, "weights and x must be 16-byte aligned");
        if (!aligned(scales, 2) || !aligned(biases, 2) || !aligned(y, 2))
            return fail(TFQ_E_INVAL, "scales/biases/y must be 2-byte aligned");
        if (ldx < k || ldx % 8 != 0) return fail(TFQ_E_INVAL, "x row stride %u must be >= k and a multiple of 8", ldx);
        if (ldy < n) return fail(TFQ_E_INVAL, "y row stride %u must be >= n", ldy);
        if (k > kProjMaxK) return fail(TFQ_E_UNSUPPORTED, "k=%u exceeds %u", k, kProjMaxK);
        if (path == TFQ_GEMM_PATH_AUTO) path = plan_gemm(t, n, k).path;
        if (path == TFQ_GEMM_PATH_GEMV) {
            // the decode GEMV once per token (bf16 rows converted while staged)
            if (bits != 4 && bits != 3) return fail(TFQ_E_INVAL, "unsupported attention weight bits %u", bits);
            const DequantInt4GEMV gemv(m_);
            NormArg stage = stage_copy();
            if (dtype == TFQ_DTYPE_BF16) stage.mode = kStageBf16;
            for (uint32_t i = 0; i < t; ++i)
                if (int rc = gemv.encode(stream, weights, scales, biases, x + (size_t)i * ldx, y + (size_t)i * ldy, n,
                                         k, nullptr, stage, bits))
                    return rc;
            return TFQ_OK;
        }
        if (path == TFQ_GEMM_PATH_SKINNY || path == TFQ_GEMM_PATH_SKINNY32) {
            const uint32_t rt = path == TFQ_GEMM_PATH_SKINNY32 ? 2 : 1;
            char sname[64];
            std::snprintf(sname, sizeof(sname), "tfq_gemm_skinny_q%u_%s_r%u_c%u", bits,
                          dtype == TFQ_DTYPE_BF16 ? "bf16" : "f16", rt, (k + 1023) / 1024);
            const uint32_t gx = (n + 16 * rt - 1) / (16 * rt), gy = (t + kSkinnyTok - 1) / kSkinnyTok;
            void* args[] = {&x, &weights, &scales, &biases, &y, &t, &n, &k, &ldx, &ldy};
            return launch2(m_, sname, gx, gy, kSkinnyThreads, 0, stream, args);
        }
        if (path != TFQ_GEMM_PATH_TILE) return fail(TFQ_E_INVAL, "unknown GEMM path %d", path);
        const char* name = bits == 3 ? (dtype == TFQ_DTYPE_BF16 ? "tfq_gemm_q3_bf16" : "tfq_gemm_q3_f16")
                                     : (dtype == TFQ_DTYPE_BF16 ? "tfq_gemm_q4_bf16" : "tfq_gemm_q4_f16");
        hipFunction_t f = m_.get(name);
        if (!f) return fail(TFQ_E_NOT_LOADED, "kernel %s is not in the code object", name);
        // blockIdx.x walks the outputs, so the token tiles that share a weight
        // slice are dispatched to the same XCD (and its L2)
        const uint32_t gx = (n + kProjBN - 1) / kProjBN, gy = (t + kProjBM - 1) / kProjBM;
        const uint32_t lds = proj_pl_lds_bytes(k);
        void* args[] = {&x, &weights, &scales, &biases, &y, &t, &n, &k, &ldx, &ldy};
        return hip_check(hipModuleLaunchKernel(f, gx, gy, 1, kProjGemmThreads, 1, 1, lds, (hipStream_t)stream,
                                               args, nullptr),
                         name);
    }

private:
    const Module& m_;
};


// S/Kernels/Prefill/MoE/PrefillSharedExpert.swift:4-60 (encodeBlock): the
// shared expert over `tokens` rows x + t·x_stride -> y + t·y_stride. The
// reference runs the decode form once per row; here int8 weights run the
// decode kernels with a token dimension (one launch each for gate/up/act and
// down), and int4 weights run the prefill GEMM (gate, up -> fp16 in the
// workspace, gelu_mul_fp16 as in SharedExpertInt4's GPU sequence, then
// down), whose kernel choice by token count picks the weight stream for few
// tokens.
class PrefillSharedExpert {
public:
    PrefillSharedExpert(const Module& m, const SharedExpertInt8& int8, const PrefillInt4QMM& qmm)
        : m_(m), int8_(int8), qmm_(qmm) {}

    static size_t workspace_bytes(uint32_t bits, uint32_t tokens, uint32_t f) {
        const size_t one = ((size_t)tokens * f * 2 + 255) / 256 * 256;
        return bits == 8 ? one : 2 * one;
    }

    int encode(void* stream, uint32_t bits, const tfq_q4_matrix& gate, const tfq_q4_matrix& up,
               const tfq_q4_matrix& down, const uint16_t* x, uint32_t x_stride, uint16_t* y, uint32_t y_stride,
               uint32_t tokens, uint32_t d, uint32_t f, void* workspace, size_t workspace_size) const {
        if (bits != 4 && bits != 8) return fail(TFQ_E_INVAL, "SharedExpert unsupported weight bits: %u", bits);
        if (tokens == 0) return TFQ_OK;                         // queryCount 0: nothing to encode
        if (x_stride < d) return fail(TFQ_E_INVAL, "x stride is too small");
        if (y_stride < d) return fail(TFQ_E_INVAL, "y stride is too small");
        if (!workspace || !aligned(workspace, 256)) return fail(TFQ_E_INVAL, "workspace must be 256-byte aligned");
        if (workspace_size < workspace_bytes(bits, tokens, f))
            return fail(TFQ_E_INVAL, "SharedExpert scratch too small");
        uint16_t* a = static_cast<uint16_t*>(workspace);
        if (bits == 8)
            return int8_.encode(stream, x, gate, up, down, y, d, f, a, stage_copy(), tokens, x_stride, y_stride);
        if (!gate.weights || !up.weights || !down.weights) return fail(TFQ_E_INVAL, "null pointer argument");
        uint16_t* u = a + ((size_t)tokens * f * 2 + 255) / 256 * 128;
        int rc = qmm_.encode(stream, gate.weights, gate.scales, gate.biases, x, a, tokens, f, d, TFQ_DTYPE_F16, 4,
                             TFQ_GEMM_PATH_AUTO, x_stride, f);
        if (rc) return rc;
        rc = qmm_.encode(stream, up.weights, up.scales, up.biases, x, u, tokens, f, d, TFQ_DTYPE_F16, 4,
                         TFQ_GEMM_PATH_AUTO, x_stride, f);
        if (rc) return rc;
        uint64_t n = (uint64_t)tokens * f;
        void* args[] = {&a, &u, &a, &n};
        const uint32_t grid = (uint32_t)std::min<uint64_t>((n + kBlock - 1) / kBlock, 4096);
        rc = launch2(m_, "tfq_gelu_mul_f16", grid, 1, kBlock, 0, stream, args);
        if (rc) return rc;
        return qmm_.encode(stream, down.weights, down.scales, down.biases, a, y, tokens, d, f, TFQ_DTYPE_F16, 4,
                           TFQ_GEMM_PATH_AUTO, f, y_stride);
    }

private:
    const Module& m_;
    const SharedExpertInt8& int8_;
    const PrefillInt4QMM& qmm_;
};

// S/Kernels/Prefill/MoE/PrefillRouter.swift:30-112.
class PrefillRouter {
public:
    explicit PrefillRouter(const Module& m) : m_(m) {}

    // PrefillRouter.encodeGemma4Block (PrefillRouter.swift:37-89).
    int encode_gemma4_block(void* stream, const tfq_router& r, const uint16_t* hidden,
                            uint32_t stride, uint32_t T, uint32_t d, uint32_t top_k,
                            uint32_t* out_idx, uint16_t* out_w, float* out_wf, float* logits) const {
        if (T == 0) return fail(TFQ_E_INVAL, "queryCount must be positive");
        if (r.num_experts == 0 || r.num_experts > 256)
            return fail(TFQ_E_INVAL, "numExperts > 256 is not supported");
        if (top_k == 0 || top_k > 64 || top_k > r.num_experts)
            return fail(TFQ_E_INVAL, "topK must be in 1...64");
        if (d == 0 || d % TFQ_GROUP_SIZE) return fail(TFQ_E_INVAL, "D must be a multiple of 64");
        if (d > 4096) return fail(TFQ_E_UNSUPPORTED, "router d=%u exceeds 4096", d);
        if (stride < d) return fail(TFQ_E_INVAL, "hidden stride is too small");
        if (!r.weights || !r.scales || !r.biases || !hidden || !out_idx || !out_w || !logits)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(r.weights, 16)) return fail(TFQ_E_INVAL, "weights are not 16-byte aligned");
        const SegShape sh = seg_shape(d / 16, 4);
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_prefill_router_logits_s%u_p%u", sh.seg, sh.p);
        const uint32_t rows_per_block = (kBlock / 64) * (64 / sh.seg);
        const uint32_t gx = (r.num_experts + rows_per_block - 1) / rows_per_block;
        uint32_t E = r.num_experts;
        void* args[] = {(void*)&r.weights, (void*)&r.scales, (void*)&r.biases, &hidden, &stride,
                        (void*)&r.effective_scale, &logits, &E, &d};
        int rc = launch2(m_, name, gx, T, kBlock, d * 6, stream, args);
        if (rc) return rc;
        void* sargs[] = {&logits, (void*)&r.per_expert_scale, &out_idx, &out_w, &out_wf, &E, &top_k};
        return launch2(m_, "tfq_prefill_select", T, 1, 256, 0, stream, sargs);
    }

private:
    const Module& m_;
};

// Device counterpart of PrefillMoEGrouping.groupTokenExpertPairs
// (S/Kernels/Prefill/MoE/PrefillMoEGrouping.swift:91-192).
class PrefillMoEGrouping {
public:
    explicit PrefillMoEGrouping(const Module& m) : m_(m) {}

    int encode(void* stream, const uint32_t* idx, const uint16_t* w, uint32_t T, uint32_t k, uint32_t E,
               tfq_pair* sorted, uint32_t* offsets, uint32_t* counts, tfq_tile* tiles,
               uint32_t* n_tiles, uint32_t* status) const {
        if (T == 0) return fail(TFQ_E_INVAL, "queryCount must be positive");
        if (k == 0) return fail(TFQ_E_INVAL, "topK must be positive");
        if (E == 0 || E > 256) return fail(TFQ_E_INVAL, "numExperts must be in 1...256");
        if ((uint64_t)T * k > 8192) return fail(TFQ_E_UNSUPPORTED, "more than 8192 pairs");
        if (!idx || !w || !sorted || !offsets || !counts || !tiles || !n_tiles || !status)
            return fail(TFQ_E_INVAL, "null pointer argument");
        void* args[] = {&idx, &w, &T, &k, &E, &sorted, &offsets, &counts, &tiles, &n_tiles, &status};
        return launch2(m_, "tfq_moe_group", 1, 1, 1024, 0, stream, args);
    }

private:
    const Module& m_;
};

// S/Kernels/Prefill/MoE/PrefillGroupedRoutedMoE.swift:390-529 (gate/up + down over tiles)
// and S/Kernels/Prefill/MoE/PrefillMoE.swift:4-40 (token-major combine).
class PrefillGroupedRoutedMoE {
public:
    explicit PrefillGroupedRoutedMoE(const Module& m) : m_(m) {}

    int encode(void* stream, const tfq_expert_pool& pool, const tfq_pair* sorted,
               const tfq_tile* tiles, uint32_t* n_tiles, uint32_t max_tiles,
               const uint16_t* hidden, uint32_t stride, uint32_t d, uint32_t f, uint32_t k,
               uint16_t* act, uint16_t* partials) const {
        int rc = check_expert_pool(pool, d, f);
        if (rc) return rc;
        if (!sorted || !tiles || !n_tiles || !hidden || !act || !partials)
            return fail(TFQ_E_INVAL, "null pointer argument");
        if (stride < d || stride % 8) return fail(TFQ_E_INVAL, "hidden stride must be >= d and a multiple of 8");
        if (!aligned(hidden, 16) || !aligned(act, 16) || !aligned(partials, 16))
            return fail(TFQ_E_INVAL, "hidden, act and partials must be 16-byte aligned");
        if (d > kProjMaxK || f > kProjMaxK)
            return fail(TFQ_E_UNSUPPORTED, "d=%u and f=%u must be at most %u", d, f, kProjMaxK);
        if (max_tiles == 0) return TFQ_OK;
        if (max_tiles > kGroupMaxTiles)
            return fail(TFQ_E_UNSUPPORTED, "max_tiles=%u exceeds %u (8192 pairs over 256 experts)", max_tiles,
                        kGroupMaxTiles);
        ExpertPool kp = kernel_pool(pool);
        // one launch per projection over the work list of the tiles: tiles of
        // at most 32 pairs as stream units (RT 4: 128 features / 256 outputs
        // per unit, NTT 1 or 2 pair sub-tiles), larger ones as 64-pair halves
        // on wide units (RT 2: 64 features / 128 outputs, NTT 2 or 4); the
        // grid is the blocks the GPU holds resident, at most the units the
        // tile bound allows
        const uint32_t bits = pool_bits(pool);
        // the _t launches stage each unit's scale/bias table through
        // registers: 16-byte aligned scale/bias arrays (base and stride are)
        // whose unit tables fit (d <= 3072 for gate/up, f <= 1024 for down)
        const tfq_expert_offsets& po = pool.offsets;
        bool sb16 = true;
        for (uint64_t v : {po.gate_s, po.gate_b, po.up_s, po.up_b, po.down_s, po.down_b}) sb16 = sb16 && v % 16 == 0;
        // (moe_prefill.hpp TableRegs: rows·K/64 words in U 16-byte pieces per thread)
        auto fits = [](uint32_t rows, uint32_t K, uint32_t U) { return rows * (K / 64u) <= 8u * U * kUnitThreads; };
        const bool tab_gu = sb16 && fits(128, d, 3), tab_dn = sb16 && fits(256, f, 2);
        char gu[48], dn[48];
        const char* bsuf = bits == 2 ? "_b2" : bits == 3 ? "_b3" : "";
        std::snprintf(gu, sizeof(gu), "tfq_moe_grouped_gate_up%s%s", bsuf, tab_gu ? "_t" : "");
        std::snprintf(dn, sizeof(dn), "tfq_moe_grouped_down%s%s", bsuf, tab_dn ? "_t" : "");
        // dynamic LDS: the largest unit (two activation buffers of 16·NTT
        // rows, then the table of 64·RT rows of K/64 words)
        auto lds_for = [](uint32_t K) {
            auto unit = [K](uint32_t rt, uint32_t ntt) { return 2u * 16u * ntt * kUnitStride * 2u + 4u * 64u * rt * (K / 64u); };
            return std::max(unit(2, 4), unit(4, 2));
        };
        auto grid_for = [&](const char* name, const GroupedLaunch& g, uint32_t lds, uint32_t& grid) {
            hipFunction_t fn = m_.get(name);
            if (!fn) return fail(TFQ_E_NOT_LOADED, "kernel %s is not in the code object", name);
            const uint32_t p = m_.resident_blocks(fn, kUnitThreads, lds);
            const uint32_t units = 2u * max_tiles * std::max(g.wx, g.sx);
            grid = std::min(p, units);
            return TFQ_OK;
        };
        GroupedLaunch g1{max_tiles, (f + 63) / 64, (f + 127) / 128};
        uint32_t grid1 = 0, grid2 = 0;
        rc = grid_for(gu, g1, lds_for(d), grid1);
        if (rc) return rc;
        void* a1[] = {&kp, &sorted, &tiles, &n_tiles, &hidden, &stride, &act, &d, &f, &g1};
        rc = launch2(m_, gu, grid1, 1, kUnitThreads, lds_for(d), stream, a1);
        if (rc) return rc;
        GroupedLaunch g2{max_tiles, (d + 127) / 128, (d + 255) / 256};
        rc = grid_for(dn, g2, lds_for(f), grid2);
        if (rc) return rc;
        void* a2[] = {&kp, &sorted, &tiles, &n_tiles, &act, &partials, &d, &f, &k, &g2};
        return launch2(m_, dn, grid2, 1, kUnitThreads, lds_for(f), stream, a2);
    }

    // PrefillMoE.encodeReduceTokenMajor (PrefillMoE.swift:11-38).
    int encode_reduce_token_major(void* stream, const uint16_t* partials, const uint16_t* w,
                                  uint16_t* h2, uint32_t T, uint32_t k, uint32_t d) const {
        if (T == 0 || k == 0 || d == 0) return fail(TFQ_E_INVAL, "empty reduce");
        if (!partials || !w || !h2) return fail(TFQ_E_INVAL, "null pointer argument");
        void* args[] = {&partials, &w, &h2, &T, &k, &d};
        // 8 outputs per thread when rows allow 16-byte accesses
        if (d % 8 == 0 && aligned(partials, 16) && aligned(h2, 16)) {
            const uint64_t n = (uint64_t)T * (d / 8);
            if (n > 0xFFFFFFFFull) return fail(TFQ_E_UNSUPPORTED, "reduce of %llu outputs", (unsigned long long)n * 8);
            return launch2(m_, "tfq_moe_combine_x8", (uint32_t)((n + 255) / 256), 1, 256, 0, stream, args);
        }
        return launch2(m_, "tfq_moe_combine", (d + 255) / 256, T, 256, 0, stream, args);
    }

private:
    const Module& m_;
};

// S/Kernels/Attention/Attention.swift:26-420: encodeFull (window 0) and
// encodeSWA (window > 0) as split-K partial + combine launches.
class Attention {
public:
    explicit Attention(const Module& m) : m_(m) {}

    static uint32_t kv_start(uint32_t seq_len, uint32_t window) {
        return (window > 0 && seq_len > window) ? seq_len - window : 0;   // Attention.swift:254
    }
    static uint32_t chunks(uint32_t seq_len, uint32_t window) {
        return (seq_len - kv_start(seq_len, window) + kAttnChunk - 1) / kAttnChunk;
    }
    static size_t workspace_bytes(uint32_t head_dim, uint32_t nq, uint32_t seq_len, uint32_t window) {
        if (seq_len == 0) return 0;
        const size_t nc = chunks(seq_len, window);
        return ((size_t)nq * nc * head_dim * 4 + 255) / 256 * 256 + ((size_t)nq * nc * 2 * 4 + 255) / 256 * 256;
    }

    // q: fp16 [nq][hd]; caches fp16 [capacity][nkv][hd]; out fp16 [nq][hd].
    // With epi.q_norm set, q is the raw projection and position seq_len-1 of
    // the caches holds the raw k/v of the new token (rewritten in place).
    int encode(void* stream, const uint16_t* q, uint16_t* k_cache, uint16_t* v_cache, uint16_t* out,
               uint32_t hd, uint32_t nq, uint32_t nkv, uint32_t seq_len, uint32_t window, float scale,
               const AttnEpilogue& epi, void* workspace, size_t workspace_bytes_given) const {
        if (nkv == 0 || nq == 0 || nq % nkv != 0)
            return fail(TFQ_E_INVAL, "numQHeads must be a multiple of numKVHeads for GQA");
        const uint32_t G = nq / nkv;
        if (hd != 128 && hd != 256 && hd != 512)
            return fail(TFQ_E_UNSUPPORTED, "head_dim=%u (supported: 128, 256, 512)", hd);
        if (hd == 512 ? (G != 1 && G != 2 && G != 4 && G != 8) : (G != 1 && G != 2 && G != 4))
            return fail(TFQ_E_UNSUPPORTED, "GQA group %u at head_dim %u (supported: 1, 2, 4%s)", G, hd,
                        hd == 512 ? ", 8" : "");
        // query heads per block (attention.hpp): the 8 of a kv head at head_dim 512 in two blocks
        const uint32_t nsub = hd == 512 && G == 8 ? 2 : 1;
        if (seq_len == 0) return fail(TFQ_E_INVAL, "attention requires at least one KV position");
        if (!q || !k_cache || !v_cache || !out || !workspace) return fail(TFQ_E_INVAL, "null pointer argument");
        if (!aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(workspace, 16))
            return fail(TFQ_E_INVAL, "KV caches and workspace must be 16-byte aligned");
        if (!aligned(q, 16) || !aligned(out, 2)) return fail(TFQ_E_INVAL, "q must be 16-byte and out 2-byte aligned");
        if (!(scale > 0.0f) && !(scale < 0.0f)) return fail(TFQ_E_INVAL, "scale must be non-zero");
        if (epi.q_norm) {
            if (!epi.k_norm) return fail(TFQ_E_INVAL, "q/k epilogue needs both norm weights");
            if (epi.rotated_pairs > hd / 2) return fail(TFQ_E_INVAL, "rotatedPairs exceeds head_dim/2");
            if (!(epi.eps > 0.0f) || !(epi.theta > 0.0f))
                return fail(TFQ_E_INVAL, "epilogue eps and rope theta must be positive");
            if ((epi.k_raw == nullptr) != (epi.v_raw == nullptr))
                return fail(TFQ_E_INVAL, "staged raw k and v go together");
            if (nsub > 1 && !epi.k_raw)
                return fail(TFQ_E_INVAL, "head_dim %u with group %u needs the new k/v staged outside the caches",
                            hd, G);
            if (epi.k_raw && (!aligned(epi.k_raw, 16) || !aligned(epi.v_raw, 16)))
                return fail(TFQ_E_INVAL, "staged k/v rows must be 16-byte aligned");
        }
        const uint32_t nc = chunks(seq_len, window);
        if (nc > kAttnMaxChunks) return fail(TFQ_E_UNSUPPORTED, "more than 65536 visible keys");
        if (workspace_bytes_given < workspace_bytes(hd, nq, seq_len, window))
            return fail(TFQ_E_INVAL, "attention workspace too small");
        float* part_o = static_cast<float*>(workspace);
        float* part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                  ((size_t)nq * nc * hd * 4 + 255) / 256 * 256);
        uint32_t ks = kv_start(seq_len, window);
        AttnEpilogue e = epi;
        e.log2_theta = epi.q_norm ? std::log2((double)epi.theta) : 0.0;
        char name[64];
        std::snprintf(name, sizeof(name), "tfq_attn_partial_h%u_g%u", hd, G);
        void* a1[] = {&q, &k_cache, &v_cache, &nkv, &seq_len, &ks, &scale, &e, &part_o, &part_ml};
        hipFunction_t pf = m_.get(name);
        if (!pf) return fail(TFQ_E_NOT_LOADED, "kernel %s is not in the code object", name);
        int rc = hip_check(hipModuleLaunchKernel(pf, nc, nkv, nsub, 256, 1, 1, 0, (hipStream_t)stream, a1, nullptr),
                           name);
        if (rc) return rc;
        std::snprintf(name, sizeof(name), "tfq_attn_combine_h%u", hd);
        uint32_t ncu = nc;
        void* a2[] = {&part_o, &part_ml, &out, &ncu};
        return launch2(m_, name, nq, hd / kAttnCombineDims, kAttnCombineThreads, 0, stream, a2);
    }

private:
    const Module& m_;
};

// One Gemma 4 decoder layer for one token (RealForwardRunner.swift:2265-2862):
// input norm + QKV, q/k/v epilogue + attention, o projection, post-attention
// setup, router, shared expert, routed experts, tail. The norms that the
// reference runs as separate kernels are formed while each consumer stages
// its activation vector (NormArg); the router also stores the post-attention
// h and r(h), from which the expert launches form their inputs without the
// reductions. Every launch is on `stream`, in order: with 4-bit routed
// experts the shared expert's (int4 or int8) gate/up/act and down run inside
// the routed phase 1 and phase 2 launches (7 launches per layer); otherwise
// as two launches of their own before the router (9). Measured at config 4
// (graph replay): the shared expert on a second stream, concurrent with the
// router and the routed experts, took 66.0 µs per layer against 58.7 µs with
// its two launches in order on the one stream (the concurrent kernels slow
// each other more than the overlap gains).
class DecodeLayer {
public:
    DecodeLayer(const Module& m, DequantInt4GEMV& gemv, MoE& moe, SharedExpertInt4& shared,
                SharedExpertInt8& shared8, Attention& attn)
        : m_(m), gemv_(gemv), moe_(moe), shared_(shared), shared8_(shared8), attn_(attn) {}

    // Segments of the workspace, 256-byte aligned. The d-sized vectors that
    // one layer leaves for the next in a chain (o, h1, h2) come first, so
    // their offsets do not depend on the layer's attention shape.
    struct Layout {
        size_t o, h1, h2, hmid, inv, q, attn, parts, parts_bytes, logits, idx, w, acts, sact, kv, total;
    };
    static Layout layout(const tfq_decode_layer_shape& s, uint32_t max_seq) {
        auto up = [](size_t v) { return (v + 255) / 256 * 256; };
        Layout L{};
        size_t off = 0;
        const size_t qd = (size_t)s.num_q_heads * s.head_dim;
        L.o = off;      off += up((size_t)s.d * 2);
        L.h1 = off;     off += up((size_t)s.d * 2);
        L.h2 = off;     off += up((size_t)s.d * 2);
        L.hmid = off;   off += up((size_t)s.d * 2);
        L.inv = off;    off += up(4);
        L.q = off;      off += up(qd * 2);
        L.attn = off;   off += up(qd * 2);
        L.parts = off;  L.parts_bytes = Attention::workspace_bytes(s.head_dim, s.num_q_heads, max_seq, s.window);
        off += up(L.parts_bytes);
        L.logits = off; off += up(TFQ_ROUTER_WORKSPACE_BYTES);
        L.idx = off;    off += up((size_t)s.top_k * 4);
        L.w = off;      off += up((size_t)s.top_k * 2);
        L.acts = off;   off += up((size_t)s.top_k * s.expert_f * 2);
        L.sact = off;   off += up((size_t)s.shared_f * 2);
        L.kv = off;     off += up((size_t)2 * s.num_kv_heads * s.head_dim * 2);   // staged raw k, v
        L.total = off;
        return L;
    }

    int encode(void* stream, const tfq_decode_layer_weights& w, const tfq_decode_layer_shape& s,
               const uint16_t* hidden_in, uint16_t* hidden_out, uint16_t* k_cache, uint16_t* v_cache,
               uint32_t position, uint32_t* out_indices, uint16_t* out_weights, void* workspace,
               size_t workspace_bytes) {
        if (!hidden_in || !hidden_out) return fail(TFQ_E_INVAL, "null pointer argument");
        if (int rc = check_layer(w, s, k_cache, v_cache, workspace)) return rc;
        for (const void* p : {(const void*)hidden_in, (const void*)hidden_out})
            if (!aligned(p, 16)) return fail(TFQ_E_INVAL, "hidden vectors and norm weights must be 16-byte aligned");
        const Layout L = layout(s, position + 1);
        if (workspace_bytes < L.total) return fail(TFQ_E_INVAL, "decode-layer workspace too small");
        const NormArg in_norm{w.input_norm, nullptr, nullptr, s.eps, kStageNorm};
        if (int rc = body(stream, w, s, hidden_in, in_norm, hidden_in, k_cache, v_cache, position, out_indices,
                          out_weights, static_cast<char*>(workspace), L))
            return rc;
        return tail(stream, w, s, hidden_in, hidden_out, static_cast<char*>(workspace), L);
    }

    // n consecutive layers for one token: layer i's tail (its output, the
    // next layer's input) is formed by layer i+1's QKV GEMV while it stages
    // that input (kStageTail), so a chain of n layers takes n - 1 launches
    // fewer than n calls of encode. hiddens [n][d] receives every layer's
    // output (row i: layer i's, written by block 0 of layer i+1's QKV launch,
    // or by the last tail). The layers share d, eps and the workspace
    // (layout(max over the layers)); layer i+1 reads layer i's o, h1, h2
    // from the workspace's first segments before it overwrites them.
    int encode_chain(void* stream, uint32_t n, const tfq_decode_layer_weights* w,
                     const tfq_decode_layer_shape* s, const uint16_t* hidden_in, uint16_t* hiddens,
                     uint16_t* const* k_caches, uint16_t* const* v_caches, uint32_t position, void* workspace,
                     size_t workspace_bytes) {
        if (n == 0 || !w || !s || !k_caches || !v_caches || !hidden_in || !hiddens)
            return fail(TFQ_E_INVAL, "null pointer argument or no layers");
        if (!aligned(hidden_in, 16) || !aligned(hiddens, 16))
            return fail(TFQ_E_INVAL, "hidden vectors and norm weights must be 16-byte aligned");
        size_t need = 0;
        for (uint32_t i = 0; i < n; ++i) {
            if (int rc = check_layer(w[i], s[i], k_caches[i], v_caches[i], workspace)) return rc;
            if (s[i].d != s[0].d || s[i].eps != s[0].eps)
                return fail(TFQ_E_INVAL, "chained layers must share d and eps (layer %u differs)", i);
            need = std::max(need, layout(s[i], position + 1).total);
        }
        if (workspace_bytes < need) return fail(TFQ_E_INVAL, "decode-layer workspace too small");
        char* ws = static_cast<char*>(workspace);
        const size_t d = s[0].d;
        for (uint32_t i = 0; i < n; ++i) {
            const Layout L = layout(s[i], position + 1);
            const uint16_t* hidden = i == 0 ? hidden_in : hiddens + (i - 1) * d;      // this layer's input
            NormArg stage{w[i].input_norm, nullptr, nullptr, s[i].eps, kStageNorm};
            const uint16_t* x = hidden;
            if (i > 0) {
                // the previous layer's tail, formed while staging: its input,
                // o, h1, h2 and norms; block 0 exports its output (= `hidden`)
                const tfq_decode_layer_weights& p = w[i - 1];
                x = i == 1 ? hidden_in : hiddens + (i - 2) * d;
                stage = NormArg{w[i].input_norm, reinterpret_cast<const uint16_t*>(ws + L.o), p.post_attention_norm,
                                s[i].eps, kStageTail, nullptr, hiddens + (i - 1) * d, nullptr,
                                reinterpret_cast<const uint16_t*>(ws + L.h1), p.post_ffn1_norm,
                                reinterpret_cast<const uint16_t*>(ws + L.h2), p.post_ffn2_norm, p.post_ffn_norm,
                                p.layer_scalar};
            }
            if (int rc = body(stream, w[i], s[i], x, stage, hidden, k_caches[i], v_caches[i], position, nullptr,
                              nullptr, ws, L))
                return rc;
        }
        const uint16_t* last_in = n == 1 ? hidden_in : hiddens + (n - 2) * d;
        return tail(stream, w[n - 1], s[n - 1], last_in, hiddens + (n - 1) * d, ws, layout(s[n - 1], position + 1));
    }

    static size_t chain_workspace_bytes(uint32_t n, const tfq_decode_layer_shape* s, uint32_t max_seq) {
        size_t need = 0;
        for (uint32_t i = 0; i < n; ++i) need = std::max(need, layout(s[i], max_seq).total);
        return need;
    }

    // Contract checks shared by encode and encode_chain.
    int check_layer(const tfq_decode_layer_weights& w, const tfq_decode_layer_shape& s, const uint16_t* k_cache,
                    const uint16_t* v_cache, const void* workspace) const {
        if (!k_cache || !v_cache || !workspace) return fail(TFQ_E_INVAL, "null pointer argument");
        if (!w.input_norm || !w.q_norm || !w.k_norm || !w.post_attention_norm || !w.pre_ffn_norm ||
            !w.pre_ffn2_norm || !w.post_ffn1_norm || !w.post_ffn2_norm || !w.post_ffn_norm)
            return fail(TFQ_E_INVAL, "every norm weight is required");
        if (s.d == 0 || s.d % 64 || s.d > 4096) return fail(TFQ_E_INVAL, "d=%u must be a multiple of 64 <= 4096", s.d);
        for (const void* p : {(const void*)w.input_norm, (const void*)w.post_attention_norm,
                              (const void*)w.pre_ffn_norm, (const void*)w.pre_ffn2_norm, (const void*)w.post_ffn1_norm,
                              (const void*)w.post_ffn2_norm, (const void*)w.post_ffn_norm})
            if (!aligned(p, 16)) return fail(TFQ_E_INVAL, "hidden vectors and norm weights must be 16-byte aligned");
        if (!aligned(workspace, 256)) return fail(TFQ_E_INVAL, "workspace must be 256-byte aligned");
        // shared expert width: Model.sharedExpertWeightBits (S/Runtime/Inference/Model.swift:59)
        const uint32_t shared_bits = w.shared_bits ? w.shared_bits : 4u;
        if (shared_bits != 4 && shared_bits != 8)
            return fail(TFQ_E_INVAL, "SharedExpert unsupported weight bits: %u", w.shared_bits);
        return TFQ_OK;
    }

    // Steps 1-6 of one layer (everything but the tail): the QKV GEMV stages
    // x as `qkv_stage` says (the input norm of `hidden`, or the previous
    // layer's tail followed by it); `hidden` is the layer's input, used by
    // the post-attention residual.
    int body(void* stream, const tfq_decode_layer_weights& w, const tfq_decode_layer_shape& s, const uint16_t* x,
             const NormArg& qkv_stage, const uint16_t* hidden, uint16_t* k_cache, uint16_t* v_cache,
             uint32_t position, uint32_t* out_indices, uint16_t* out_weights, char* ws, const Layout& L) {
        const uint32_t seq_len = position + 1;
        const uint32_t shared_bits = w.shared_bits ? w.shared_bits : 4u;
        uint16_t* q = reinterpret_cast<uint16_t*>(ws + L.q);
        uint16_t* attn = reinterpret_cast<uint16_t*>(ws + L.attn);
        uint16_t* o = reinterpret_cast<uint16_t*>(ws + L.o);
        float* logits = reinterpret_cast<float*>(ws + L.logits);
        uint32_t* idx = out_indices ? out_indices : reinterpret_cast<uint32_t*>(ws + L.idx);
        uint16_t* rw = out_weights ? out_weights : reinterpret_cast<uint16_t*>(ws + L.w);
        uint16_t* acts = reinterpret_cast<uint16_t*>(ws + L.acts);
        uint16_t* sact = reinterpret_cast<uint16_t*>(ws + L.sact);
        uint16_t* h1 = reinterpret_cast<uint16_t*>(ws + L.h1);
        uint16_t* h2 = reinterpret_cast<uint16_t*>(ws + L.h2);
        uint16_t* hmid = reinterpret_cast<uint16_t*>(ws + L.hmid);
        float* hinv = reinterpret_cast<float*>(ws + L.inv);
        const uint32_t qd = s.num_q_heads * s.head_dim, kvd = s.num_kv_heads * s.head_dim;
        const size_t slot = (size_t)position * kvd;

        // 1. input RMSNorm fused into the QKV GEMV; k and v land in the cache
        //    slot, or in the workspace when the attention blocks of a kv head
        //    all read them (head_dim 512 with group 8) or V is the k
        //    projection (v_proj absent: the full-attention layers,
        //    RealForwardRunner.swift:2252-2255, whose fused QKV runs k_proj as
        //    the v projection; one k GEMV serves both here)
        const bool v_from_k = w.v_proj.weights == nullptr;
        const bool staged = v_from_k || (s.head_dim == 512 && s.num_q_heads == 8 * s.num_kv_heads);
        uint16_t* kraw = staged ? reinterpret_cast<uint16_t*>(ws + L.kv) : k_cache + slot;
        uint16_t* vraw = !staged ? v_cache + slot : v_from_k ? kraw : kraw + kvd;
        int rc = v_from_k ? gemv_.encode_qk(stream, w.q_proj, w.k_proj, x, q, kraw, qd, kvd, s.d, qkv_stage)
                          : gemv_.encode_qkv(stream, w.q_proj, w.k_proj, w.v_proj, x, q, kraw, vraw, qd, kvd,
                                             s.d, qkv_stage);
        if (rc) return rc;
        // 2. q/k/v epilogue + attention
        const AttnEpilogue epi{w.q_norm, w.k_norm, s.eps, s.rope_theta, s.rotated_pairs, 0, 0.0,
                               staged ? kraw : nullptr, staged ? vraw : nullptr};
        rc = attn_.encode(stream, q, k_cache, v_cache, attn, s.head_dim, s.num_q_heads, s.num_kv_heads,
                          seq_len, s.window, s.attn_scale, epi, ws + L.parts, L.parts_bytes);
        if (rc) return rc;
        // 3. o projection
        rc = gemv_.encode(stream, w.o_proj.weights, w.o_proj.scales, w.o_proj.biases, attn, o, s.d, qd);
        if (rc) return rc;
        // 4. shared expert, input = pre_feedforward_layernorm(h): inside the
        //    routed launches (fused), or here from the layer input and o
        const bool fused = pool_bits(w.experts) == 4 && s.shared_f <= 4096;
        if (!fused) {
            const NormArg dense{w.pre_ffn_norm, o, w.post_attention_norm, s.eps, kStagePostAttn};
            rc = shared_bits == 8 ? shared8_.encode(stream, hidden, w.shared_gate, w.shared_up, w.shared_down, h1,
                                                    s.d, s.shared_f, sact, dense)
                                  : shared_.encode(stream, hidden, w.shared_gate, w.shared_up, w.shared_down, h1,
                                                   s.d, s.shared_f, sact, dense);
            if (rc) return rc;
        }
        // 5. router on the no-scale norm of h; its block 0 also stores h and
        //    r(h), so the expert launches form their inputs without the reductions
        const NormArg router_x{nullptr, o, w.post_attention_norm, s.eps, kStagePostAttn, nullptr, hmid, hinv};
        const tfq_router& r = w.router;
        float* logits_used = nullptr;
        rc = moe_.encode_router_logits(stream, r.weights, r.scales, r.biases, hidden, r.effective_scale,
                                       logits, r.num_experts, s.d, s.top_k, logits, router_x, &logits_used);
        if (rc) return rc;
        // 6. routed experts on pre_feedforward_layernorm_2(h), the top-k selected inside
        //    phase 1; phase 2 without residual
        const NormArg routed{w.pre_ffn2_norm, nullptr, nullptr, s.eps, kStageScaled, hinv, nullptr, nullptr};
        if (fused) {
            rc = moe_.encode_phase1_shared(stream, w.experts, logits, r.per_expert_scale, r.num_experts, idx, rw,
                                           hmid, acts, s.d, s.expert_f, s.top_k, routed, w.shared_gate,
                                           w.shared_up, w.pre_ffn_norm, sact, s.shared_f, shared_bits);
            if (rc) return rc;
            return moe_.encode_phase2_shared(stream, w.experts, idx, acts, rw, h2, s.d, s.expert_f, s.top_k,
                                             w.shared_down, sact, h1, s.shared_f, shared_bits);
        }
        rc = moe_.encode_phase1_routed(stream, w.experts, logits, r.per_expert_scale, r.num_experts, idx, rw,
                                       nullptr, hmid, acts, s.d, s.expert_f, s.top_k, routed);
        if (rc) return rc;
        return moe_.encode_phase2(stream, w.experts, idx, acts, rw, nullptr, h2, s.d, s.expert_f, s.top_k);
    }

    // 7. the tail kernel: out from the layer's input `hidden` and its o, h1, h2.
    int tail(void* stream, const tfq_decode_layer_weights& w, const tfq_decode_layer_shape& s,
             const uint16_t* hidden, uint16_t* out, char* ws, const Layout& L) {
        const uint16_t* o = reinterpret_cast<const uint16_t*>(ws + L.o);
        const uint16_t* h1 = reinterpret_cast<const uint16_t*>(ws + L.h1);
        const uint16_t* h2 = reinterpret_cast<const uint16_t*>(ws + L.h2);
        float eps = s.eps, scalar = w.layer_scalar;
        uint32_t d = s.d;
        void* ta[] = {(void*)&hidden, (void*)&o, (void*)&w.post_attention_norm, (void*)&h1, (void*)&w.post_ffn1_norm,
                      (void*)&h2, (void*)&w.post_ffn2_norm, (void*)&w.post_ffn_norm, &eps, &scalar, &out, &d};
        return launch2(m_, "tfq_layer_tail", 1, 1, 1024, 0, stream, ta);
    }

private:

    const Module& m_;
    DequantInt4GEMV& gemv_;
    MoE& moe_;
    SharedExpertInt4& shared_;
    SharedExpertInt8& shared8_;
    Attention& attn_;
};

}  // namespace tfq
