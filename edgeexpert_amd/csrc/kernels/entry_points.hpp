// entry_points.hpp — the macros that instantiate libtfq's kernel entry
// points, shared by the tfq_*.hip translation units.
//
// Each tfq_*.hip file is built by edgeexpert_amd/build.py into its own gfx950
// code object (edgeexpert_amd/lib/tfq_*.co, compiled in parallel) and loaded
// at run time with hipModuleLoad; entry points have C names so the host
// resolves them with hipModuleGetFunction across the loaded objects. Shapes
// are compile-time template parameters: SEG = lanes per output row (power of
// two, <= 64) and P = 16-byte chunks per lane; the host picks the
// instantiation from n.
#pragma once

#include "abi_types.h"
#include "attention.hpp"
#include "gemm.hpp"
#include "gemm_skinny.hpp"
#include "moe_decode.hpp"
#include "moe_prefill.hpp"

using namespace tfq;

// Rows each segment keeps in flight (loads issued before the previous rows
// are reduced): one; the next row's loads are issued while this row's partial
// sums are reduced and stored.
constexpr int kRowsInFlight = 1;

// Each int4 GEMV-family shape comes in three forms: plain (x staged as is),
// _rms (x RMS-normalised while staged) and _norm (x staged as NormArg says,
// any mode). The plain and _rms forms fix the staging mode at compile time
// and take only 16-byte aligned inputs of n <= 4096 (the host checks, and
// sends other calls to _norm); the plain form needs the fewest registers and
// so runs the most wavefronts per SIMD. The 2- and 3-bit forms of a kernel
// carry the width in the name (tfq_q3_gemv_*, tfq_moe_phase1_b3_*).
#define TFQ_GEMV_FORMS(TAG, BITS, SEG, P)                                                        \
    extern "C" __global__ __launch_bounds__(256) void tfq_##TAG##_gemv_s##SEG##_p##P(            \
        Q4Multi mats, const uint16_t* x, uint32_t n) {                                            \
        q4_gemv_multi<SEG, P, kRowsInFlight, false, BITS, false, kThreads, (int)kStageCopy>(mats, x, \
                                                                                            n);  \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(256) void tfq_##TAG##_gemv_rms_s##SEG##_p##P(        \
        Q4Multi mats, const uint16_t* x, uint32_t n) {                                            \
        q4_gemv_multi<SEG, P, kRowsInFlight, true, BITS, false, kThreads, (int)kStageNorm>(mats, x, \
                                                                                           n);   \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(256) void tfq_##TAG##_gemv_norm_s##SEG##_p##P(       \
        Q4Multi mats, const uint16_t* x, uint32_t n) {                                            \
        q4_gemv_multi<SEG, P, kRowsInFlight, true, BITS>(mats, x, n);                             \
    }
#define TFQ_Q4_GEMV(SEG, P) TFQ_GEMV_FORMS(q4, 4, SEG, P)
// The plain int4 GEMV for aligned x of 4096 < n <= 8192 (four staged chunks
// per thread; the full-attention layers' o projection, n = 16 heads x 512).
#define TFQ_Q4_GEMV_WIDE(SEG, P)                                                                 \
    extern "C" __global__ __launch_bounds__(256) void tfq_q4_gemv_wide_s##SEG##_p##P(            \
        Q4Multi mats, const uint16_t* x, uint32_t n) {                                            \
        q4_gemv_multi<SEG, P, kRowsInFlight, false, 4, false, kThreads, (int)kStageCopy, 4>(mats, x, n); \
    }
// The int4 GEMV staging the previous decoder layer's tail (kStageTail; the
// chained decode layers' fused QKV), 1024-thread blocks.
constexpr uint32_t kTailGemvThreads = 1024;
#define TFQ_Q4_GEMV_TAIL(SEG, P)                                                                 \
    extern "C" __global__ __launch_bounds__(kTailGemvThreads) void tfq_q4_gemv_tail_s##SEG##_p##P( \
        Q4Multi mats, const uint16_t* x, uint32_t n) {                                            \
        q4_gemv_multi<SEG, P, kRowsInFlight, true, 4, true, kTailGemvThreads>(mats, x, n);        \
    }
#define TFQ_Q3_GEMV(SEG, P) TFQ_GEMV_FORMS(q3, 3, SEG, P)

// _c_: x 16-byte aligned (every token's row), the copy staging fixed at compile time
#define TFQ_Q8_GEMV_FORM(NAME, FIXED, SEG, P)                                                    \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        const uint8_t* W, const uint16_t* S, const uint16_t* B, const uint16_t* x,               \
        uint32_t x_stride, uint16_t* y, uint32_t y_stride, uint32_t m, uint32_t n) {              \
        q8_gemv<SEG, P, kRowsInFlight, FIXED>(W, S, B, x, x_stride, y, y_stride, m, n, blockIdx.x, \
                                              gridDim.x);                                         \
    }
#define TFQ_Q8_GEMV(SEG, P)                                                                      \
    TFQ_Q8_GEMV_FORM(tfq_q8_gemv_s##SEG##_p##P, -1, SEG, P)                                      \
    TFQ_Q8_GEMV_FORM(tfq_q8_gemv_c_s##SEG##_p##P, (int)kStageCopy, SEG, P)

// Shared expert, int8 rows: fused gate/up/act in the plain and norm staging forms.
// _c_: x 16-byte aligned (every token's row): the copy staging fixed at compile time
#define TFQ_Q8_GATE_UP_FORM(NAME, NORM, FIXED, SEG, P)                                           \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        Q8Mat gate, Q8Mat up, const uint16_t* x, uint32_t x_stride, uint16_t* act, uint32_t D,   \
        uint32_t F, NormArg norm) {                                                               \
        q8_gate_up_act<SEG, P, kRowsInFlight, NORM, FIXED>(gate, up, x, x_stride, act, D, F, norm, \
                                                           blockIdx.x, gridDim.x);                \
    }
#define TFQ_Q8_GATE_UP(SEG, P)                                                                   \
    TFQ_Q8_GATE_UP_FORM(tfq_q8_gate_up_act_s##SEG##_p##P, false, -1, SEG, P)                     \
    TFQ_Q8_GATE_UP_FORM(tfq_q8_gate_up_act_norm_s##SEG##_p##P, true, -1, SEG, P)                 \
    TFQ_Q8_GATE_UP_FORM(tfq_q8_gate_up_act_c_s##SEG##_p##P, false, (int)kStageCopy, SEG, P)

// The router GEMV: any staging mode and alignment, and the copy (_c_) and
// post-attention (_pa_) modes fixed at compile time for aligned inputs.
#define TFQ_ROUTER_FORM(NAME, FIXED, SEG, P)                                                     \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        const uint8_t* W, const uint16_t* S, const uint16_t* B, const uint16_t* h,               \
        const uint16_t* eff, float* logits, uint32_t E, uint32_t d, NormArg norm) {              \
        router_logits<SEG, P, FIXED>(W, S, B, h, eff, logits, E, d, norm);                        \
    }
#define TFQ_ROUTER(SEG, P)                                                                       \
    TFQ_ROUTER_FORM(tfq_router_logits_s##SEG##_p##P, -1, SEG, P)                                 \
    TFQ_ROUTER_FORM(tfq_router_logits_c_s##SEG##_p##P, (int)kStageCopy, SEG, P)                  \
    TFQ_ROUTER_FORM(tfq_router_logits_pa_s##SEG##_p##P, (int)kStagePostAttn, SEG, P)

// GB: query heads per block (G / GB blocks per (chunk, kv head), blockIdx.z).
#define TFQ_ATTN_GB(HD, G, GB)                                                                   \
    extern "C" __global__ __launch_bounds__(kAttnThreads) void tfq_attn_partial_h##HD##_g##G(    \
        const uint16_t* q, uint16_t* kc, uint16_t* vc, uint32_t nkv, uint32_t seq_len,           \
        uint32_t kv_start, float scale, AttnEpilogue epi, float* part_o, float* part_ml) {        \
        attn_partial<HD, G, GB>(q, kc, vc, nkv, seq_len, kv_start, scale, epi, part_o, part_ml);  \
    }
#define TFQ_ATTN(HD, G) TFQ_ATTN_GB(HD, G, G)

#define TFQ_ATTN_COMBINE(HD)                                                                     \
    extern "C" __global__ __launch_bounds__(kAttnCombineThreads) void tfq_attn_combine_h##HD(    \
        const float* part_o, const float* part_ml, uint16_t* out, uint32_t nchunks) {             \
        attn_combine<HD>(part_o, part_ml, out, nchunks);                                          \
    }

// Prefill router: blockIdx.y selects the token (row stride `stride` halves).
#define TFQ_PREFILL_ROUTER(SEG, P)                                                               \
    extern "C" __global__ __launch_bounds__(256) void tfq_prefill_router_logits_s##SEG##_p##P(   \
        const uint8_t* W, const uint16_t* S, const uint16_t* B, const uint16_t* hidden,          \
        uint32_t stride, const uint16_t* eff, float* logits, uint32_t E, uint32_t d) {           \
        router_logits<SEG, P>(W, S, B, hidden + (size_t)blockIdx.y * stride, eff,               \
                              logits + (size_t)blockIdx.y * E, E, d);                            \
    }

#define TFQ_PHASE1_FORM(NAME, NORM, BITS, SEG, P)                                                \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        ExpertPool pool, const uint32_t* indices, const uint32_t* active_slots,                  \
        uint32_t n_active, uint32_t top_k, const uint16_t* x, uint16_t* acts, uint32_t D,        \
        uint32_t F, NormArg norm) {                                                               \
        moe_phase1<SEG, P, kRowsInFlight, NORM, BITS>(pool, indices, active_slots, n_active,     \
                                                      top_k, x, acts, D, F, norm);                \
    }
#define TFQ_PHASE1(SEG, P)                                                                       \
    TFQ_PHASE1_FORM(tfq_moe_phase1_s##SEG##_p##P, false, 4, SEG, P)                              \
    TFQ_PHASE1_FORM(tfq_moe_phase1_norm_s##SEG##_p##P, true, 4, SEG, P)
#define TFQ_PHASE1_B(SEG, P)                                                                     \
    TFQ_PHASE1_FORM(tfq_moe_phase1_b2_s##SEG##_p##P, false, 2, SEG, P)                           \
    TFQ_PHASE1_FORM(tfq_moe_phase1_b2_norm_s##SEG##_p##P, true, 2, SEG, P)                       \
    TFQ_PHASE1_FORM(tfq_moe_phase1_b3_s##SEG##_p##P, false, 3, SEG, P)                           \
    TFQ_PHASE1_FORM(tfq_moe_phase1_b3_norm_s##SEG##_p##P, true, 3, SEG, P)

#define TFQ_PHASE1_ROUTED_FORM(NAME, NORM, BITS, SEG, P)                                         \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        ExpertPool pool, const float* logits, const uint16_t* gain, uint32_t E, uint32_t top_k,  \
        uint32_t* out_idx, uint16_t* out_w, float* out_wf, const uint16_t* x, uint16_t* acts,    \
        uint32_t D, uint32_t F, NormArg norm) {                                                   \
        moe_phase1_routed<SEG, P, kRowsInFlight, NORM, BITS>(pool, logits, gain, E, top_k,       \
                                                             out_idx, out_w, out_wf, x, acts, D, \
                                                             F, norm, blockIdx.x, gridDim.x);     \
    }
#define TFQ_PHASE1_ROUTED(SEG, P)                                                                \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_s##SEG##_p##P, false, 4, SEG, P)                \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_norm_s##SEG##_p##P, true, 4, SEG, P)
#define TFQ_PHASE1_ROUTED_B(SEG, P)                                                              \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b2_s##SEG##_p##P, false, 2, SEG, P)             \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b2_norm_s##SEG##_p##P, true, 2, SEG, P)         \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b3_s##SEG##_p##P, false, 3, SEG, P)             \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b3_norm_s##SEG##_p##P, true, 3, SEG, P)

// Phase 2 stages the acts with the mode read at run time: the fixed-mode
// copy (exact waits, the staging overlapping the weight stream) measured
// 6.17 against 6.00 us per config-1 launch; the fused launches of the
// decoder layer fix it (faster there).
#define TFQ_PHASE2_FORM(NAME, BITS, P)                                                           \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        ExpertPool pool, const uint32_t* indices, const uint16_t* acts, const uint16_t* rw,      \
        const uint16_t* residual, uint16_t* y, uint32_t D, uint32_t F, uint32_t top_k) {         \
        moe_phase2<P, kRowsInFlight, BITS>(pool, indices, acts, rw, residual, y, D, F, top_k,     \
                                           blockIdx.x, gridDim.x);                                \
    }
#define TFQ_PHASE2(P)                                                                            \
    TFQ_PHASE2_FORM(tfq_moe_phase2_p##P, 4, P)                                                   \
    TFQ_PHASE2_FORM(tfq_moe_phase2_b2_p##P, 2, P)                                                \
    TFQ_PHASE2_FORM(tfq_moe_phase2_b3_p##P, 3, P)

#define TFQ_PHASE1_SHARED_FORM(NAME, BITS, SEG, P)                                               \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        ExpertPool pool, const float* logits, const uint16_t* gain, uint32_t E, uint32_t top_k,  \
        uint32_t* out_idx, uint16_t* out_w, float* out_wf, const uint16_t* x, uint16_t* acts,    \
        uint32_t D, uint32_t F, NormArg norm, Q4Mat sgate, Q4Mat sup, const uint16_t* snorm_w,   \
        uint16_t* sact, uint32_t Fs, uint32_t shared_blocks) {                                    \
        moe_phase1_routed_shared<SEG, P, kRowsInFlight, BITS>(pool, logits, gain, E, top_k,      \
                                                              out_idx, out_w, out_wf, x, acts,   \
                                                              D, F, norm, sgate, sup, snorm_w,   \
                                                              sact, Fs, shared_blocks);          \
    }
#define TFQ_PHASE1_SHARED(SEG, P) TFQ_PHASE1_SHARED_FORM(tfq_moe_phase1_shared_s##SEG##_p##P, 4, SEG, P)

#define TFQ_PHASE2_SHARED_FORM(NAME, BITS, P2, SP)                                               \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        ExpertPool pool, const uint32_t* indices, const uint16_t* acts, const uint16_t* rw,      \
        uint16_t* y, uint32_t D, uint32_t F, uint32_t top_k, Q4Mat sdown, const uint16_t* sact,  \
        uint16_t* sy, uint32_t Fs, uint32_t shared_blocks) {                                      \
        moe_phase2_shared<P2, SP, kRowsInFlight, BITS>(pool, indices, acts, rw, y, D, F, top_k,  \
                                                       sdown, sact, sy, Fs, shared_blocks);       \
    }
#define TFQ_PHASE2_SHARED_SP(P2, SP) TFQ_PHASE2_SHARED_FORM(tfq_moe_phase2_shared_p##P2##_sp##SP, 4, P2, SP)
#define TFQ_PHASE2_SHARED(P2)                                                                    \
    TFQ_PHASE2_SHARED_SP(P2, 1) TFQ_PHASE2_SHARED_SP(P2, 2) TFQ_PHASE2_SHARED_SP(P2, 3)          \
    TFQ_PHASE2_SHARED_SP(P2, 4)

// int8 shared expert: (SEG, P) of the routed rows (d/32 chunks) and (SEG8,
// P8) of the shared gate/up rows (d/16 chunks) are both set by d.
#define TFQ_PHASE1_SHARED8(SEG, P, SEG8, P8)                                                      \
    extern "C" __global__ __launch_bounds__(256) void                                             \
        tfq_moe_phase1_shared8_s##SEG##_p##P##_q##SEG8##_##P8(                                    \
            ExpertPool pool, const float* logits, const uint16_t* gain, uint32_t E, uint32_t top_k, \
            uint32_t* out_idx, uint16_t* out_w, float* out_wf, const uint16_t* x, uint16_t* acts,  \
            uint32_t D, uint32_t F, NormArg norm, Q8Mat sgate, Q8Mat sup, const uint16_t* snorm_w,  \
            uint16_t* sact, uint32_t Fs, uint32_t shared_blocks) {                                  \
        moe_phase1_routed_shared8<SEG, P, SEG8, P8, kRowsInFlight>(pool, logits, gain, E, top_k,  \
                                                                   out_idx, out_w, out_wf, x,     \
                                                                   acts, D, F, norm, sgate, sup,  \
                                                                   snorm_w, sact, Fs,             \
                                                                   shared_blocks);                \
    }
#define TFQ_PHASE2_SHARED8_FORM(P2, SEG8, P8)                                                     \
    extern "C" __global__ __launch_bounds__(256) void                                             \
        tfq_moe_phase2_shared8_p##P2##_q##SEG8##_##P8(                                            \
            ExpertPool pool, const uint32_t* indices, const uint16_t* acts, const uint16_t* rw,  \
            uint16_t* y, uint32_t D, uint32_t F, uint32_t top_k, Q8Mat sdown, const uint16_t* sact, \
            uint16_t* sy, uint32_t Fs, uint32_t shared_blocks) {                                    \
        moe_phase2_shared8<P2, SEG8, P8, kRowsInFlight>(pool, indices, acts, rw, y, D, F, top_k,  \
                                                        sdown, sact, sy, Fs, shared_blocks);      \
    }
#define TFQ_PHASE2_SHARED8_P1(SEG8, P8) TFQ_PHASE2_SHARED8_FORM(1, SEG8, P8)
#define TFQ_PHASE2_SHARED8_P2(SEG8, P8) TFQ_PHASE2_SHARED8_FORM(2, SEG8, P8)
#define TFQ_PHASE2_SHARED8_P3(SEG8, P8) TFQ_PHASE2_SHARED8_FORM(3, SEG8, P8)
#define TFQ_PHASE2_SHARED8_P4(SEG8, P8) TFQ_PHASE2_SHARED8_FORM(4, SEG8, P8)

#define TFQ_LM_HEAD_FORM(NAME, FIXED, SEG, P)                                                    \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        Q4Multi mats, const uint16_t* x, uint32_t n, uint64_t* summaries) {                      \
        lm_head_greedy_rows<SEG, P, kRowsInFlight, FIXED>(mats, x, n, summaries);                \
    }
#define TFQ_LM_HEAD(SEG, P)                                                                      \
    TFQ_LM_HEAD_FORM(tfq_lm_head_greedy_s##SEG##_p##P, -1, SEG, P)                               \
    TFQ_LM_HEAD_FORM(tfq_lm_head_greedy_rms_s##SEG##_p##P, (int)kStageNorm, SEG, P)

// _c_: x 16-byte aligned, D <= 4096: the copy staging fixed at compile time
#define TFQ_GATE_UP_FORM(NAME, NORM, FIXED, SEG, P)                                              \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        Q4Mat gate, Q4Mat up, const uint16_t* x, uint16_t* act, uint32_t D, uint32_t F,          \
        NormArg norm) {                                                                           \
        q4_gate_up_act<SEG, P, kRowsInFlight, NORM, FIXED>(gate, up, x, act, D, F, norm,         \
                                                           blockIdx.x, gridDim.x);                \
    }
#define TFQ_GATE_UP(SEG, P)                                                                      \
    TFQ_GATE_UP_FORM(tfq_gate_up_act_s##SEG##_p##P, false, -1, SEG, P)                           \
    TFQ_GATE_UP_FORM(tfq_gate_up_act_norm_s##SEG##_p##P, true, -1, SEG, P)                       \
    TFQ_GATE_UP_FORM(tfq_gate_up_act_c_s##SEG##_p##P, false, (int)kStageCopy, SEG, P)

// n/32 chunks (of 32 codes) per row at every code width; (SEG, P) with SEG·P >= chunks (the host picks
// the pair that wastes the fewest lanes).
#define TFQ_Q4_TABLE(X) X(2, 1) X(4, 1) X(8, 1) X(8, 2) X(8, 3) X(8, 4) X(16, 1) X(16, 2) X(16, 3) \
    X(16, 4) X(32, 1) X(32, 2) X(32, 3) X(32, 4) X(64, 1) X(64, 2) X(64, 3) X(64, 4)
// int8: n/16 chunks per row (n <= 4096).
#define TFQ_Q8_TABLE(X) X(4, 1) X(8, 1) X(16, 1) X(32, 1) X(64, 1) X(64, 2) X(64, 3) X(64, 4)
