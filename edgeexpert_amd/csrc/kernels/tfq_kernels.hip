// tfq_kernels.hip — gfx950 code object: every kernel entry point of libtfq.
//
// Built by edgeexpert_amd/build.py into edgeexpert_amd/lib/tfq_kernels.co and
// loaded at run time with hipModuleLoad; entry points have C names so the
// host resolves them with hipModuleGetFunction. Shapes are compile-time
// template parameters: SEG = lanes per output row (power of two, <= 64) and
// P = 16-byte chunks per lane; the host picks the instantiation from n.
#include "abi_types.h"
#include "attention.hpp"
#include "gemm.hpp"
#include "moe_decode.hpp"
#include "moe_prefill.hpp"

using namespace tfq;

// Rows each segment keeps in flight (loads issued before the previous rows are reduced).
#ifndef TFQ_ROWS_IN_FLIGHT
#define TFQ_ROWS_IN_FLIGHT 1
#endif
constexpr int kRowsInFlight = TFQ_ROWS_IN_FLIGHT;

// Each int4 GEMV-family shape comes in two forms: plain (x staged as is) and
// _norm (x normalised while staged, NormArg); the plain form needs fewer
// registers and so runs more wavefronts per SIMD. The 2- and 3-bit forms of
// a kernel carry the width in the name (tfq_q3_gemv_*, tfq_moe_phase1_b3_*).
#define TFQ_GEMV_FORMS(TAG, BITS, SEG, P)                                                        \
    extern "C" __global__ __launch_bounds__(256) void tfq_##TAG##_gemv_s##SEG##_p##P(            \
        Q4Multi mats, const uint16_t* x, uint32_t n) {                                            \
        q4_gemv_multi<SEG, P, kRowsInFlight, false, BITS>(mats, x, n);                            \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(256) void tfq_##TAG##_gemv_norm_s##SEG##_p##P(       \
        Q4Multi mats, const uint16_t* x, uint32_t n) {                                            \
        q4_gemv_multi<SEG, P, kRowsInFlight, true, BITS>(mats, x, n);                             \
    }
#define TFQ_Q4_GEMV(SEG, P) TFQ_GEMV_FORMS(q4, 4, SEG, P)
#define TFQ_Q3_GEMV(SEG, P) TFQ_GEMV_FORMS(q3, 3, SEG, P)

#define TFQ_Q8_GEMV(SEG, P)                                                                      \
    extern "C" __global__ __launch_bounds__(256) void tfq_q8_gemv_s##SEG##_p##P(                 \
        const uint8_t* W, const uint16_t* S, const uint16_t* B, const uint16_t* x, uint16_t* y,  \
        uint32_t m, uint32_t n) {                                                                 \
        q8_gemv<SEG, P, kRowsInFlight>(W, S, B, x, y, m, n);                                      \
    }

#define TFQ_ROUTER(SEG, P)                                                                       \
    extern "C" __global__ __launch_bounds__(256) void tfq_router_logits_s##SEG##_p##P(           \
        const uint8_t* W, const uint16_t* S, const uint16_t* B, const uint16_t* h,               \
        const uint16_t* eff, float* logits, uint32_t E, uint32_t d, NormArg norm) {              \
        router_logits<SEG, P>(W, S, B, h, eff, logits, E, d, norm);                               \
    }

#define TFQ_ATTN(HD, G)                                                                          \
    extern "C" __global__ __launch_bounds__(kAttnThreads) void tfq_attn_partial_h##HD##_g##G(    \
        const uint16_t* q, uint16_t* kc, uint16_t* vc, uint32_t nkv, uint32_t seq_len,           \
        uint32_t kv_start, float scale, AttnEpilogue epi, float* part_o, float* part_ml) {        \
        attn_partial<HD, G>(q, kc, vc, nkv, seq_len, kv_start, scale, epi, part_o, part_ml);      \
    }

#define TFQ_ATTN_COMBINE(HD)                                                                     \
    extern "C" __global__ __launch_bounds__(HD) void tfq_attn_combine_h##HD(                     \
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
                                                             F, norm);                            \
    }
#define TFQ_PHASE1_ROUTED(SEG, P)                                                                \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_s##SEG##_p##P, false, 4, SEG, P)                \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_norm_s##SEG##_p##P, true, 4, SEG, P)
#define TFQ_PHASE1_ROUTED_B(SEG, P)                                                              \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b2_s##SEG##_p##P, false, 2, SEG, P)             \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b2_norm_s##SEG##_p##P, true, 2, SEG, P)         \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b3_s##SEG##_p##P, false, 3, SEG, P)             \
    TFQ_PHASE1_ROUTED_FORM(tfq_moe_phase1_routed_b3_norm_s##SEG##_p##P, true, 3, SEG, P)

#define TFQ_PHASE2_FORM(NAME, BITS, P)                                                           \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        ExpertPool pool, const uint32_t* indices, const uint16_t* acts, const uint16_t* rw,      \
        const uint16_t* residual, uint16_t* y, uint32_t D, uint32_t F, uint32_t top_k) {         \
        moe_phase2<P, kRowsInFlight, BITS>(pool, indices, acts, rw, residual, y, D, F, top_k);    \
    }
#define TFQ_PHASE2(P)                                                                            \
    TFQ_PHASE2_FORM(tfq_moe_phase2_p##P, 4, P)                                                   \
    TFQ_PHASE2_FORM(tfq_moe_phase2_b2_p##P, 2, P)                                                \
    TFQ_PHASE2_FORM(tfq_moe_phase2_b3_p##P, 3, P)

#define TFQ_LM_HEAD(SEG, P)                                                                      \
    extern "C" __global__ __launch_bounds__(256) void tfq_lm_head_greedy_s##SEG##_p##P(          \
        Q4Multi mats, const uint16_t* x, uint32_t n, uint64_t* summaries) {                      \
        lm_head_greedy_rows<SEG, P, kRowsInFlight>(mats, x, n, summaries);                       \
    }

#define TFQ_GATE_UP_FORM(NAME, NORM, SEG, P)                                                     \
    extern "C" __global__ __launch_bounds__(256) void NAME(                                       \
        Q4Mat gate, Q4Mat up, const uint16_t* x, uint16_t* act, uint32_t D, uint32_t F,          \
        NormArg norm) {                                                                           \
        q4_gate_up_act<SEG, P, kRowsInFlight, NORM>(gate, up, x, act, D, F, norm);                \
    }
#define TFQ_GATE_UP(SEG, P)                                                                      \
    TFQ_GATE_UP_FORM(tfq_gate_up_act_s##SEG##_p##P, false, SEG, P)                               \
    TFQ_GATE_UP_FORM(tfq_gate_up_act_norm_s##SEG##_p##P, true, SEG, P)

// n/32 chunks (of 32 codes) per row at every code width; (SEG, P) with SEG·P >= chunks (the host picks
// the pair that wastes the fewest lanes).
#define TFQ_Q4_TABLE(X) X(2, 1) X(4, 1) X(8, 1) X(8, 2) X(8, 3) X(8, 4) X(16, 1) X(16, 2) X(16, 3) \
    X(16, 4) X(32, 1) X(32, 2) X(32, 3) X(32, 4) X(64, 1) X(64, 2) X(64, 3) X(64, 4)
// int8: n/16 chunks per row (n <= 4096).
#define TFQ_Q8_TABLE(X) X(4, 1) X(8, 1) X(16, 1) X(32, 1) X(64, 1) X(64, 2) X(64, 3) X(64, 4)

TFQ_Q4_TABLE(TFQ_Q4_GEMV)
TFQ_Q4_TABLE(TFQ_Q3_GEMV)
TFQ_Q4_TABLE(TFQ_PHASE1)
TFQ_Q4_TABLE(TFQ_PHASE1_B)
TFQ_Q4_TABLE(TFQ_PHASE1_ROUTED)
TFQ_Q4_TABLE(TFQ_PHASE1_ROUTED_B)
TFQ_Q4_TABLE(TFQ_GATE_UP)
TFQ_Q4_TABLE(TFQ_LM_HEAD)
TFQ_Q8_TABLE(TFQ_Q8_GEMV)
TFQ_Q8_TABLE(TFQ_ROUTER)
TFQ_Q8_TABLE(TFQ_PREFILL_ROUTER)
TFQ_ATTN(128, 1)
TFQ_ATTN(128, 2)
TFQ_ATTN(128, 4)
TFQ_ATTN(256, 1)
TFQ_ATTN(256, 2)
TFQ_ATTN(256, 4)
TFQ_ATTN_COMBINE(128)
TFQ_ATTN_COMBINE(256)
TFQ_PHASE2(1)
TFQ_PHASE2(2)
TFQ_PHASE2(3)
TFQ_PHASE2(4)

#define TFQ_GEMM(TAG, BITS, DT, X_BF16)                                                          \
    extern "C" __global__ __launch_bounds__(kProjGemmThreads) void tfq_gemm_##TAG##_##DT(        \
        const uint16_t* X, const uint8_t* W, const uint16_t* S, const uint16_t* B, uint16_t* Y,  \
        uint32_t M, uint32_t N, uint32_t K) {                                                     \
        gemm_q4_proj<X_BF16, BITS>(X, W, S, B, Y, M, N, K);                                       \
    }
TFQ_GEMM(q4, 4, f16, false)
TFQ_GEMM(q4, 4, bf16, true)
TFQ_GEMM(q3, 3, f16, false)
TFQ_GEMM(q3, 3, bf16, true)

extern "C" __global__ __launch_bounds__(256) void tfq_lm_head_reduce(const uint64_t* summaries, uint32_t n,
                                                                     uint32_t* out_token) {
    lm_head_greedy_reduce(summaries, n, out_token);
}

extern "C" __global__ __launch_bounds__(256) void tfq_router_select(const float* logits,
                                                                    const uint16_t* gain,
                                                                    uint32_t* out_idx,
                                                                    uint16_t* out_w,
                                                                    float* out_wf, uint32_t E,
                                                                    uint32_t k) {
    router_select(logits, gain, out_idx, out_w, out_wf, E, k);
}

// Per-token selection for a prefill chunk: one block per token.
extern "C" __global__ __launch_bounds__(256) void tfq_prefill_select(const float* logits,
                                                                     const uint16_t* gain,
                                                                     uint32_t* out_idx,
                                                                     uint16_t* out_w,
                                                                     float* out_wf, uint32_t E,
                                                                     uint32_t k) {
    const size_t t = blockIdx.x;
    router_select(logits + t * E, gain, out_idx + t * k, out_w + t * k, out_wf ? out_wf + t * k : nullptr,
                  E, k);
}

extern "C" __global__ __launch_bounds__(kGroupThreads) void tfq_moe_group(
    const uint32_t* idx, const uint16_t* w, uint32_t T, uint32_t k, uint32_t E, Pair* sorted,
    uint32_t* offsets, uint32_t* counts, Tile* tiles, uint32_t* n_tiles, uint32_t* status) {
    moe_group(idx, w, T, k, E, sorted, offsets, counts, tiles, n_tiles, status);
}

#define TFQ_GROUPED(SUFFIX, BITS)                                                                \
    extern "C" __global__ __launch_bounds__(kProjThreads, 2) void tfq_moe_grouped_gate_up##SUFFIX( \
        ExpertPool pool, const Pair* sorted, const Tile* tiles, const uint32_t* n_tiles,         \
        const uint16_t* hidden, uint32_t stride, uint16_t* act, uint32_t D, uint32_t F) {        \
        moe_grouped_gate_up<BITS>(pool, sorted, tiles, n_tiles, hidden, stride, act, D, F);      \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(kProjThreads, 2) void tfq_moe_grouped_down##SUFFIX(  \
        ExpertPool pool, const Pair* sorted, const Tile* tiles, const uint32_t* n_tiles,         \
        const uint16_t* act, uint16_t* partials, uint32_t D, uint32_t F, uint32_t k) {           \
        moe_grouped_down<BITS>(pool, sorted, tiles, n_tiles, act, partials, D, F, k);            \
    }
TFQ_GROUPED(, 4)
TFQ_GROUPED(_b2, 2)
TFQ_GROUPED(_b3, 3)

extern "C" __global__ __launch_bounds__(256) void tfq_moe_combine(const uint16_t* partials,
                                                                  const uint16_t* w, uint16_t* h2,
                                                                  uint32_t T, uint32_t k, uint32_t D) {
    moe_combine(partials, w, h2, T, k, D);
}

extern "C" __global__ __launch_bounds__(256) void tfq_read_ceiling(const uint4* src, uint64_t n16,
                                                                     uint32_t* sink) {
    read_ceiling<4>(src, n16, sink);
}

extern "C" __global__ __launch_bounds__(256) void tfq_convert_bf16_f16(const uint16_t* src,
                                                                         uint16_t* dst, uint64_t n,
                                                                         uint32_t* inexact) {
    convert_bf16_to_f16(src, dst, n, inexact);
}

extern "C" __global__ __launch_bounds__(kLayerTailThreads) void tfq_layer_tail(
    const uint16_t* hidden, const uint16_t* attn, const uint16_t* w_post_attn, const uint16_t* h1,
    const uint16_t* w_sp, const uint16_t* h2, const uint16_t* w_pf2, const uint16_t* w_pf, float eps,
    float layer_scalar, uint16_t* out, uint32_t D) {
    layer_tail(hidden, attn, w_post_attn, h1, w_sp, h2, w_pf2, w_pf, eps, layer_scalar, out, D);
}
