// moe_decode.hpp — routed top-k MoE decode block and the int4 shared expert.
//
// The routed experts of a layer live in one HBM pool: expert e's blob is
// pool + e*stride, holding [gateW gateS gateB upW upS upB downW downS downB]
// at fixed offsets (S/Kernels/MoE/MoE.swift:4-29). The kernels read the
// router's index buffer and form the blob address on the device; there is no
// host round trip between routing and the expert GEMVs.
//
// Phase 1 (S/Metal/MoE/moe.metal:248-369): one segment per (slot, f) row;
//   gate and up rows share the activation registers;
//   acts[slot][f] = fp16(gelu(g)·u), g and u accumulated in fp32.
// Phase 2 (moe.metal:189-244,475-511): one wavefront per output d; its eight
//   8-lane segments each own one slot's down row d, so the eight expert dot
//   products finish inside one wave and lane 0 adds
//   residual + Σ_slot w[slot]·dot[slot] in fixed slot order.
// Both start with the loads that nothing depends on (activations, expert
// indices, routing weights), issue the weight loads as soon as the indices
// are in, and stage the activations into LDS while the weights arrive.
// Every phase is templated on the experts' code width (BITS = 4, or the
// 2/3-bit variants of moe.metal:644-1180); only the chunk load and unpack
// differ (common.hpp QChunk / dot_chunk).
#pragma once

#include "gemv.hpp"

namespace tfq {

// Pointers of one (gate row, up row) pair; valid == false poisons the output.
struct GateUpRow {
    const uint8_t* gw;
    const uint16_t* gs;
    const uint16_t* gb;
    const uint8_t* uw;
    const uint16_t* us;
    const uint16_t* ub;
    bool live;     // the row exists (writes an output)
    bool valid;    // its expert index is in range (else the output is NaN)
};

// Streams gate/up row pairs of length D against x (fp16, staged to LDS):
// `rowfn(row)` -> GateUpRow, `out(row, act)` for live rows (lane 0 of the
// segment). `prologue()` runs after the x loads are issued and before the
// first weight loads (routing: it makes rowfn's expert indices available).
// NORM == false: x is staged as is (norm ignored). BITS: code width of the
// rows (2, 3 or 4). Gate and up stay in fp32 up to the activation, as in
// moe.metal:368 and in the CPU references of every form. X_FIRST: the
// prologue waits for loads issued after x (expert indices, logits), so x has
// arrived when it ends; staging it before the weight loads then keeps the
// staging off the stall a wave takes while the memory pipeline backs up
// under them. blk / nblk: this block's index among the blocks that share
// the rows, and their count (q4_rows). FIXED: the staging mode when known at
// compile time (XStage), else -1.
template <int SEG, int P, int R, bool NORM, int BITS, bool X_FIRST, int FIXED, typename Pro, typename RowFn,
          typename OutFn>
__device__ __forceinline__ void gate_up_rows(const uint16_t* __restrict__ x, uint32_t D, uint32_t total,
                                             const NormArg& norm, Pro prologue, RowFn rowfn, OutFn out,
                                             uint32_t blk, uint32_t nblk) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_xh[];
    constexpr uint32_t NT = kThreads;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    constexpr uint32_t nwaves = NT / 64;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = D >> 5;
    constexpr uint32_t spw = kWave / SEG;
    const uint32_t seg_id = (blk * nwaves + wave) * spw + lane / SEG;
    const uint32_t seg_total = nblk * nwaves * spw;

    // Two row groups in flight per wave (buffers A and B alternate): the next
    // group's loads are issued before the current group's dot. Every issue is
    // unconditional (rows past the end re-read the last row, chunks past the
    // row its last chunk, dead or invalid rows expert 0's; none is stored),
    // so each wait covers exactly the group it consumes, and the wave-uniform
    // group count ends the loop without a branch around any load.
    struct Buf {
        QChunk<BITS> gv[R][P], uv[R][P];
        uint32_t gs[R][P], gb[R][P], us[R][P], ub[R][P];    // raw fp16 scales / biases
    };
    Buf A, B;
    auto issue = [&](uint32_t grp, Buf& f) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row0 = seg_id + (grp * R + r) * seg_total;
            const GateUpRow q = rowfn(row0 < total ? row0 : total - 1);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c0 = sl + p * SEG;
                const uint32_t c = c0 < lpr ? c0 : lpr - 1;
                f.gv[r][p] = ldg_chunk<BITS>(q.gw, c);
                f.uv[r][p] = ldg_chunk<BITS>(q.uw, c);
                f.gs[r][p] = q.gs[c >> 1];
                f.gb[r][p] = q.gb[c >> 1];
                f.us[r][p] = q.us[c >> 1];
                f.ub[r][p] = q.ub[c >> 1];
            }
        }
    };
    auto consume = [&](uint32_t grp, const Buf& f, const XPairs& xp) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float ga = 0.0f, ua = 0.0f;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c = sl + p * SEG;
                if (c < lpr) {
                    XChunk xc;
                    read_xpairs(xp, c, xc);
                    const float gd = dot_chunk<BITS>(f.gv[r][p], xc);
                    const float ud = dot_chunk<BITS>(f.uv[r][p], xc);
                    ga = fmaf(h2f((uint16_t)f.gs[r][p]), gd, ga);
                    ga = fmaf(h2f((uint16_t)f.gb[r][p]), xc.sum, ga);
                    ua = fmaf(h2f((uint16_t)f.us[r][p]), ud, ua);
                    ua = fmaf(h2f((uint16_t)f.ub[r][p]), xc.sum, ua);
                }
            }
            const float g = seg_sum<SEG>(ga);
            const float u = seg_sum<SEG>(ua);
            const uint32_t row = seg_id + (grp * R + r) * seg_total;
            if (row < total && sl == 0) {
                const GateUpRow q = rowfn(row);
                if (q.live) out(row, q.valid ? gelu_tanh(g) * u : __builtin_nanf(""));
            }
        }
    };
    XStage<NT, kStageChunks, NORM, true, false, FIXED> xs;
    xs.load(x, D, norm);
    // groups of the wave's first segment (the most of its segments)
    const uint32_t seg0 = (blk * nwaves + wave) * spw;
    const uint32_t ng = __builtin_amdgcn_readfirstlane(
        seg0 < total ? (total - seg0 + R * seg_total - 1) / (R * seg_total) : 0u);   // wave-uniform
    prologue();
    XPairs xp;
    if constexpr (X_FIRST) xp = xs.pairs(x, lds_xh, D, norm);
    issue(0, A);
    if constexpr (!X_FIRST) xp = xs.pairs(x, lds_xh, D, norm);
    uint32_t grp = 0;
    for (; grp + 1 < ng; grp += 2) {
        issue(grp + 1, B);
        consume(grp, A, xp);
        issue(grp + 2, A);      // past the last group: the last row, not stored
        consume(grp + 1, B, xp);
    }
    if (grp < ng) consume(grp, A, xp);
}

// Row `row` of phase 1 given the slot it belongs to and that slot's expert.
template <int BITS>
__device__ __forceinline__ GateUpRow expert_gate_up_row(const ExpertPool& pool, uint32_t slot, uint32_t e,
                                                        uint32_t f, uint32_t top_k, uint32_t D) {
    const uint32_t row_bytes = (D >> 3) * BITS;
    const uint32_t ngroups = D >> 6;
    GateUpRow q{};
    q.live = slot < top_k;                          // moe.metal:387 semantics
    q.valid = q.live && e < pool.num_experts;
    const uint8_t* blob = pool.base + (uint64_t)(q.valid ? e : 0u) * pool.stride;
    const ExpertOffsets& o = pool.off;
    q.gw = blob + o.gate_w + (size_t)f * row_bytes;
    q.gs = reinterpret_cast<const uint16_t*>(blob + o.gate_s) + (size_t)f * ngroups;
    q.gb = reinterpret_cast<const uint16_t*>(blob + o.gate_b) + (size_t)f * ngroups;
    q.uw = blob + o.up_w + (size_t)f * row_bytes;
    q.us = reinterpret_cast<const uint16_t*>(blob + o.up_s) + (size_t)f * ngroups;
    q.ub = reinterpret_cast<const uint16_t*>(blob + o.up_b) + (size_t)f * ngroups;
    return q;
}

// Phase 1 over n_active slots (active_slots == nullptr: slots 0..n_active-1).
// The (slot, expert) of every active index is read once per block into LDS
// (n_active <= kRouterMaxTopK, checked by the host).
template <int SEG, int P, int R, bool NORM, int BITS = 4>
__device__ __forceinline__ void moe_phase1(const ExpertPool& pool, const uint32_t* __restrict__ indices,
                                           const uint32_t* __restrict__ active_slots, uint32_t n_active,
                                           uint32_t top_k, const uint16_t* __restrict__ x,
                                           uint16_t* __restrict__ acts, uint32_t D, uint32_t F,
                                           const NormArg& norm) {
    __shared__ uint32_t act_slot[kRouterMaxTopK];
    __shared__ uint32_t act_expert[kRouterMaxTopK];
    gate_up_rows<SEG, P, R, NORM, BITS, true, -1>(
        x, D, n_active * F, norm,
        [&]() {
            if (threadIdx.x < n_active) {
                const uint32_t slot = active_slots ? active_slots[threadIdx.x] : threadIdx.x;
                act_slot[threadIdx.x] = slot;
                act_expert[threadIdx.x] = slot < top_k ? indices[slot] : 0u;
            }
            __syncthreads();
        },
        [&](uint32_t row) {
            const uint32_t a = row / F;
            return expert_gate_up_row<BITS>(pool, act_slot[a], act_expert[a], row % F, top_k, D);
        },
        [&](uint32_t row, float act) { acts[(size_t)act_slot[row / F] * F + row % F] = f2h(act); },
        blockIdx.x, gridDim.x);
}

// Phase 1 with the router's selection folded in: every block selects the
// top-k experts from the logits itself (block_topk, identical bits in every
// block), so routing costs no launch of its own between the router GEMV and
// the experts. Block 0 publishes indices and fp16 / fp32 weights for
// phase 2 and the caller (MoE.encodeRouterGemma4's outputs,
// S/Kernels/MoE/MoE.swift:147-197). blk / nblk as in gate_up_rows (blk 0
// publishes).
template <int SEG, int P, int R, bool NORM, int BITS = 4, int FIXED = -1>
__device__ __forceinline__ void moe_phase1_routed(const ExpertPool& pool, const float* __restrict__ logits,
                                                  const uint16_t* __restrict__ gain, uint32_t E, uint32_t top_k,
                                                  uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w,
                                                  float* __restrict__ out_wf, const uint16_t* __restrict__ x,
                                                  uint16_t* __restrict__ acts, uint32_t D, uint32_t F,
                                                  const NormArg& norm, uint32_t blk, uint32_t nblk) {
    __shared__ __attribute__((aligned(16))) float stage[kRouterMaxExperts];
    __shared__ uint32_t sel_idx[kRouterMaxTopK];
    __shared__ float sel_val[kRouterMaxTopK];
    gate_up_rows<SEG, P, R, NORM, BITS, true, FIXED>(
        x, D, top_k * F, norm,
        [&]() {
            for (uint32_t e = threadIdx.x; e < ((E + 3) & ~3u); e += kThreads)
                stage[e] = e < E ? logits[e] : -__builtin_inff();
            __syncthreads();
            block_topk(stage, E, top_k, sel_idx, sel_val);
            // phase 1 needs only the indices; the routing weights (for
            // phase 2) are formed by block 0 alone
            if (blk == 0) {
                __shared__ float ex[kRouterMaxTopK];
                __shared__ float sel_w[kRouterMaxTopK];
                block_softmax_gain(sel_idx, sel_val, top_k, gain, ex, sel_w);
                for (uint32_t r = threadIdx.x; r < top_k; r += kThreads) {
                    out_idx[r] = sel_idx[r];
                    out_w[r] = f2h(sel_w[r]);
                    if (out_wf) out_wf[r] = sel_w[r];
                }
            }
        },
        [&](uint32_t row) {
            return expert_gate_up_row<BITS>(pool, row / F, sel_idx[row / F], row % F, top_k, D);
        },
        [&](uint32_t row, float act) { acts[(size_t)(row / F) * F + row % F] = f2h(act); }, blk, nblk);
}

// Shared-expert gate/up/act, int4 rows: act[i] = fp16(gelu(g)·u), g =
// gate[i]·x and u = up[i]·x in fp32 (SharedExpertInt4.swift:30-94 computes
// the same product; its GPU sequence stores g and u as fp16 first, which
// moves the expert's output ~8e-4 from the CPU reference, so they stay fp32).
template <int SEG, int P, int R, bool NORM, int FIXED = -1>
__device__ __forceinline__ void q4_gate_up_act(const Q4Mat& gate, const Q4Mat& up,
                                               const uint16_t* __restrict__ x, uint16_t* __restrict__ act,
                                               uint32_t D, uint32_t F, const NormArg& norm, uint32_t blk,
                                               uint32_t nblk) {
    const uint32_t row_bytes = D >> 1;
    const uint32_t ngroups = D >> 6;
    gate_up_rows<SEG, P, R, NORM, 4, false, FIXED>(
        x, D, F, norm, [] {},
        [&](uint32_t f) {
            GateUpRow q{};
            q.live = true;
            q.valid = true;
            q.gw = gate.w + (size_t)f * row_bytes;
            q.gs = gate.s + (size_t)f * ngroups;
            q.gb = gate.b + (size_t)f * ngroups;
            q.uw = up.w + (size_t)f * row_bytes;
            q.us = up.s + (size_t)f * ngroups;
            q.ub = up.b + (size_t)f * ngroups;
            return q;
        },
        [&](uint32_t f, float a) { act[f] = f2h(a); }, blk, nblk);
}

// Shared-expert gate/up/act, int8 rows (shared_int8_gate_up_act_simd,
// S/Metal/Quant/dequant_int8.metal:99-154): act[i] = fp16(gelu(g)·u) with
// g, u the fp32 dot products of gate/up row i with x (the reference kernel
// rounds g and u to fp16 first, :150-152, which moves the expert's output
// ~4e-4 from its CPU reference; here they stay fp32). Rows of D bytes,
// 16 codes per lane-chunk (q8_rows' mapping); x is staged as NormArg says
// and held as fp32 in LDS, each lane keeping its chunks' activations in
// registers across rows. blockIdx.y selects the token of a prefill block
// (x + y·x_stride, act + y·F). Dynamic LDS: D floats + D halves. blk / nblk
// as in gate_up_rows.
template <int SEG, int P, int R, bool NORM, int FIXED = -1>
__device__ __forceinline__ void q8_gate_up_act(const Q8Mat& gate, const Q8Mat& up, const uint16_t* __restrict__ x,
                                               uint32_t x_stride, uint16_t* __restrict__ act, uint32_t D,
                                               uint32_t F, const NormArg& norm, uint32_t blk, uint32_t nblk) {
    extern __shared__ __attribute__((aligned(16))) float lds_x[];
    constexpr uint32_t NT = kThreads;
    x += (size_t)blockIdx.y * x_stride;
    act += (size_t)blockIdx.y * F;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    constexpr uint32_t nwaves = NT / 64;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = D >> 4;              // 16-code chunks per row
    const uint32_t ngroups = D >> 6;
    constexpr uint32_t spw = kWave / SEG;
    const uint32_t seg_id = (blk * nwaves + wave) * spw + lane / SEG;
    const uint32_t seg_total = nblk * nwaves * spw;

    uint4 gv[R][P], uv[R][P];
    uint32_t gsr[R][P], gbr[R][P], usr[R][P], ubr[R][P];     // raw fp16 scales / biases
    auto issue = [&](uint32_t grp, auto first_c) {      // first group unconditional, as in gate_up_rows
        constexpr bool FIRST = decltype(first_c)::value;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row0 = seg_id + (grp * R + r) * seg_total;
            const uint32_t row = FIRST && row0 >= F ? F - 1 : row0;
            if (FIRST || row < F) {
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c0 = sl + p * SEG;
                    const uint32_t c = FIRST && c0 >= lpr ? lpr - 1 : c0;
                    if (FIRST || c < lpr) {
                        gv[r][p] = ldg16_stream(gate.w + (size_t)row * D + 16u * c);
                        uv[r][p] = ldg16_stream(up.w + (size_t)row * D + 16u * c);
                        gsr[r][p] = gate.s[(size_t)row * ngroups + (c >> 2)];
                        gbr[r][p] = gate.b[(size_t)row * ngroups + (c >> 2)];
                        usr[r][p] = up.s[(size_t)row * ngroups + (c >> 2)];
                        ubr[r][p] = up.b[(size_t)row * ngroups + (c >> 2)];
                    }
                }
            }
        }
    };
    {
        uint16_t* hs = reinterpret_cast<uint16_t*>(lds_x + D);
        XStage<NT, kStageChunks, NORM, true, false, FIXED> st;
        st.load(x, D, norm);
        issue(0, std::true_type{});
        if (st.vec) {
            // the staged chunks (after the NormArg transform) widened straight
            // into the fp32 vector (clamped and unconditional like the loads)
            st.transform(D, norm);
#pragma unroll
            for (uint32_t i = 0; i < kStageChunks; ++i) {
                const uint32_t c0 = threadIdx.x + i * NT;
                const uint32_t c = c0 < (D >> 3) ? c0 : (D >> 3) - 1;
#pragma unroll
                for (int e = 0; e < 8; ++e) lds_x[8 * c + e] = (float)st.xv[i][e];
            }
        } else {
            st.plain(x, hs, D, norm);
            for (uint32_t i = threadIdx.x; i < D; i += NT) lds_x[i] = h2f(hs[i]);
        }
        __syncthreads();
    }
    float xr[P][16];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_x16(lds_x, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }
    for (uint32_t grp = 0; seg_id + grp * R * seg_total < F; ++grp) {
        float ga[R], ua[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            ga[r] = 0.0f;
            ua[r] = 0.0f;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c = sl + p * SEG;
                if (c < lpr) {
                    const float gd = dot16_q8(gv[r][p], xr[p]);
                    const float ud = dot16_q8(uv[r][p], xr[p]);
                    ga[r] = fmaf(h2f((uint16_t)gsr[r][p]), gd, ga[r]);
                    ga[r] = fmaf(h2f((uint16_t)gbr[r][p]), xs[p], ga[r]);
                    ua[r] = fmaf(h2f((uint16_t)usr[r][p]), ud, ua[r]);
                    ua[r] = fmaf(h2f((uint16_t)ubr[r][p]), xs[p], ua[r]);
                }
            }
        }
        issue(grp + 1, std::false_type{});
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float g = seg_sum<SEG>(ga[r]);
            const float u = seg_sum<SEG>(ua[r]);
            const uint32_t row = seg_id + (grp * R + r) * seg_total;
            if (sl == 0 && row < F) act[row] = f2h(gelu_tanh(g) * u);
        }
    }
}

// act[t][i] = fp16(gelu(g[t][i])·u[t][i]) over fp16 g and u (gelu_mul_fp16,
// S/Metal/Primitives/utility.metal:7-18): the activation between the gate/up
// and down GEMMs of the prefill shared expert. act may alias g.
__device__ __forceinline__ void gelu_mul_f16(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                             uint16_t* act, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kThreads)
        act[i] = f2h(gelu_tanh(h2f(g[i])) * h2f(u[i]));
}

constexpr uint32_t kPhase2Chunks = 4;     // 16-byte act pieces per thread: top_k·F <= 8192

// Phase 2: 8 slots × 8-lane segments per wave; P chunks of 32 per lane
// (F <= 256*P); R output rows per wave in flight. Dynamic LDS:
// xpairs_lds_bytes(top_k*F). BITS: code width of the down rows.
// blk / nblk as in gate_up_rows. FIXED = kStageCopy: acts 16-byte aligned
// (the activation staging's loads then carry exact waits: the fused layer
// launches), -1: any alignment, the mode read at run time.
template <int P, int R, int BITS = 4, int FIXED = -1>
__device__ __forceinline__ void moe_phase2(const ExpertPool& pool, const uint32_t* __restrict__ indices,
                                           const uint16_t* __restrict__ acts,
                                           const uint16_t* __restrict__ rw,
                                           const uint16_t* __restrict__ residual,
                                           uint16_t* __restrict__ y, uint32_t D, uint32_t F,
                                           uint32_t top_k, uint32_t blk, uint32_t nblk) {
    constexpr int SEG = 8;
    constexpr uint32_t NT = kThreads;
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_a[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    constexpr uint32_t nwaves = NT / 64;
    const uint32_t slot = lane >> 3;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = F >> 5;
    const uint32_t row_bytes = (F >> 3) * BITS;
    const uint32_t ngroups = F >> 6;
    const bool live = slot < top_k;
    const uint32_t wave_id = blk * nwaves + wave;
    const uint32_t wave_total = nblk * nwaves;
    const uint32_t n_acts = top_k * F;

    // independent loads first: the activations, the slot's expert index and
    // routing weight (unpredicated: dead slots read slot 0)
    XStage<NT, kPhase2Chunks, false, false, false, FIXED> xs;
    const NormArg copy{nullptr, nullptr, nullptr, 0.0f, kStageCopy};
    xs.load(acts, n_acts, copy);
    const uint32_t e_raw = indices[live ? slot : 0u];
    const uint16_t w_raw = rw[live ? slot : 0u];
    const uint32_t e = live ? e_raw : 0u;
    const bool valid = live && e < pool.num_experts;
    const uint8_t* blob = pool.base + (uint64_t)(valid ? e : 0u) * pool.stride;
    const uint8_t* dw = blob + pool.off.down_w;
    const uint16_t* ds = reinterpret_cast<const uint16_t*>(blob + pool.off.down_s);
    const uint16_t* db = reinterpret_cast<const uint16_t*>(blob + pool.off.down_b);

    QChunk<BITS> wv[R][P];
    uint32_t sr[R][P], br[R][P];      // raw fp16 scale / bias
    uint16_t res[R] = {};             // the rows' residuals, loaded with their weights
    auto issue = [&](uint32_t grp, auto first_c) {      // first group unconditional, as in gate_up_rows
        constexpr bool FIRST = decltype(first_c)::value;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t d0 = wave_id + (grp * R + r) * wave_total;
            const uint32_t d = FIRST && d0 >= D ? D - 1 : d0;
            if (FIRST || (d < D && valid)) {
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c0 = sl + p * SEG;
                    const uint32_t c = FIRST && c0 >= lpr ? lpr - 1 : c0;
                    if (FIRST || c < lpr) {
                        wv[r][p] = ldg_chunk<BITS>(dw + (size_t)d * row_bytes, c);
                        sr[r][p] = ds[(size_t)d * ngroups + (c >> 1)];
                        br[r][p] = db[(size_t)d * ngroups + (c >> 1)];
                    }
                }
            }
            if (residual && d < D) res[r] = residual[d];   // needed last: issued last
        }
    };
    issue(0, std::true_type{});
    // (staging the activations before the weight loads, as gate_up_rows
    // X_FIRST does, measured 6.3 against 6.0 us per config-1 launch)
    const XPairs xp = xs.pairs(acts, lds_a, n_acts, copy);      // slot s owns chunks s·lpr ..
    const float w_slot = live ? h2f(w_raw) : 0.0f;

    for (uint32_t grp = 0; wave_id + grp * R * wave_total < D; ++grp) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
            if (valid) {
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c = sl + p * SEG;
                    if (c < lpr) {
                        XChunk xc;
                        read_xpairs(xp, slot * lpr + c, xc);
                        // literal magic: measured 6.2 us per config-1 launch
                        // against 6.8 us with the magic in a VGPR
                        const float dd = dot_chunk<BITS, false>(wv[r][p], xc);
                        acc[r] = fmaf(h2f((uint16_t)sr[r][p]), dd, acc[r]);
                        acc[r] = fmaf(h2f((uint16_t)br[r][p]), xc.sum, acc[r]);
                    }
                }
            } else if (live) {
                acc[r] = __builtin_nanf("");
            }
        }
        uint16_t res_now[R];          // issue() reloads res for the next group
#pragma unroll
        for (int r = 0; r < R; ++r) res_now[r] = res[r];
        issue(grp + 1, std::false_type{});
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t d = wave_id + (grp * R + r) * wave_total;
            const float part = w_slot * seg_sum<SEG>(acc[r]);   // partial[slot] = w·value (moe.metal:499)
            if (d < D) {
                float out = residual ? h2f(res_now[r]) : 0.0f;
#pragma unroll
                for (uint32_t s = 0; s < 8; ++s) {
                    const float ps = __shfl(part, (int)(s * SEG), kWave);   // v_readlane measured slower
                    if (s < top_k) out += ps;                   // fixed slot order (moe.metal:505-509)
                }
                if (lane == 0) y[d] = f2h(out);
            }
        }
    }
}

// The decoder layer's feed-forward launches with the int4 shared expert
// folded in. Each launch splits its blocks: [0, shared_blocks) compute the
// shared expert's part, the rest the routed experts' part (the same work as
// moe_phase1_routed / moe_phase2 launched alone). The shared blocks depend on
// nothing the routed blocks compute, so their weight stream runs while the
// routed blocks select their experts (phase 1) or read the indices (phase 2).
//
// Phase 1 + shared gate/up/act: the shared expert's input is h's RMSNorm with
// its own weight (pre_feedforward_layernorm), formed from the h and r(h) that
// the router's block 0 exported — `norm` (kStageScaled) with w = snorm_w.
template <int SEG, int P, int R, int BITS>
__device__ __forceinline__ void moe_phase1_routed_shared(
    const ExpertPool& pool, const float* __restrict__ logits, const uint16_t* __restrict__ gain, uint32_t E,
    uint32_t top_k, uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w, float* __restrict__ out_wf,
    const uint16_t* __restrict__ x, uint16_t* __restrict__ acts, uint32_t D, uint32_t F, const NormArg& norm,
    const Q4Mat& sgate, const Q4Mat& sup, const uint16_t* __restrict__ snorm_w, uint16_t* __restrict__ sact,
    uint32_t Fs, uint32_t shared_blocks) {
    if (blockIdx.x < shared_blocks) {
        NormArg ns = norm;
        ns.w = snorm_w;
        q4_gate_up_act<SEG, P, R, true, (int)kStageScaled>(sgate, sup, x, sact, D, Fs, ns, blockIdx.x,
                                                           shared_blocks);
    } else {
        moe_phase1_routed<SEG, P, R, true, BITS, (int)kStageScaled>(pool, logits, gain, E, top_k, out_idx, out_w,
                                                                    out_wf, x, acts, D, F, norm,
                                                                    blockIdx.x - shared_blocks,
                                                                    gridDim.x - shared_blocks);
    }
}

// Phase 2 + the shared expert's down GEMV (rows of Fs codes, 32-lane
// segments, SP chunks per lane: Fs <= 1024·SP) into sy. Dynamic LDS: the
// larger of phase 2's and the GEMV's.
template <int P2, int SP, int R, int BITS>
__device__ __forceinline__ void moe_phase2_shared(const ExpertPool& pool, const uint32_t* __restrict__ indices,
                                                  const uint16_t* __restrict__ acts, const uint16_t* __restrict__ rw,
                                                  uint16_t* __restrict__ y, uint32_t D, uint32_t F, uint32_t top_k,
                                                  const Q4Mat& sdown, const uint16_t* __restrict__ sact,
                                                  uint16_t* __restrict__ sy, uint32_t Fs, uint32_t shared_blocks) {
    if (blockIdx.x < shared_blocks) {
        Q4Multi mats{};
        mats.m[0] = {sdown.w, sdown.s, sdown.b, sy, nullptr, D, 0};
        mats.nmat = 1;
        mats.total_rows = D;
        mats.norm = NormArg{nullptr, nullptr, nullptr, 0.0f, kStageCopy};
        // sact: the workspace's 16-byte aligned act vector, Fs <= 4096
        q4_rows<32, SP, R, false, false, 4, false, kThreads, (int)kStageCopy>(
            mats, sact, Fs, [&](uint32_t row, float v) { sy[row] = f2h(v); }, blockIdx.x, shared_blocks);
    } else {
        moe_phase2<P2, R, BITS, (int)kStageCopy>(pool, indices, acts, rw, nullptr, y, D, F, top_k,
                                                 blockIdx.x - shared_blocks, gridDim.x - shared_blocks);
    }
}

// The same two launches with the int8 shared expert: its gate/up/act rows
// (q8_gate_up_act, SEG8 x P8 lanes per row of D bytes) beside phase 1, and
// its down rows (q8_gemv, rows of Fs bytes) beside phase 2. Dynamic LDS: the
// larger of the two parts'.
template <int SEG, int P, int SEG8, int P8, int R>
__device__ __forceinline__ void moe_phase1_routed_shared8(
    const ExpertPool& pool, const float* __restrict__ logits, const uint16_t* __restrict__ gain, uint32_t E,
    uint32_t top_k, uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w, float* __restrict__ out_wf,
    const uint16_t* __restrict__ x, uint16_t* __restrict__ acts, uint32_t D, uint32_t F, const NormArg& norm,
    const Q8Mat& sgate, const Q8Mat& sup, const uint16_t* __restrict__ snorm_w, uint16_t* __restrict__ sact,
    uint32_t Fs, uint32_t shared_blocks) {
    if (blockIdx.x < shared_blocks) {
        NormArg ns = norm;
        ns.w = snorm_w;
        q8_gate_up_act<SEG8, P8, R, true, (int)kStageScaled>(sgate, sup, x, 0, sact, D, Fs, ns, blockIdx.x,
                                                             shared_blocks);
    } else {
        moe_phase1_routed<SEG, P, R, true, 4, (int)kStageScaled>(pool, logits, gain, E, top_k, out_idx, out_w,
                                                                 out_wf, x, acts, D, F, norm,
                                                                 blockIdx.x - shared_blocks,
                                                                 gridDim.x - shared_blocks);
    }
}

template <int P2, int SEG8, int P8, int R>
__device__ __forceinline__ void moe_phase2_shared8(const ExpertPool& pool, const uint32_t* __restrict__ indices,
                                                   const uint16_t* __restrict__ acts,
                                                   const uint16_t* __restrict__ rw, uint16_t* __restrict__ y,
                                                   uint32_t D, uint32_t F, uint32_t top_k, const Q8Mat& sdown,
                                                   const uint16_t* __restrict__ sact, uint16_t* __restrict__ sy,
                                                   uint32_t Fs, uint32_t shared_blocks) {
    if (blockIdx.x < shared_blocks) {
        q8_gemv<SEG8, P8, R, (int)kStageCopy>(sdown.w, sdown.s, sdown.b, sact, 0, sy, 0, D, Fs, blockIdx.x,
                                              shared_blocks);
    } else {
        moe_phase2<P2, R, 4, (int)kStageCopy>(pool, indices, acts, rw, nullptr, y, D, F, top_k,
                                              blockIdx.x - shared_blocks, gridDim.x - shared_blocks);
    }
}

}  // namespace tfq
