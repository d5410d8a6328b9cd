// gemv.hpp — decode-side GEMVs: int4 g64 (plain and fused QKV), int8 g64,
// the int8 router logits + top-k selection, and the BF16 -> fp16 converter.
//
// Mapping (all GEMVs): one chunk of a weight row per lane — 32 codes, 16
// bytes at 4 bits (12 at 3, 8 at 2; 16 int8 codes) — so every weight byte
// arrives through one wide load and a segment's lanes read one contiguous
// run of the row. A row of n codes has n/32 (2/3/4-bit) or n/16 (int8)
// chunks; a segment of SEG lanes walks them with stride SEG (P chunks per
// lane). Lane <-> chunk is fixed for the whole kernel, so each lane keeps the
// activations of its P chunks in registers (staged once through LDS) together
// with the per-chunk activation sum needed by the affine factoring
//     Σ_k (q_k·s + b)·x_k = s·Σ q_k x_k + b·Σ x_k        (per group of 64)
// (S/Metal/Quant/dequant_int4.metal:14-17).
//
// Latency: the kernels are HBM-latency bound at decode sizes, so every
// segment issues the weight/scale/bias loads of its first R rows *before*
// staging x, and each later group of R rows is requested before the group
// ahead of it is consumed (two groups in flight per wavefront, q4_rows).
#pragma once

#include "abi_types.h"
#include "common.hpp"

namespace tfq {

// Row r of a multi-matrix launch -> (weights row, scales row, biases row, y slot, residual slot).
struct Q4Row {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint16_t* y;
    const uint16_t* r;
};

__device__ __forceinline__ Q4Row resolve_row(const Q4Multi& mats, uint32_t row, uint32_t row_bytes,
                                             uint32_t ngroups) {
    uint32_t r = row;
    const uint8_t* w = mats.m[0].w;
    const uint16_t* s = mats.m[0].s;
    const uint16_t* b = mats.m[0].b;
    uint16_t* y = mats.m[0].y;
    const uint16_t* res = mats.m[0].r;
    if (mats.nmat > 1 && r >= mats.m[0].rows) {
        r -= mats.m[0].rows;
        w = mats.m[1].w; s = mats.m[1].s; b = mats.m[1].b; y = mats.m[1].y; res = mats.m[1].r;
        if (mats.nmat > 2 && r >= mats.m[1].rows) {
            r -= mats.m[1].rows;
            w = mats.m[2].w; s = mats.m[2].s; b = mats.m[2].b; y = mats.m[2].y; res = mats.m[2].r;
        }
    }
    return {w + (size_t)r * row_bytes, s + (size_t)r * ngroups, b + (size_t)r * ngroups, y + r,
            res ? res + r : nullptr};
}

// int4 GEMV over 1..3 matrices with a shared x. Dynamic LDS: xpairs_lds_bytes(n).
// Order of work: the x loads, then every weight / scale / bias load of the
// first R rows (scale and bias kept raw, so nothing waits on them), then the
// staging, which waits for x alone; the weights arrive meanwhile.
// NORM == false: the staging only copies x (mats.norm is ignored), which
// keeps the norm inputs' registers out of the kernel and its occupancy up.
// The row loop; out(row, v) receives each row's fp32 result on lane 0 of its
// segment. STAGE_FIRST: finish staging x before the first weight loads, so
// the staging's registers are free before the weight registers fill (one
// memory latency later start, worth it for long launches: higher occupancy).
// BITS: code width of the weight rows (2, 3 or 4; rows of n·BITS/8 bytes).
// TAIL: the kStageTail staging form (the previous decoder layer's tail).
// NT: threads per block (256; 1024 for the tail form, whose staging reads
// nine vectors: a quarter of the blocks, each staging once for four times
// the rows, keeps that L2 traffic to a quarter).
// FIXED: the staging mode when it is known at compile time (XStage; the
// tail form always is), -1 when the kernel reads it from mats.norm. CHX:
// staged 16-byte chunks per thread (0: 2, 1 with 512+ threads), which
// bounds the fixed-mode staging's n at 8·CH·NT.
// blk / nblk: this block's index among the blocks that share the rows, and
// their count (blockIdx.x / gridDim.x unless a launch splits its blocks
// between two kinds of work).
template <int SEG, int P, int R, bool NORM, bool STAGE_FIRST = false, int BITS = 4, bool TAIL = false,
          uint32_t NT = kThreads, int FIXED = (TAIL ? (int)kStageTail : -1), uint32_t CHX = 0, typename Out>
__device__ __forceinline__ void q4_rows(const Q4Multi& mats, const uint16_t* __restrict__ x, uint32_t n,
                                        Out out, uint32_t blk, uint32_t nblk) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds_xh[];
    // staged 16-byte chunks per thread (CHX: chosen by the caller)
    constexpr uint32_t CH = CHX ? CHX : NT >= 512 ? 1 : kStageChunks;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    constexpr uint32_t nwaves = NT / 64;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = n >> 5;              // 32-code chunks per row
    const uint32_t row_bytes = (n >> 3) * BITS;
    const uint32_t ngroups = n >> 6;
    constexpr uint32_t spw = kWave / SEG;     // segments per wave
    const uint32_t seg_id = (blk * nwaves + wave) * spw + lane / SEG;
    const uint32_t seg_total = nblk * nwaves * spw;
    const uint32_t total = mats.total_rows;

    QChunk<BITS> wv[R][P];
    uint32_t sr[R][P], br[R][P];      // raw fp16 scale / bias
    // issue(grp): a group's loads, unconditional (rows past the end re-read
    // the last row, chunks past the row its last chunk), so the waits after
    // them are exact (a load under a branch makes the compiler wait for
    // everything at the join)
    auto issue = [&](uint32_t grp) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row0 = seg_id + (grp * R + r) * seg_total;
            const Q4Row q = resolve_row(mats, row0 < total ? row0 : total - 1, row_bytes, ngroups);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c0 = sl + p * SEG;
                const uint32_t c = c0 < lpr ? c0 : lpr - 1;
                wv[r][p] = ldg_chunk<BITS>(q.w, c);
                sr[r][p] = q.s[c >> 1];
                br[r][p] = q.b[c >> 1];
            }
        }
    };
    XStage<NT, CH, NORM, true, TAIL, FIXED> xs;
    xs.load(x, n, mats.norm);
    {
        // Two row groups in flight per wave: the next group's loads are
        // issued before the current group's dot (buffers wv and w2
        // alternate). Every issue is unconditional (rows past the end
        // re-read the last row, chunks past the row its last chunk; neither
        // is stored), so each wait covers exactly the group it consumes,
        // and the wave-uniform group count ends the loop without a branch
        // around any load. (With one group in flight and the next one's
        // loads issued after the dot, skipped past the end: config 0 3.68
        // against 3.42 us, the greedy LM head 71.2 against 67.4 us, the
        // 3-bit LM-head-shape GEMV 75.3 against 62.3 us.)
        QChunk<BITS> w2[R][P];
        uint32_t s2[R][P], b2[R][P];
        auto issue2 = [&](uint32_t grp) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t row0 = seg_id + (grp * R + r) * seg_total;
                const Q4Row q = resolve_row(mats, row0 < total ? row0 : total - 1, row_bytes, ngroups);
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c0 = sl + p * SEG;
                    const uint32_t c = c0 < lpr ? c0 : lpr - 1;
                    w2[r][p] = ldg_chunk<BITS>(q.w, c);
                    s2[r][p] = q.s[c >> 1];
                    b2[r][p] = q.b[c >> 1];
                }
            }
        };
        auto consume = [&](uint32_t grp, const QChunk<BITS> (&w)[R][P], const uint32_t (&s)[R][P],
                           const uint32_t (&b)[R][P], const XPairs& xpp) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float acc = 0.0f;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c = sl + p * SEG;
                    if (c < lpr) {
                        XChunk xc;
                        read_xpairs(xpp, c, xc);
                        const float d = dot_chunk<BITS>(w[r][p], xc);
                        acc = fmaf(h2f((uint16_t)s[r][p]), d, acc);
                        acc = fmaf(h2f((uint16_t)b[r][p]), xc.sum, acc);
                    }
                }
                const float v = seg_sum<SEG>(acc);
                const uint32_t row = seg_id + (grp * R + r) * seg_total;
                if (sl == 0 && row < total) out(row, v);
            }
        };
        // groups of the wave's first segment (the most of its segments)
        const uint32_t seg0 = (blk * nwaves + wave) * spw;
        const uint32_t ng = __builtin_amdgcn_readfirstlane(
            seg0 < total ? (total - seg0 + R * seg_total - 1) / (R * seg_total) : 0u);   // wave-uniform
        if (!STAGE_FIRST) issue(0);
        const XPairs xp2 = xs.pairs(x, lds_xh, n, mats.norm);
        if (STAGE_FIRST) issue(0);
        uint32_t grp = 0;
        for (; grp + 1 < ng; grp += 2) {
            issue2(grp + 1);
            consume(grp, wv, sr, br, xp2);
            issue(grp + 2);      // past the last group: the last row, not stored
            consume(grp + 1, w2, s2, b2, xp2);
        }
        if (grp < ng) consume(grp, wv, sr, br, xp2);
    }
}

template <int SEG, int P, int R, bool NORM, int BITS = 4, bool TAIL = false, uint32_t NT = kThreads,
          int FIXED = (TAIL ? (int)kStageTail : -1), uint32_t CHX = 0>
__device__ __forceinline__ void q4_gemv_multi(const Q4Multi& mats, const uint16_t* __restrict__ x,
                                              uint32_t n) {
    const uint32_t row_bytes = (n >> 3) * BITS, ngroups = n >> 6;
    const bool out_bf16 = NORM && mats.norm.mode == kStageBf16;
    q4_rows<SEG, P, R, NORM, false, BITS, TAIL, NT, FIXED, CHX>(mats, x, n, [&](uint32_t row, float v) {
        const Q4Row q = resolve_row(mats, row, row_bytes, ngroups);
        const float o = q.r ? h2f(*q.r) + v : v;
        *q.y = out_bf16 ? __builtin_bit_cast(uint16_t, (__bf16)o) : f2h(o);
    }, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------- int8 ----
//
// The int8 paths (router logits, DequantInt8GEMV) keep fp32 activations:
// the router multiplies h by the effective scale in fp32 before the dot,
// and its top-k ordering must not see an extra fp16 rounding.

// Load the 16 fp32 activations of int8 chunk c and their sum.
__device__ __forceinline__ void load_x16(const float* __restrict__ lds, uint32_t c, float* xr,
                                         float& xs) {
    const float4* src = reinterpret_cast<const float4*>(lds + 16u * c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = src[i];
        xr[4 * i + 0] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += xr[i];
    xs = s;
}

// Rows of an int8 GEMV. `stage(issue0)` must fill lds_x (fp32, n values) and
// synchronise; it calls issue0() (the first row group's loads) once its own
// input loads are in flight, before it waits for them.
// Emits fp32 results through `out(row, value)` from lane 0 of each segment.
// blk / nblk as in q4_rows.
template <int SEG, int P, int R, typename Stage, typename Out>
__device__ __forceinline__ void q8_rows(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                        const uint16_t* __restrict__ B, float* __restrict__ lds_x,
                                        uint32_t M, uint32_t n, Stage stage, Out out, uint32_t blk,
                                        uint32_t nblk) {
    constexpr uint32_t NT = kThreads;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    constexpr uint32_t nwaves = NT / 64;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = n >> 4;
    const uint32_t ngroups = n >> 6;
    constexpr uint32_t spw = kWave / SEG;
    const uint32_t seg_id = (blk * nwaves + wave) * spw + lane / SEG;
    const uint32_t seg_total = nblk * nwaves * spw;

    uint4 wv[R][P];
    uint32_t sr[R][P], br[R][P];      // raw fp16 scale / bias
    auto issue = [&](uint32_t grp, auto first_c) {      // first group unconditional, as in q4_rows
        constexpr bool FIRST = decltype(first_c)::value;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row0 = seg_id + (grp * R + r) * seg_total;
            const uint32_t row = FIRST && row0 >= M ? M - 1 : row0;
            if (FIRST || row < M) {
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c0 = sl + p * SEG;
                    const uint32_t c = FIRST && c0 >= lpr ? lpr - 1 : c0;
                    if (FIRST || c < lpr) {
                        wv[r][p] = ldg16_stream(W + (size_t)row * n + 16u * c);
                        sr[r][p] = S[(size_t)row * ngroups + (c >> 2)];
                        br[r][p] = B[(size_t)row * ngroups + (c >> 2)];
                    }
                }
            }
        }
    };
    stage([&]() { issue(0, std::true_type{}); });
    float xr[P][16];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_x16(lds_x, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }
    for (uint32_t grp = 0; seg_id + grp * R * seg_total < M; ++grp) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c = sl + p * SEG;
                if (c < lpr) {
                    const float d = dot16_q8(wv[r][p], xr[p]);
                    acc[r] = fmaf(h2f((uint16_t)sr[r][p]), d, acc[r]);
                    acc[r] = fmaf(h2f((uint16_t)br[r][p]), xs[p], acc[r]);
                }
            }
        }
        issue(grp + 1, std::false_type{});
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = seg_sum<SEG>(acc[r]);
            const uint32_t row = seg_id + (grp * R + r) * seg_total;
            if (sl == 0 && row < M) out(row, v);
        }
    }
}

// blockIdx.y selects the token of a block of inputs: x + y·x_stride, y + y·y_stride.
// blk / nblk as in q4_rows; FIXED = kStageCopy: x 16-byte aligned, n <= 4096.
template <int SEG, int P, int R, int FIXED = -1>
__device__ __forceinline__ void q8_gemv(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                        const uint16_t* __restrict__ B, const uint16_t* __restrict__ x,
                                        uint32_t x_stride, uint16_t* __restrict__ y, uint32_t y_stride,
                                        uint32_t M, uint32_t n, uint32_t blk, uint32_t nblk) {
    extern __shared__ __attribute__((aligned(16))) float lds_x[];
    x += (size_t)blockIdx.y * x_stride;
    y += (size_t)blockIdx.y * y_stride;
    q8_rows<SEG, P, R>(
        W, S, B, lds_x, M, n,
        [&](auto issue0) {
            uint16_t* xs = reinterpret_cast<uint16_t*>(lds_x + n);
            const NormArg copy{nullptr, nullptr, nullptr, 0.0f, kStageCopy};
            XStage<kThreads, kStageChunks, true, true, false, FIXED> st;
            st.load(x, n, copy);
            issue0();
            if (st.vec) {
                // the staged chunks widened straight into the fp32 vector
                // (clamped and unconditional like the loads)
#pragma unroll
                for (uint32_t i = 0; i < kStageChunks; ++i) {
                    const uint32_t c0 = threadIdx.x + i * kThreads;
                    const uint32_t c = c0 < (n >> 3) ? c0 : (n >> 3) - 1;
#pragma unroll
                    for (int e = 0; e < 8; ++e) lds_x[8 * c + e] = (float)st.xv[i][e];
                }
                __syncthreads();
                return;
            }
            st.plain(x, xs, n, copy);
            for (uint32_t i = threadIdx.x; i < n; i += kThreads) lds_x[i] = h2f(xs[i]);
            __syncthreads();
        },
        [&](uint32_t row, float v) { y[row] = f2h(v); }, blk, nblk);
}

// -------------------------------------------------------------- router ----

constexpr uint32_t kRouterMaxExperts = 256;
constexpr uint32_t kRouterMaxTopK = 64;

// logits[e] = Σ_g s·Σ q·(h⊙eff) + b·Σ(h⊙eff), fp32 (S/Metal/MoE/moe.metal:78-116).
// Dynamic LDS: d floats.
// With norm.w set, h is first RMS-normalised (to fp16, as a separate norm
// kernel would store it). Dynamic LDS: d floats + d halves.
// FIXED: the staging mode when known at compile time (XStage; h, eff and the
// norm vectors then 16-byte aligned, d <= 4096), else -1.
template <int SEG, int P, int FIXED = -1>
__device__ __forceinline__ void router_logits(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                              const uint16_t* __restrict__ B, const uint16_t* __restrict__ h,
                                              const uint16_t* __restrict__ eff,
                                              float* __restrict__ logits, uint32_t E, uint32_t d,
                                              NormArg norm = {nullptr, nullptr, nullptr, 0.0f, kStageCopy}) {
    extern __shared__ __attribute__((aligned(16))) float lds_x[];
    q8_rows<SEG, P, 1>(
        W, S, B, lds_x, E, d,
        [&](auto issue0) {
            constexpr uint32_t NT = kThreads;
            uint16_t* hs = reinterpret_cast<uint16_t*>(lds_x + d);
            XStage<NT, kStageChunks, true, true, false, FIXED> st;
            st.load(h, d, norm);
            // the effective-scale chunks are loaded with h, before the weights
            const bool vec =
                FIXED >= 0 || ((((uintptr_t)eff) & 15u) == 0 && (d & 7u) == 0 && (d >> 3) <= kStageChunks * NT);
            h8 ev[kStageChunks];
            if (FIXED >= 0 || (eff && vec))
#pragma unroll
                for (uint32_t i = 0; i < kStageChunks; ++i) {
                    const uint32_t c = threadIdx.x + i * NT;
                    ev[i] = __builtin_bit_cast(h8, ld16h(eff ? eff : h, c < (d >> 3) ? c : (d >> 3) - 1));
                }
            issue0();
            if (st.vec && vec) {
                // the staged chunks (after the NormArg transform) times eff
                // straight into the fp32 vector: no fp16 copy in LDS and one
                // barrier; clamped and unconditional like the loads
                st.transform(d, norm);
#pragma unroll
                for (uint32_t i = 0; i < kStageChunks; ++i) {
                    const uint32_t c0 = threadIdx.x + i * NT;
                    const uint32_t c = c0 < (d >> 3) ? c0 : (d >> 3) - 1;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        lds_x[8 * c + e] = eff ? (float)st.xv[i][e] * (float)ev[i][e] : (float)st.xv[i][e];
                }
                __syncthreads();
                return;
            }
            st.plain(h, hs, d, norm);
            if (vec) {
#pragma unroll
                for (uint32_t i = 0; i < kStageChunks; ++i) {
                    // clamped like the loads: chunks past the end rewrite the
                    // last chunk's identical values, so no branch holds the
                    // eff load (see XStage::plain)
                    const uint32_t c0 = threadIdx.x + i * NT;
                    const uint32_t c = c0 < (d >> 3) ? c0 : (d >> 3) - 1;
                    const h8 hv = reinterpret_cast<const h8*>(hs)[c];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        lds_x[8 * c + e] = eff ? (float)hv[e] * (float)ev[i][e] : (float)hv[e];
                }
            } else {
                for (uint32_t i = threadIdx.x; i < d; i += NT) {
                    const float hv = h2f(hs[i]);
                    lds_x[i] = eff ? hv * h2f(eff[i]) : hv;
                }
            }
            __syncthreads();
        },
        [&](uint32_t row, float v) { logits[row] = v; }, blockIdx.x, gridDim.x);
}

// Order key of logit v at index t: larger key = ranked first. The float
// bits are mapped to an unsigned order (topk_order: sign-magnitude ->
// biased), and the low half holds ~t so that equal logits rank by lower
// index. -0 ranks as +0 (they compare equal, so the lower index wins), and
// NaN ranks below -inf: router_topk_select_k8 (S/Metal/MoE/moe.metal:152-168)
// never prefers a NaN score to a number. Every finite or infinite v gets an
// order value > 0.
__device__ __forceinline__ uint32_t topk_order(float v) {
    uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t mag = b & 0x7FFFFFFFu;
    if (mag == 0) b = 0;
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return mag > 0x7F800000u ? 0u : o;
}
__device__ __forceinline__ uint64_t topk_key(float v, uint32_t t) {
    return ((uint64_t)topk_order(v) << 32) | (uint32_t)(0xFFFFFFFFu - t);
}

// Greedy int4 LM head, rows stage (logit.metal:688-737): z = W·x for every
// vocab row, x the RMSNorm of the hidden state staged like every GEMV input
// (fp16, as the reference's xNormed buffer); each block writes the largest
// finite z of its rows with the lowest row on ties as a topk_key
// (0 = no finite z) to summaries[blockIdx.x]. FIXED = kStageNorm: the RMSNorm
// staging with its mode fixed at compile time (x and the norm weight 16-byte
// aligned, n <= 4096), -1: the mode read at run time.
template <int SEG, int P, int R, int FIXED = -1>
__device__ __forceinline__ void lm_head_greedy_rows(const Q4Multi& mats, const uint16_t* __restrict__ x,
                                                    uint32_t n, uint64_t* __restrict__ summaries) {
    // a lane's rows arrive in increasing order, so a strict > keeps the lowest
    // row among equal values (and -0 vs +0, which compare equal)
    float best_v = -__builtin_inff();
    uint32_t best_row = 0xFFFFFFFFu;
    q4_rows<SEG, P, R, true, true, 4, false, kThreads, FIXED>(mats, x, n, [&](uint32_t row, float v) {
        if (__builtin_isfinite(v) && (best_row == 0xFFFFFFFFu || v > best_v)) {
            best_v = v;
            best_row = row;
        }
    }, blockIdx.x, gridDim.x);
    uint64_t best = best_row == 0xFFFFFFFFu ? 0ull : topk_key(best_v, best_row);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t other = __shfl_xor(best, o, kWave);
        best = other > best ? other : best;
    }
    __shared__ uint64_t wave_best[kThreads / 64];
    if ((threadIdx.x & 63u) == 0) wave_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wave_best[0];
        for (uint32_t w = 1; w < kThreads / 64; ++w) b = wave_best[w] > b ? wave_best[w] : b;
        summaries[blockIdx.x] = b;
    }
}

// Greedy int4 LM head, reduce stage (logit.metal:740-787): the token of the
// largest key over n block summaries, 0 when none holds a finite z.
__device__ __forceinline__ void lm_head_greedy_reduce(const uint64_t* __restrict__ summaries, uint32_t n,
                                                      uint32_t* __restrict__ out_token) {
    // eight summaries per thread in flight together (indices past n re-read
    // the last one, which leaves the maximum unchanged): one memory round
    // trip per 2048 summaries instead of one per 256
    constexpr uint32_t U = 8;
    uint64_t best = 0;
    for (uint32_t base = 0; base < n; base += U * kThreads) {
        uint64_t v[U];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = base + u * kThreads + threadIdx.x;
            v[u] = summaries[i < n ? i : n - 1];
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) best = v[u] > best ? v[u] : best;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t other = __shfl_xor(best, o, kWave);
        best = other > best ? other : best;
    }
    __shared__ uint64_t wave_best[kThreads / 64];
    if ((threadIdx.x & 63u) == 0) wave_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = wave_best[0];
        for (uint32_t w = 1; w < kThreads / 64; ++w) b = wave_best[w] > b ? wave_best[w] : b;
        *out_token = b ? ~(uint32_t)b : 0u;      // the key's low word is ~row
    }
}

// Top-k of E <= 256 logits by (value desc, index asc). Logit t's rank is
// the number of logits ordered before it: rank_t = #{o_j > o_t} +
// #{j < t : o_j == o_t}, o = topk_order + 1 (>= 1; padding 0). The logits are
// cut into blocks of 8; thread (row a, column c) of each 16-lane row counts,
// for the 8 logits of block a, those of blocks c, c + 16, ... that are
// ordered before them, the tie-break folded into a threshold per pair
// (o_j >= o_t  <=>  o_j > o_t - 1); the row's 16 partial counts are added
// with DPP (8-bit fields, 4 per word: a rank is at most 255). Ranks are
// unique, so the k logits with rank < k each write their slot. `stage`
// holds the E logits; `sel_idx` / `sel_val` receive the k winners in rank
// order. Ends with a block barrier.
__device__ __forceinline__ void block_topk(const float* stage, uint32_t E, uint32_t k,
                                           uint32_t* sel_idx, float* sel_val) {
    static_assert(kThreads == 256 && kRouterMaxExperts <= 256, "16 rows of 16 lanes, 8-bit ranks");
    __shared__ __attribute__((aligned(16))) uint32_t ord[kRouterMaxExperts];
    for (uint32_t t = threadIdx.x; t < kRouterMaxExperts; t += kThreads)
        ord[t] = t < E ? topk_order(stage[t]) + 1u : 0u;
    __syncthreads();
    const uint32_t nb = (E + 7) / 8;
    const uint32_t row = threadIdx.x / 16, col = threadIdx.x % 16;
    for (uint32_t a = row; a < nb; a += kThreads / 16) {
        const uint4 a0 = reinterpret_cast<const uint4*>(ord)[2 * a];
        const uint4 a1 = reinterpret_cast<const uint4*>(ord)[2 * a + 1];
        const uint32_t oi[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        uint32_t cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (uint32_t b = col; b < nb; b += 16) {
            const uint4 b0 = reinterpret_cast<const uint4*>(ord)[2 * b];
            const uint4 b1 = reinterpret_cast<const uint4*>(ord)[2 * b + 1];
            const uint32_t oj[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            const uint32_t lt = b < a ? 1u : 0u, le = b <= a ? 1u : 0u;
#pragma unroll
            for (int ii = 0; ii < 8; ++ii) {
                // real keys have o >= 1, so their thresholds are >= 0 and
                // padding (o = 0) never counts
                const uint32_t t_lt = oi[ii] - lt, t_le = oi[ii] - le;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) cnt[ii] += oj[jj] > (jj < ii ? t_le : t_lt) ? 1u : 0u;
            }
        }
        uint32_t lo = cnt[0] | cnt[1] << 8 | cnt[2] << 16 | cnt[3] << 24;
        uint32_t hi = cnt[4] | cnt[5] << 8 | cnt[6] << 16 | cnt[7] << 24;
        lo = row16_sum_u32(lo);
        hi = row16_sum_u32(hi);
        const uint32_t t = 8 * a + col;
        if (col < 8 && t < E) {
            const uint32_t rank = ((col < 4 ? lo : hi) >> (8 * (col % 4))) & 0xFFu;
            if (rank < k) {
                sel_idx[rank] = t;
                sel_val[rank] = stage[t];
            }
        }
    }
    __syncthreads();
}

// Softmax over the k selected logits times the per-expert gain
// (S/Metal/MoE/moe.metal:169-184): weights[r] = exp(v_r - v_0) / Σ exp × gain.
// Exponentials in parallel, their sum in rank order by one thread.
__device__ __forceinline__ void block_softmax_gain(const uint32_t* sel_idx, const float* sel_val,
                                                   uint32_t k, const uint16_t* __restrict__ gain,
                                                   float* ex, float* sel_w) {
    const float vmax = sel_val[0];
    for (uint32_t r = threadIdx.x; r < k; r += kThreads) ex[r] = expf(sel_val[r] - vmax);
    __syncthreads();
    __shared__ float total;
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (uint32_t r = 0; r < k; ++r) sum += ex[r];
        total = sum;
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < k; r += kThreads)
        sel_w[r] = ex[r] / total * (gain ? h2f(gain[sel_idx[r]]) : 1.0f);
    __syncthreads();
}

// Selection of one block from logits already staged in LDS (16-byte
// aligned, padded to a multiple of 4 with -inf): top-k indices and
// softmax × gain weights into the caller's LDS arrays (k entries).
// Deterministic: every block that runs it on the same logits gets the same
// bits.
__device__ __forceinline__ void router_select_staged(const float* stage, const uint16_t* __restrict__ gain,
                                                     uint32_t E, uint32_t k, uint32_t* sel_idx, float* sel_w) {
    __shared__ float sel_val[kRouterMaxTopK];
    __shared__ float ex[kRouterMaxTopK];
    block_topk(stage, E, k, sel_idx, sel_val);
    block_softmax_gain(sel_idx, sel_val, k, gain, ex, sel_w);
}

// As router_select_staged, reading the logits from global memory.
__device__ __forceinline__ void router_select_lds(const float* __restrict__ logits,
                                                  const uint16_t* __restrict__ gain, uint32_t E, uint32_t k,
                                                  uint32_t* sel_idx, float* sel_w) {
    __shared__ __attribute__((aligned(16))) float stage[kRouterMaxExperts];
    for (uint32_t e = threadIdx.x; e < ((E + 3) & ~3u); e += kThreads)
        stage[e] = e < E ? logits[e] : -__builtin_inff();
    __syncthreads();
    router_select_staged(stage, gain, E, k, sel_idx, sel_w);
}

// Selection kernel body: logits (global) -> indices, fp16 weights, fp32 weights.
__device__ __forceinline__ void router_select(const float* __restrict__ logits,
                                              const uint16_t* __restrict__ gain,
                                              uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w,
                                              float* __restrict__ out_wf, uint32_t E, uint32_t k) {
    __shared__ uint32_t sel_idx[kRouterMaxTopK];
    __shared__ float sel_w[kRouterMaxTopK];
    router_select_lds(logits, gain, E, k, sel_idx, sel_w);
    for (uint32_t r = threadIdx.x; r < k; r += kThreads) {
        out_idx[r] = sel_idx[r];
        out_w[r] = f2h(sel_w[r]);
        if (out_wf) out_wf[r] = sel_w[r];
    }
}

// ------------------------------------------------------------ read probe ----

// Pure HBM read ceiling (the role of bw_ceiling_read, S/Metal/Quant/
// dequant_int4.metal:487-502): every lane reads U 16-byte chunks with one
// coalesced non-temporal 128-bit load each (the load the GEMVs stream their
// weights with), all issued before any is consumed; the xor of
// everything read goes to sink[block] so nothing is optimised away.
template <int U>
__device__ __forceinline__ void read_ceiling(const uint4* __restrict__ src, uint64_t n16,
                                             uint32_t* __restrict__ sink) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kThreads;
    uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    uint32_t acc = 0;
    for (; i < n16; i += nthreads * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t j = i + (uint64_t)u * nthreads;
            v[u] = j < n16 ? ldg16_stream(reinterpret_cast<const uint8_t*>(src + j)) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    __shared__ uint32_t red;
    if (threadIdx.x == 0) red = 0;
    __syncthreads();
    atomicXor(&red, acc);
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red;
}

// ------------------------------------------------------------- convert ----

// src and dst may be the same buffer (each element is read, then written, by
// one thread).
__device__ __forceinline__ void convert_bf16_to_f16(const uint16_t* src, uint16_t* dst, uint64_t n,
                                                    uint32_t* __restrict__ inexact) {
    uint32_t bad = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * kThreads) {
        const float v = bf2f(src[i]);
        const uint16_t hbits = f2h(v);
        dst[i] = hbits;
        const float back = h2f(hbits);
        if (!(back == v) && !(v != v)) ++bad;   // NaN passes through as NaN
    }
    if (inexact && bad) atomicAdd(inexact, bad);
}

}  // namespace tfq
