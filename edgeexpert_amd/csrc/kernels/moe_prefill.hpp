// moe_prefill.hpp — routed MoE over a chunk of T prompt tokens:
//   router logits for every token -> per-token top-k -> device grouping of
//   the (token, expert, rank) pairs by expert -> grouped int4 GEMMs
//   (gate/up + GeGLU, then down) on the matrix cores -> token-major combine.
// Reference path: PrefillRouter.encodeGemma4Block
// (S/Kernels/Prefill/MoE/PrefillRouter.swift:37-89), the CPU grouping
// PrefillMoEGrouping.groupTokenExpertPairs (PrefillMoEGrouping.swift:91-192),
// PrefillGroupedRoutedMoE.encodeStreamedBatched
// (PrefillGroupedRoutedMoE.swift:446-527; kernels S/Metal/Prefill/prefill.metal:598-670)
// and PrefillMoE.encodeReduceTokenMajor (PrefillMoE.swift:11-38; prefill.metal:575-596).
// Here the pairs never leave the device; every expert's rows become one or
// more 128-row tiles, each run as two 64-row halves on the matrix cores.
#pragma once

#include "abi_types.h"
#include "gemm.hpp"
#include "gemv.hpp"

namespace tfq {

constexpr uint32_t kGroupMaxPairs = 8192;
constexpr uint32_t kGroupMaxExperts = 256;
constexpr uint32_t kGroupChunks = kGroupMaxPairs / 64;
constexpr uint32_t kGroupThreads = 1024;
// status codes (the PrefillMoEGroupingError cases the device can detect)
constexpr uint32_t kGroupOk = 0;
constexpr uint32_t kGroupExpertOutOfRange = 8;

// Stable counting sort of the token-major pairs (token t, rank r) -> expert
// idx[t*k + r], one block of 1024 threads. Pairs come out ordered by
// (expert, token, rank) exactly as the reference's sort
// (PrefillMoEGrouping.swift:145-154 without sort keys): each wavefront
// ranks its 64 pairs among equal experts with ballots, a per-expert scan
// over the 64-pair chunks (in order) gives each chunk's base, and an
// exclusive scan over experts gives the offsets. Empty experts get offset
// 0xFFFFFFFF and count 0. The tile list cuts each expert's run into
// 128-row tiles. On an out-of-range expert index nothing is grouped and
// *status = kGroupExpertOutOfRange.
__device__ __forceinline__ void moe_group(const uint32_t* __restrict__ idx, const uint16_t* __restrict__ w,
                                          uint32_t T, uint32_t k, uint32_t E, Pair* __restrict__ sorted,
                                          uint32_t* __restrict__ offsets, uint32_t* __restrict__ counts,
                                          Tile* __restrict__ tiles, uint32_t* __restrict__ n_tiles,
                                          uint32_t* __restrict__ status) {
    __shared__ uint16_t cnt[kGroupChunks][kGroupMaxExperts];
    __shared__ uint8_t rank_in_chunk[kGroupMaxPairs];
    __shared__ uint32_t base[kGroupMaxExperts], tot[kGroupMaxExperts], tile_base[kGroupMaxExperts + 1];
    __shared__ uint32_t bad;
    constexpr uint32_t kPer = kGroupMaxPairs / kGroupThreads;     // pairs per thread (8)
    const uint32_t tid = threadIdx.x;
    const uint32_t n = T * k;
    const uint32_t nchunks = (n + 63) / 64;
    // every thread loads its pairs' experts and weights once, all loads in flight together
    uint32_t my_e[kPer];
    uint16_t my_w[kPer];
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
        const uint32_t i = tid + j * kGroupThreads;
        my_e[j] = i < n ? idx[i] : 0u;
        my_w[j] = i < n ? w[i] : (uint16_t)0;
    }
    if (tid == 0) bad = 0;
    for (uint32_t i = tid; i < nchunks * kGroupMaxExperts; i += kGroupThreads)
        (&cnt[0][0])[i] = 0;
    uint32_t my_bad = 0;
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j)
        if (tid + j * kGroupThreads < n && my_e[j] >= E) my_bad = 1;
    __syncthreads();
    if (my_bad) atomicOr(&bad, 1u);
    __syncthreads();
    if (bad) {
        for (uint32_t e = tid; e < E; e += kGroupThreads) {
            offsets[e] = 0xFFFFFFFFu;
            counts[e] = 0;
        }
        if (tid == 0) {
            *n_tiles = 0;
            *status = kGroupExpertOutOfRange;
        }
        return;
    }

    // rank of each pair among equal experts inside its 64-pair chunk: pair
    // i = tid + j·1024 sits in chunk i/64 = (tid/64) + 16j, lane tid%64. The
    // lanes holding the same expert are found with one ballot per bit of the
    // expert id (a wave-wide match), so the cost does not grow with the
    // number of distinct experts in the chunk.
    const uint32_t lane = tid & 63u;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint32_t ebits = E > 1 ? 32u - (uint32_t)__clz((int)(E - 1)) : 1u;
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
        const uint32_t i = tid + j * kGroupThreads;
        const uint32_t c = i >> 6;
        if (c >= nchunks) continue;                       // wave-uniform
        const bool valid = i < n;
        const uint32_t e = my_e[j];
        uint64_t same = __ballot(valid);
        for (uint32_t b = 0; b < ebits; ++b) {
            const bool bit = (e >> b) & 1u;
            const uint64_t set = __ballot(bit);
            same &= bit ? set : ~set;
        }
        if (valid) {
            const uint32_t my_rank = (uint32_t)__popcll(same & lt_mask);
            if (my_rank == 0) cnt[c][e] = (uint16_t)__popcll(same);
            rank_in_chunk[i] = (uint8_t)my_rank;
        }
    }
    __syncthreads();
    // per expert: exclusive scan over the chunks (in chunk order)
    for (uint32_t e = tid; e < E; e += kGroupThreads) {
        uint32_t run = 0;
        for (uint32_t c = 0; c < nchunks; ++c) {
            const uint32_t v = cnt[c][e];
            cnt[c][e] = (uint16_t)run;
            run += v;
        }
        tot[e] = run;
    }
    __syncthreads();
    // exclusive scans over the experts of the pair counts and tile counts:
    // one wavefront, 64 experts per pass with a shuffle scan
    if (tid < 64) {
        uint32_t carry_p = 0, carry_t = 0;
        for (uint32_t e0 = 0; e0 < E; e0 += 64) {
            const uint32_t e = e0 + tid;
            const uint32_t p = e < E ? tot[e] : 0u;
            const uint32_t t = (p + kGemmBM - 1) / kGemmBM;
            uint32_t sp = p, st = t;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t up = (uint32_t)__shfl_up((int)sp, o, kWave);
                const uint32_t ut = (uint32_t)__shfl_up((int)st, o, kWave);
                if ((int)tid >= o) {
                    sp += up;
                    st += ut;
                }
            }
            if (e < E) {
                base[e] = carry_p + sp - p;
                tile_base[e] = carry_t + st - t;
            }
            carry_p += (uint32_t)__shfl((int)sp, 63, kWave);
            carry_t += (uint32_t)__shfl((int)st, 63, kWave);
        }
        if (tid == 0) {
            tile_base[E] = carry_t;
            *n_tiles = carry_t;
            *status = kGroupOk;
        }
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += kGroupThreads) {
        offsets[e] = tot[e] ? base[e] : 0xFFFFFFFFu;
        counts[e] = tot[e];
        for (uint32_t t = tile_base[e]; t < tile_base[e + 1]; ++t) {
            const uint32_t start = base[e] + (t - tile_base[e]) * kGemmBM;
            const uint32_t left = base[e] + tot[e] - start;
            tiles[t] = {e, start, left < (uint32_t)kGemmBM ? left : (uint32_t)kGemmBM, 0u};
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
        const uint32_t i = tid + j * kGroupThreads;
        if (i < n) {
            const uint32_t e = my_e[j];
            const uint32_t pos = base[e] + cnt[i / 64][e] + rank_in_chunk[i];
            sorted[pos] = {i / k, e, i % k, (uint32_t)my_w[j]};
        }
    }
}

// The grouped GEMMs run each 128-row grouping tile as two 64-row halves
// (blockIdx.x = 2·tile + half) on the projection tile of gemm.hpp, so an
// expert with few rows costs one half's matrix work, not a full tile's.
// Returns false for a half with no rows (block-uniform).
struct GroupedRows {
    uint32_t first;   // index of the half's first row in the sorted pairs
    uint32_t count;   // rows in this half (1..64)
    uint32_t expert;
};

__device__ __forceinline__ bool grouped_rows(const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                             GroupedRows& gr) {
    const uint32_t tile = blockIdx.x >> 1, half = blockIdx.x & 1u;
    if (tile >= *n_tiles) return false;
    const Tile t = tiles[tile];
    if (t.count <= kProjBM * half) return false;
    const uint32_t left = t.count - kProjBM * half;
    gr = {t.start + kProjBM * half, left < kProjBM ? left : kProjBM, t.expert};
    return true;
}

// Grouped gate/up + GeGLU over one 64-row half tile (blockIdx.x) and 128
// features of F (blockIdx.y): act[p][f] = fp16(gelu(gate_e[f]·x_p) · (up_e[f]·x_p))
// for sorted pairs p of the half, x_p = hidden row of the pair's token
// (prefill.metal:598-637). Wave w takes features f0 + 32w .. +31 with the gate
// rows as its first 32-output sub-tile and the up rows as its second, so each
// lane holds gate and up of the same (pair, feature) and applies the GeGLU
// in registers. LDS table rows 0..127: gate scales/biases, 128..255: up.
// BITS: code width of the expert rows (2, 3 or 4; prefill.metal:1304-1450
// for the 2/3-bit experts).
template <int BITS = 4>
__device__ __forceinline__ void moe_grouped_gate_up(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                    const Tile* __restrict__ tiles,
                                                    const uint32_t* __restrict__ n_tiles,
                                                    const uint16_t* __restrict__ hidden, uint32_t stride,
                                                    uint16_t* __restrict__ act, uint32_t D, uint32_t F) {
    GroupedRows gr;
    if (!grouped_rows(tiles, n_tiles, gr)) return;
    extern __shared__ __attribute__((aligned(16))) _Float16 proj_lds[];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t G = D >> 6, f0 = blockIdx.y * 128u;
    const uint8_t* blob = pool.base + (uint64_t)gr.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    const uint16_t* gs = reinterpret_cast<const uint16_t*>(blob + o.gate_s);
    const uint16_t* gb = reinterpret_cast<const uint16_t*>(blob + o.gate_b);
    const uint16_t* us = reinterpret_cast<const uint16_t*>(blob + o.up_s);
    const uint16_t* ub = reinterpret_cast<const uint16_t*>(blob + o.up_b);
    uint16_t* s_lds = reinterpret_cast<uint16_t*>(proj_lds + 2 * kProjBM * kGemmLdsStride);
    uint16_t* b_lds = s_lds + kProjBN * G;
    const uint32_t nf = F - f0 < 128u ? F - f0 : 128u;
    copy_pair_to_lds<kProjThreads>(gs + (size_t)f0 * G, gb + (size_t)f0 * G, s_lds, b_lds, nf * G);
    copy_pair_to_lds<kProjThreads>(us + (size_t)f0 * G, ub + (size_t)f0 * G, s_lds + 128u * G, b_lds + 128u * G,
                                   nf * G);
    const uint32_t col = lane & 31u, h = lane >> 5;
    const uint32_t f = f0 + 32u * wave + col, fc = f < F ? f : F - 1;   // features past F: clamped, not stored
    ProjLanes pl;
    pl.wp0 = blob + o.gate_w + (size_t)fc * ((D >> 3) * BITS) + 4u * BITS * h;
    pl.wp1 = blob + o.up_w + (size_t)fc * ((D >> 3) * BITS) + 4u * BITS * h;
    pl.sidx0 = (fc - f0) * G;
    pl.sidx1 = (128u + fc - f0) * G;
    // rows past the half's count read its first row: their results are never stored
    const uint32_t xrow = tid >> 2;
    const uint32_t tok = sorted[gr.first + (xrow < gr.count ? xrow : 0u)].token;
    const uint16_t* xp = hidden + (size_t)tok * stride + 16u * (tid & 3u);
    // a half with at most 32 rows runs one token sub-tile (block-uniform)
    auto run = [&](auto mi_c) {
        constexpr int MI = decltype(mi_c)::value;
        f32x16 acc[MI][2];
        proj_core<false, MI, BITS>(acc, proj_lds, s_lds, b_lds, pl, xp, G);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = 32u * i + 8u * (r >> 2) + 4u * h + (r & 3);
                if (m < gr.count && f < F)
                    act[(size_t)(gr.first + m) * F + f] = f2h(gelu_tanh(acc[i][0][r]) * acc[i][1][r]);
            }
    };
    if (gr.count <= 32u) run(std::integral_constant<int, 1>{});
    else run(std::integral_constant<int, 2>{});
}

// Grouped down projection over one 64-row half tile (blockIdx.x) and 256
// outputs of D (blockIdx.y): partials[(token*k + rank)*D + d] = fp16(down_e[d]·act_p)
// (prefill.metal:639-670). BITS as for moe_grouped_gate_up.
template <int BITS = 4>
__device__ __forceinline__ void moe_grouped_down(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                 const Tile* __restrict__ tiles,
                                                 const uint32_t* __restrict__ n_tiles,
                                                 const uint16_t* __restrict__ act, uint16_t* __restrict__ partials,
                                                 uint32_t D, uint32_t F, uint32_t k) {
    GroupedRows gr;
    if (!grouped_rows(tiles, n_tiles, gr)) return;
    extern __shared__ __attribute__((aligned(16))) _Float16 proj_lds[];
    __shared__ uint32_t dst_row[kProjBM];
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    const uint32_t G = F >> 6, n0 = blockIdx.y * kProjBN;
    const uint8_t* blob = pool.base + (uint64_t)gr.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    uint16_t* s_lds = reinterpret_cast<uint16_t*>(proj_lds + 2 * kProjBM * kGemmLdsStride);
    uint16_t* b_lds = s_lds + kProjBN * G;
    if (tid < gr.count) {
        const Pair p = sorted[gr.first + tid];
        dst_row[tid] = p.token * k + p.rank;
    }
    const uint32_t nrows = D - n0 < kProjBN ? D - n0 : kProjBN;
    copy_pair_to_lds<kProjThreads>(reinterpret_cast<const uint16_t*>(blob + o.down_s) + (size_t)n0 * G,
                                   reinterpret_cast<const uint16_t*>(blob + o.down_b) + (size_t)n0 * G, s_lds,
                                   b_lds, nrows * G);
    const ProjLanes pl = proj_lanes<2, BITS>(blob + o.down_w, (F >> 3) * BITS, n0, wave, D, 0, G);
    const uint32_t xrow = tid >> 2;
    const uint16_t* xp = act + (size_t)(gr.first + (xrow < gr.count ? xrow : 0u)) * F + 16u * (tid & 3u);
    // a half with at most 32 rows runs one token sub-tile (block-uniform)
    auto run = [&](auto mi_c) {
        constexpr int MI = decltype(mi_c)::value;
        f32x16 acc[MI][2];
        proj_core<false, MI, BITS>(acc, proj_lds, s_lds, b_lds, pl, xp, G);   // its barriers publish dst_row
        proj_for_each<2>(acc, [&](uint32_t m, uint32_t n, float v) {
            if (m < gr.count && n0 + n < D) partials[(size_t)dst_row[m] * D + n0 + n] = f2h(v);
        });
    };
    if (gr.count <= 32u) run(std::integral_constant<int, 1>{});
    else run(std::integral_constant<int, 2>{});
}

// h2[t][d] = fp16(Σ_r fma(w[t][r], partials[(t*k+r)*D + d])) in rank order
// (prefill.metal:575-596). Grid: (ceil(D/256), T).
__device__ __forceinline__ void moe_combine(const uint16_t* __restrict__ partials,
                                            const uint16_t* __restrict__ w, uint16_t* __restrict__ h2,
                                            uint32_t T, uint32_t k, uint32_t D) {
    const uint32_t d = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t t = blockIdx.y;
    if (t >= T || d >= D) return;
    float acc = 0.0f;
    for (uint32_t r = 0; r < k; ++r)
        acc = fmaf(h2f(w[t * k + r]), h2f(partials[((size_t)t * k + r) * D + d]), acc);
    h2[(size_t)t * D + d] = f2h(acc);
}

}  // namespace tfq
