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
// Here the pairs never leave the device and every expert's rows become one
// or more 128-row MFMA tiles.
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

// Grouped gate/up + GeGLU over one expert tile (blockIdx.x) and 128 outputs of
// F (blockIdx.y): act[p][f] = fp16(gelu(gate_e[f]·x_p) · (up_e[f]·x_p)) for
// sorted pairs p of the tile, x_p = hidden row of the pair's token
// (prefill.metal:598-637).
__device__ __forceinline__ void moe_grouped_gate_up(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                    const Tile* __restrict__ tiles,
                                                    const uint32_t* __restrict__ n_tiles,
                                                    const uint16_t* __restrict__ hidden, uint32_t stride,
                                                    uint16_t* __restrict__ act, uint32_t D, uint32_t F) {
    if (blockIdx.x >= *n_tiles) return;                  // block-uniform
    __shared__ __attribute__((aligned(16))) GemmLds<2> L;
    __shared__ const uint16_t* rows_ptr[kGemmBM];
    const Tile t = tiles[blockIdx.x];
    if (threadIdx.x < t.count)
        rows_ptr[threadIdx.x] = hidden + (size_t)sorted[t.start + threadIdx.x].token * stride;
    __syncthreads();
    const uint8_t* blob = pool.base + (uint64_t)t.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    const Q4Tile mats[2] = {
        {blob + o.gate_w, reinterpret_cast<const uint16_t*>(blob + o.gate_s),
         reinterpret_cast<const uint16_t*>(blob + o.gate_b)},
        {blob + o.up_w, reinterpret_cast<const uint16_t*>(blob + o.up_s),
         reinterpret_cast<const uint16_t*>(blob + o.up_b)}};
    gemm_tile<false, 2>(L, rows_ptr, t.count, mats, blockIdx.y * kGemmBN, F, D,
                        [&](uint32_t j, uint32_t f, const float* v) {
                            act[(size_t)(t.start + j) * F + f] = f2h(gelu_tanh(v[0]) * v[1]);
                        });
}

// Grouped down projection over one expert tile (blockIdx.x) and 128 outputs of
// D (blockIdx.y): partials[(token*k + rank)*D + d] = fp16(down_e[d]·act_p)
// (prefill.metal:639-670).
__device__ __forceinline__ void moe_grouped_down(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                 const Tile* __restrict__ tiles,
                                                 const uint32_t* __restrict__ n_tiles,
                                                 const uint16_t* __restrict__ act, uint16_t* __restrict__ partials,
                                                 uint32_t D, uint32_t F, uint32_t k) {
    if (blockIdx.x >= *n_tiles) return;
    __shared__ __attribute__((aligned(16))) GemmLds<1> L;
    __shared__ const uint16_t* rows_ptr[kGemmBM];
    __shared__ uint32_t dst_row[kGemmBM];
    const Tile t = tiles[blockIdx.x];
    if (threadIdx.x < t.count) {
        const Pair p = sorted[t.start + threadIdx.x];
        rows_ptr[threadIdx.x] = act + (size_t)(t.start + threadIdx.x) * F;
        dst_row[threadIdx.x] = p.token * k + p.rank;
    }
    __syncthreads();
    const uint8_t* blob = pool.base + (uint64_t)t.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    const Q4Tile mats[1] = {{blob + o.down_w, reinterpret_cast<const uint16_t*>(blob + o.down_s),
                             reinterpret_cast<const uint16_t*>(blob + o.down_b)}};
    gemm_tile<false, 1>(L, rows_ptr, t.count, mats, blockIdx.y * kGemmBN, D, F,
                        [&](uint32_t j, uint32_t d, const float* v) {
                            partials[(size_t)dst_row[j] * D + d] = f2h(v[0]);
                        });
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
