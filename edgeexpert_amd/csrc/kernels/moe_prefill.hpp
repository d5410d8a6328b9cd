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
#include "gemm_skinny.hpp"
#include "gemv.hpp"

namespace tfq {

constexpr uint32_t kGroupMaxPairs = 8192;
constexpr uint32_t kGroupMaxExperts = 256;
constexpr uint32_t kGroupChunks = kGroupMaxPairs / 64;
constexpr uint32_t kGroupThreads = 1024;
// status codes (the PrefillMoEGroupingError cases the device can detect)
constexpr uint32_t kGroupOk = 0;
constexpr uint32_t kGroupExpertOutOfRange = 8;
// grouping tiles of at most kGroupStreamMax pairs run as a weight stream
// (moe_stream_*), larger ones on the matrix-core tile (moe_grouped_*)
constexpr uint32_t kGroupStreamMax = 32;
constexpr uint32_t kGroupStreamThreads = 256;  // 4 wavefronts, 64 weight rows each
constexpr uint32_t kGroupStreamRows = 64 * (kGroupStreamThreads / 64);   // rows per block

// dst[n + e] = fp16(v[e]) for e < 4 and n + e < lim: one 8-byte store when
// all four are in range and dst + n is 8-byte aligned, else per element.
__device__ __forceinline__ void store_f16x4(uint16_t* __restrict__ dst, uint32_t n, uint32_t lim, const float (&v)[4]) {
    const uint16_t o0 = f2h(v[0]), o1 = f2h(v[1]), o2 = f2h(v[2]), o3 = f2h(v[3]);
    if (n + 3 < lim && ((reinterpret_cast<uintptr_t>(dst + n) & 7u) == 0)) {
        *reinterpret_cast<uint2*>(dst + n) =
            make_uint2((uint32_t)o0 | ((uint32_t)o1 << 16), (uint32_t)o2 | ((uint32_t)o3 << 16));
    } else {
        const uint16_t o[4] = {o0, o1, o2, o3};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < lim) dst[n + e] = o[e];
    }
}

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
// (block x = 2·tile + half) on the projection tile of gemm.hpp, so an
// expert with few rows costs one half's matrix work, not a full tile's.
// Returns false for a half with no rows (block-uniform).
struct GroupedRows {
    uint32_t first;   // index of the half's first row in the sorted pairs
    uint32_t count;   // rows in this half (1..64)
    uint32_t expert;
};

__device__ __forceinline__ bool grouped_rows(const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                             uint32_t bx, GroupedRows& gr) {
    const uint32_t tile = bx >> 1, half = bx & 1u;
    if (tile >= *n_tiles) return false;
    const Tile t = tiles[tile];
    if (t.count <= kGroupStreamMax || t.count <= kProjBM * half) return false;   // small tiles: the stream
    const uint32_t left = t.count - kProjBM * half;
    gr = {t.start + kProjBM * half, left < kProjBM ? left : kProjBM, t.expert};
    return true;
}

// Grouped gate/up + GeGLU over one 64-row half tile (block x) and 128
// features of F (block y): act[p][f] = fp16(gelu(gate_e[f]·x_p) · (up_e[f]·x_p))
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
                                                    uint16_t* __restrict__ act, uint32_t D, uint32_t F, uint32_t bx,
                                                    uint32_t by) {
    GroupedRows gr;
    if (!grouped_rows(tiles, n_tiles, bx, gr)) return;
    extern __shared__ __attribute__((aligned(16))) _Float16 proj_lds[];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t G = D >> 6, f0 = by * 128u;
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

// Grouped down projection over one 64-row half tile (block x) and 256
// outputs of D (block y): partials[(token*k + rank)*D + d] = fp16(down_e[d]·act_p)
// (prefill.metal:639-670). BITS as for moe_grouped_gate_up.
template <int BITS = 4>
__device__ __forceinline__ void moe_grouped_down(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                 const Tile* __restrict__ tiles,
                                                 const uint32_t* __restrict__ n_tiles,
                                                 const uint16_t* __restrict__ act, uint16_t* __restrict__ partials,
                                                 uint32_t D, uint32_t F, uint32_t k, uint32_t bx, uint32_t by) {
    GroupedRows gr;
    if (!grouped_rows(tiles, n_tiles, bx, gr)) return;
    extern __shared__ __attribute__((aligned(16))) _Float16 proj_lds[];
    __shared__ uint32_t dst_row[kProjBM];
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    const uint32_t G = F >> 6, n0 = by * kProjBN;
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

// ------------------------------------------- weight stream for small tiles ----
//
// Under a skewed popularity most experts see a handful of tokens (config 3:
// 101 of 128 experts take at most 32 of the 4096 pairs, yet hold 80% of the
// active weights). On the matrix-core tile such an expert costs a 64-row
// half of MFMA work and the tile's per-group barriers for a few rows; the
// work is a weight stream instead. A grouping tile with at most
// kGroupStreamMax pairs is skipped by the two kernels above and run here:
// each wavefront owns 64 weight rows (four 16-row v_mfma_f32_16x16x32_f16
// A operands) and the whole K loop, the pairs as one or two 16-token B
// operands (NTT), so every activation load feeds four row tiles. Lane l
// holds row l%16 of each A operand and the quarter q = l/16 of every
// 128-code k-tile (chunk 4m + q: one 16-byte load at 4 bits, word j feeds
// k-step j), the B lane (pair l%16 of the sub-tile, quarter q) the matching
// 32 activations, permuted like the unpack. The block's scales and biases
// sit in an LDS table (one word per row and group), so the loop issues only
// 16-byte loads. Weights are dequantised as everywhere else (fp16(q·s + b),
// one rounding), so the result differs from the tile's only in the fp32
// summation order. DEPTH k-tiles are in flight per wave.

template <int BITS, int NTT>
struct StreamStage {
    QChunk<BITS> w[4];
    uint4 x[NTT][4];
};

// acc[i][j]: 16x16 D tile of row tile i and token sub-tile j (column =
// lane % 16 = token, rows 4·(lane/16) + r). sbt[i]: the LDS table row
// (scale | bias << 16 per group) of this lane's row in tile i, published by
// the barrier that `publish` runs once the first DEPTH k-tiles' loads are in
// flight.
template <int BITS, int NTT, typename Publish, int DEPTH = (NTT == 1 ? 3 : 2)>
__device__ __forceinline__ void stream_rows(const uint8_t* const (&wrow)[4], const uint32_t* const (&sbt)[4],
                                            const uint16_t* const (&xrow)[NTT], uint32_t K, f32x4 (&acc)[4][NTT],
                                            Publish publish) {
    const uint32_t q = (threadIdx.x & 63u) >> 4;
    const uint32_t nch = K >> 5;                       // 32-code chunks per row
    const uint32_t nk = (nch + 3u) >> 2;               // 128-code k-tiles
    uint32_t magic_v;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic_v));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NTT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // k-tiles past the end re-read the last chunk (and are not computed);
    // the missing quarters of a half-filled last k-tile are masked to zero
    auto load = [&](uint32_t m, StreamStage<BITS, NTT>& st) {
        const uint32_t c = 4u * m + q, cc = c < nch ? c : nch - 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) st.w[i] = ldg_chunk<BITS, false>(wrow[i], cc);
#pragma unroll
        for (int j = 0; j < NTT; ++j) {
            const uint4* xp = reinterpret_cast<const uint4*>(xrow[j] + 32u * cc);
#pragma unroll
            for (int u = 0; u < 4; ++u) st.x[j][u] = xp[u];
        }
    };
    auto compute = [&](uint32_t m, const StreamStage<BITS, NTT>& st, auto mask_c) {
        constexpr bool MASK = decltype(mask_c)::value;
        const uint32_t c = 4u * m + q, g = (c < nch ? c : nch - 1) >> 1;
        const uint32_t mask = MASK && c >= nch ? 0u : 0xFFFFFFFFu;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h8 a[4];
            dequant_chunk_sb(st.w[i], sbt[i][g], magic_v, a);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const h8 ai = MASK ? mask_h8(a[u], mask) : a[u];
#pragma unroll
                for (int j = 0; j < NTT; ++j) {
                    const h8 bj = perm_0415(__builtin_bit_cast(h8, st.x[j][u]));
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ai, MASK ? mask_h8(bj, mask) : bj, acc[i][j],
                                                                       0, 0, 0);
                }
            }
        }
    };
    // the last k-tile is masked when K is not a multiple of 128 codes
    const uint32_t nfull = (nch & 3u) ? nk - 1 : nk;
    StreamStage<BITS, NTT> st[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load((uint32_t)d, st[d]);
    publish();
    uint32_t m = 0;
    for (; m + DEPTH <= nfull; m += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            compute(m + (uint32_t)d, st[d], std::false_type{});
            load(m + (uint32_t)(d + DEPTH), st[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        const uint32_t mm = m + (uint32_t)d;
        if (mm < nfull) compute(mm, st[d], std::false_type{});
        else if (mm < nk) compute(mm, st[d], std::true_type{});
    }
}

// Grouping tile `by` if it takes the weight stream (block-uniform).
__device__ __forceinline__ bool stream_tile(const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                            uint32_t by, Tile& t) {
    if (by >= *n_tiles) return false;
    t = tiles[by];
    return t.count > 0 && t.count <= kGroupStreamMax;
}

// Dynamic LDS of the stream kernels: the scale/bias table of a block's
// kGroupStreamRows rows (gate/up: the gate rows, then the up rows).
constexpr uint32_t stream_lds_bytes(uint32_t K) { return 4u * kGroupStreamRows * (K / 64u); }

// Gate/up + GeGLU of one small tile (block y) over kGroupStreamRows/2
// features (block x): wave w takes features f = f_blk + 32w + (0..31),
// its gate rows as row tiles 0, 1 and its up rows as row tiles 2, 3, so each
// lane holds gate and up of the same (pair, feature).
template <int BITS, int NTT>
__device__ __forceinline__ void stream_gate_up_tile(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                    const Tile& t, const uint16_t* __restrict__ hidden,
                                                    uint32_t stride, uint16_t* __restrict__ act, uint32_t D,
                                                    uint32_t F, uint32_t bx) {
    extern __shared__ __attribute__((aligned(16))) uint32_t stream_sb[];
    constexpr uint32_t NF = kGroupStreamRows / 2u;                       // features per block
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t G = D >> 6, row_bytes = (D >> 3) * BITS;
    const uint32_t f_blk = bx * NF;
    const uint32_t fb = f_blk + 32u * wave;
    const uint8_t* blob = pool.base + (uint64_t)t.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    const uint8_t* wrow[4];
    const uint32_t* sbt[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t f = fb + 16u * i + r16, fc = f < F ? f : F - 1;   // features past F: clamped, not stored
        wrow[i] = blob + o.gate_w + (size_t)fc * row_bytes;
        wrow[2 + i] = blob + o.up_w + (size_t)fc * row_bytes;
        sbt[i] = stream_sb + (fc - f_blk) * G;
        sbt[2 + i] = stream_sb + (NF + fc - f_blk) * G;
    }
    const uint16_t* xrow[NTT];
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;                                // pairs past the tile: row 0, not stored
        xrow[j] = hidden + (size_t)sorted[t.start + (p < t.count ? p : 0u)].token * stride;
    }
    f32x4 acc[4][NTT];
    stream_rows<BITS, NTT>(wrow, sbt, xrow, D, acc, [&]() {
        const uint32_t nf = F - f_blk < NF ? F - f_blk : NF;
        copy_sb_to_lds<kGroupStreamThreads, 2>(reinterpret_cast<const uint16_t*>(blob + o.gate_s) + (size_t)f_blk * G,
                                               reinterpret_cast<const uint16_t*>(blob + o.gate_b) + (size_t)f_blk * G,
                                               stream_sb, nf * G);
        copy_sb_to_lds<kGroupStreamThreads, 2>(reinterpret_cast<const uint16_t*>(blob + o.up_s) + (size_t)f_blk * G,
                                               reinterpret_cast<const uint16_t*>(blob + o.up_b) + (size_t)f_blk * G,
                                               stream_sb + NF * G, nf * G);
        __syncthreads();
    });
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        if (p >= t.count) continue;
        uint16_t* dst = act + (size_t)(t.start + p) * F;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = gelu_tanh(acc[i][j][r]) * acc[2 + i][j][r];
            store_f16x4(dst, fb + 16u * i + 4u * q, F, v);
        }
    }
}

// Down projection of one small tile (block y) over kGroupStreamRows
// outputs of D (block x): wave w takes rows d = d_blk + 64w + (0..63).
template <int BITS, int NTT>
__device__ __forceinline__ void stream_down_tile(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                 const Tile& t, const uint16_t* __restrict__ act,
                                                 uint16_t* __restrict__ partials, uint32_t D, uint32_t F,
                                                 uint32_t k, uint32_t bx) {
    extern __shared__ __attribute__((aligned(16))) uint32_t stream_sb[];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t G = F >> 6, row_bytes = (F >> 3) * BITS;
    const uint32_t d_blk = bx * kGroupStreamRows;
    const uint32_t db = d_blk + 64u * wave;
    const uint8_t* blob = pool.base + (uint64_t)t.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    const uint8_t* wrow[4];
    const uint32_t* sbt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = db + 16u * i + r16, dc = d < D ? d : D - 1;   // rows past D: clamped, not stored
        wrow[i] = blob + o.down_w + (size_t)dc * row_bytes;
        sbt[i] = stream_sb + (dc - d_blk) * G;
    }
    const uint16_t* xrow[NTT];
    uint32_t dst_row[NTT];          // partials row of each pair, loaded before the K loop
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16, pc = p < t.count ? p : 0u;
        xrow[j] = act + (size_t)(t.start + pc) * F;
        const Pair pr = sorted[t.start + pc];
        dst_row[j] = pr.token * k + pr.rank;
    }
    f32x4 acc[4][NTT];
    stream_rows<BITS, NTT>(wrow, sbt, xrow, F, acc, [&]() {
        const uint32_t nd = D - d_blk < kGroupStreamRows ? D - d_blk : kGroupStreamRows;
        copy_sb_to_lds<kGroupStreamThreads, 2>(reinterpret_cast<const uint16_t*>(blob + o.down_s) + (size_t)d_blk * G,
                                               reinterpret_cast<const uint16_t*>(blob + o.down_b) + (size_t)d_blk * G,
                                               stream_sb, nd * G);
        __syncthreads();
    });
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        if (p >= t.count) continue;
        uint16_t* dst = partials + (size_t)dst_row[j] * D;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            store_f16x4(dst, db + 16u * i + 4u * q, D, v);
        }
    }
}

template <int BITS>
__device__ __forceinline__ void moe_stream_gate_up(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                   const Tile* __restrict__ tiles,
                                                   const uint32_t* __restrict__ n_tiles,
                                                   const uint16_t* __restrict__ hidden, uint32_t stride,
                                                   uint16_t* __restrict__ act, uint32_t D, uint32_t F, uint32_t bx,
                                                   uint32_t by) {
    Tile t;
    if (!stream_tile(tiles, n_tiles, by, t)) return;
    if (t.count <= 16u) stream_gate_up_tile<BITS, 1>(pool, sorted, t, hidden, stride, act, D, F, bx);
    else stream_gate_up_tile<BITS, 2>(pool, sorted, t, hidden, stride, act, D, F, bx);
}

template <int BITS>
__device__ __forceinline__ void moe_stream_down(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                                const uint16_t* __restrict__ act, uint16_t* __restrict__ partials,
                                                uint32_t D, uint32_t F, uint32_t k, uint32_t bx, uint32_t by) {
    Tile t;
    if (!stream_tile(tiles, n_tiles, by, t)) return;
    if (t.count <= 16u) stream_down_tile<BITS, 1>(pool, sorted, t, act, partials, D, F, k, bx);
    else stream_down_tile<BITS, 2>(pool, sorted, t, act, partials, D, F, k, bx);
}

// ----------------------------------------------- wide role for large tiles ----
//
// A grouping tile of more than kGroupStreamMax pairs runs as 64-pair halves
// (block y = 2·tile + half), each block over kGroupWideRows weight rows
// (block x): gate/up 64 features (gate and up rows), down 128 outputs. Wave
// w owns 32 rows as two 16-row A operands of v_mfma_f32_16x16x32_f16 (lane
// l: row l%16, the quarter q = l/16 of every 128-code k-tile, chunk 4m + q
// from a DEPTH-deep register ring, dequantised exactly as in the stream);
// the half's activations (NTT 16-pair sub-tiles) are staged per k-tile into
// a double-buffered LDS tile [64 pairs][128 codes + 8] in the unpack order,
// from a two-deep register ring, one barrier per k-tile; the B lane (pair
// l%16 of sub-tile j, quarter q) reads its 16 bytes of k-step u at column
// 32q + 8u. Codes past K (a half-filled last k-tile) are zero in both
// operands. Per k-tile a wave issues 8·NTT MFMAs and dequantises 64 codes
// per lane.
template <int B, int E, typename Fn>
__device__ __forceinline__ void sfor_w(Fn&& f) {             // f(integral_constant<B>) ... f(<E-1>)
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        sfor_w<B + 1, E>(f);
    }
}

constexpr uint32_t kGroupWideRows = 128;                  // weight rows per block (4 waves x 32)
constexpr uint32_t kGroupWidePairs = 64;                  // pairs per block (a half tile)
constexpr uint32_t kWideStride = 128 + 8;                 // halves per LDS activation row
constexpr uint32_t kWideBuf = kGroupWidePairs * kWideStride;   // halves per activation buffer
// Dynamic LDS of the wide role: two activation buffers, then the scale/bias
// table of the block's rows.
constexpr uint32_t wide_lds_bytes(uint32_t K) { return 2u * kWideBuf * 2u + 4u * kGroupWideRows * (K / 64u); }

// Rows of half `by` of a large tile (false: nothing to do; block-uniform).
__device__ __forceinline__ bool wide_rows(const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                          uint32_t by, GroupedRows& gr) {
    const uint32_t tile = by >> 1, half = by & 1u;
    if (tile >= *n_tiles) return false;
    const Tile t = tiles[tile];
    if (t.count <= kGroupStreamMax || t.count <= kGroupWidePairs * half) return false;
    const uint32_t left = t.count - kGroupWidePairs * half;
    gr = {t.start + kGroupWidePairs * half, left < kGroupWidePairs ? left : kGroupWidePairs, t.expert};
    return true;
}

// acc[i][j]: row tile i, pair sub-tile j (16x16 D layout). xrow(p): the
// activation row of pair p (< NTT·16; past the half's count: any valid row,
// not stored). sbt[i]: this lane's row of the scale/bias table.
template <int BITS, int NTT, typename XRow, typename Publish, int DEPTH = 3>
__device__ __forceinline__ void wide_rows_loop(const uint8_t* const (&wrow)[2], const uint32_t* const (&sbt)[2],
                                               XRow xrow, uint32_t K, _Float16* __restrict__ xs,
                                               f32x4 (&acc)[2][NTT], Publish publish) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, q = lane >> 4, r16 = lane & 15u;
    const uint32_t nch = K >> 5, nk = (nch + 3u) >> 2;
    constexpr uint32_t NP = NTT * 16u;                     // staged pairs
    constexpr uint32_t PIECES = NP * 16u / kGroupStreamThreads;   // 16-byte activation pieces per thread
    uint32_t magic_v;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic_v));
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NTT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // activation piece p of this thread: pair (p·256 + tid) / 16, 16-byte column (tid % 16)
    const uint16_t* xr_row[PIECES];
#pragma unroll
    for (uint32_t p = 0; p < PIECES; ++p) xr_row[p] = xrow((p * kGroupStreamThreads + tid) >> 4);
    const uint32_t xcol = tid & 15u;
    QChunk<BITS> wr[DEPTH][2];
    uint4 xr[2][PIECES];
    auto load_w = [&](uint32_t m, QChunk<BITS> (&dst)[2]) {
        const uint32_t c = 4u * m + q, cc = c < nch ? c : nch - 1;
#pragma unroll
        for (int i = 0; i < 2; ++i) dst[i] = ldg_chunk<BITS, false>(wrow[i], cc);
    };
    // columns past K load a valid piece and are stored as zeros
    auto load_x = [&](uint32_t m, uint4 (&dst)[PIECES]) {
        const uint32_t col = 128u * (m < nk ? m : nk - 1) + 8u * xcol;
        const uint32_t cc = col < K ? col : 0u;
#pragma unroll
        for (uint32_t p = 0; p < PIECES; ++p) dst[p] = *reinterpret_cast<const uint4*>(xr_row[p] + cc);
    };
    auto store_x = [&](uint32_t m, const uint4 (&src)[PIECES], _Float16* buf) {
        const bool live = 128u * m + 8u * xcol < K;
#pragma unroll
        for (uint32_t p = 0; p < PIECES; ++p) {
            const uint32_t pr = (p * kGroupStreamThreads + tid) >> 4;
            const h8 v = live ? perm_0415(__builtin_bit_cast(h8, src[p])) : h8{};
            *reinterpret_cast<h8*>(buf + pr * kWideStride + 8u * xcol) = v;
        }
    };
    auto compute = [&](uint32_t m, const QChunk<BITS> (&w)[2], const _Float16* buf) {
        const uint32_t c = 4u * m + q, g = (c < nch ? c : nch - 1) >> 1;
        const uint32_t mask = c < nch ? 0xFFFFFFFFu : 0u;
        h8 a[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            dequant_chunk_sb(w[i], sbt[i][g], magic_v, a[i]);
#pragma unroll
            for (int u = 0; u < 4; ++u) a[i][u] = mask_h8(a[i][u], mask);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < NTT; ++j) {
                const h8 b = *reinterpret_cast<const h8*>(buf + (16u * j + r16) * kWideStride + 32u * q + 8u * u);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i][u], b, acc[i][j], 0, 0, 0);
            }
    };

    // prologue: weights of k-tiles 0..DEPTH-1, activations of 0 and 1; stage 0
    load_x(0, xr[0]);
    load_x(1, xr[1]);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load_w((uint32_t)d, wr[d]);
    publish();                                   // the scale/bias table (ends with a barrier)
    store_x(0, xr[0], xs);
    load_x(2, xr[0]);
    __syncthreads();
    // step m: k-tile m from buffer m%2 and ring stage m%DEPTH; stage k-tile
    // m+1 into the other buffer; refill the rings (weights m+DEPTH,
    // activations m+3)
    auto step = [&](uint32_t m, auto st_c, auto pa_c) {
        constexpr int ST = decltype(st_c)::value, PA = decltype(pa_c)::value;
        compute(m, wr[ST], xs + PA * kWideBuf);
        store_x(m + 1, xr[PA ^ 1], xs + (PA ^ 1) * kWideBuf);
        load_w(m + DEPTH, wr[ST]);
        load_x(m + 3, xr[PA ^ 1]);
        __syncthreads();
    };
    constexpr int U = DEPTH * 2;                 // steps per unrolled run (ring stage and buffer parity)
    uint32_t m = 0;
    for (; m + U <= nk; m += U)
        sfor_w<0, U>([&](auto c) {
            step(m + c.value, std::integral_constant<int, c.value % DEPTH>{}, std::integral_constant<int, c.value & 1>{});
        });
    sfor_w<0, U - 1>([&](auto c) {
        if (m + c.value < nk)
            step(m + c.value, std::integral_constant<int, c.value % DEPTH>{}, std::integral_constant<int, c.value & 1>{});
    });
}

// Gate/up + GeGLU of one large-tile half (block y) over 64 features (block
// x): wave w takes features f_blk + 16w + (0..15), its gate rows as row tile
// 0 and its up rows as row tile 1.
template <int BITS, int NTT>
__device__ __forceinline__ void wide_gate_up_half(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                  const GroupedRows& gr, const uint16_t* __restrict__ hidden,
                                                  uint32_t stride, uint16_t* __restrict__ act, uint32_t D, uint32_t F,
                                                  uint32_t bx) {
    extern __shared__ __attribute__((aligned(16))) _Float16 wide_lds[];
    constexpr uint32_t NF = kGroupWideRows / 2u;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t G = D >> 6, row_bytes = (D >> 3) * BITS;
    const uint32_t f_blk = bx * NF, fb = f_blk + 16u * wave;
    const uint32_t f = fb + r16, fc = f < F ? f : F - 1;                 // features past F: clamped, not stored
    const uint8_t* blob = pool.base + (uint64_t)gr.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    uint32_t* sb_lds = reinterpret_cast<uint32_t*>(wide_lds + 2u * kWideBuf);
    const uint8_t* const wrow[2] = {blob + o.gate_w + (size_t)fc * row_bytes, blob + o.up_w + (size_t)fc * row_bytes};
    const uint32_t* const sbt[2] = {sb_lds + (fc - f_blk) * G, sb_lds + (NF + fc - f_blk) * G};
    f32x4 acc[2][NTT];
    wide_rows_loop<BITS, NTT>(
        wrow, sbt,
        [&](uint32_t p) { return hidden + (size_t)sorted[gr.first + (p < gr.count ? p : 0u)].token * stride; }, D,
        wide_lds, acc, [&]() {
            const uint32_t nf = F - f_blk < NF ? F - f_blk : NF;
            copy_sb_to_lds<kGroupStreamThreads, 2>(reinterpret_cast<const uint16_t*>(blob + o.gate_s) + (size_t)f_blk * G,
                                                   reinterpret_cast<const uint16_t*>(blob + o.gate_b) + (size_t)f_blk * G,
                                                   sb_lds, nf * G);
            copy_sb_to_lds<kGroupStreamThreads, 2>(reinterpret_cast<const uint16_t*>(blob + o.up_s) + (size_t)f_blk * G,
                                                   reinterpret_cast<const uint16_t*>(blob + o.up_b) + (size_t)f_blk * G,
                                                   sb_lds + NF * G, nf * G);
            __syncthreads();
        });
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        if (p >= gr.count) continue;
        uint16_t* dst = act + (size_t)(gr.first + p) * F;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = gelu_tanh(acc[0][j][r]) * acc[1][j][r];
        store_f16x4(dst, fb + 4u * q, F, v);
    }
}

// Down projection of one large-tile half (block y) over 128 outputs of D
// (block x): wave w takes rows d_blk + 32w + (0..31).
template <int BITS, int NTT>
__device__ __forceinline__ void wide_down_half(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                               const GroupedRows& gr, const uint16_t* __restrict__ act,
                                               uint16_t* __restrict__ partials, uint32_t D, uint32_t F, uint32_t k,
                                               uint32_t bx) {
    extern __shared__ __attribute__((aligned(16))) _Float16 wide_lds[];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t G = F >> 6, row_bytes = (F >> 3) * BITS;
    const uint32_t d_blk = bx * kGroupWideRows, db = d_blk + 32u * wave;
    const uint8_t* blob = pool.base + (uint64_t)gr.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    uint32_t* sb_lds = reinterpret_cast<uint32_t*>(wide_lds + 2u * kWideBuf);
    const uint8_t* wrow[2];
    const uint32_t* sbt[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t d = db + 16u * i + r16, dc = d < D ? d : D - 1;   // rows past D: clamped, not stored
        wrow[i] = blob + o.down_w + (size_t)dc * row_bytes;
        sbt[i] = sb_lds + (dc - d_blk) * G;
    }
    uint32_t dst_row[NTT];          // partials row of each pair, loaded before the K loop
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        const Pair pr = sorted[gr.first + (p < gr.count ? p : 0u)];
        dst_row[j] = pr.token * k + pr.rank;
    }
    f32x4 acc[2][NTT];
    wide_rows_loop<BITS, NTT>(
        wrow, sbt, [&](uint32_t p) { return act + (size_t)(gr.first + (p < gr.count ? p : 0u)) * F; }, F, wide_lds, acc,
        [&]() {
            const uint32_t nd = D - d_blk < kGroupWideRows ? D - d_blk : kGroupWideRows;
            copy_sb_to_lds<kGroupStreamThreads, 2>(reinterpret_cast<const uint16_t*>(blob + o.down_s) + (size_t)d_blk * G,
                                                   reinterpret_cast<const uint16_t*>(blob + o.down_b) + (size_t)d_blk * G,
                                                   sb_lds, nd * G);
            __syncthreads();
        });
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        if (p >= gr.count) continue;
        uint16_t* dst = partials + (size_t)dst_row[j] * D;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            store_f16x4(dst, db + 16u * i + 4u * q, D, v);
        }
    }
}

template <int BITS>
__device__ __forceinline__ void moe_wide_gate_up(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                 const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                                 const uint16_t* __restrict__ hidden, uint32_t stride,
                                                 uint16_t* __restrict__ act, uint32_t D, uint32_t F, uint32_t bx,
                                                 uint32_t by) {
    GroupedRows gr;
    if (!wide_rows(tiles, n_tiles, by, gr)) return;
    if (gr.count <= 32u) wide_gate_up_half<BITS, 2>(pool, sorted, gr, hidden, stride, act, D, F, bx);
    else wide_gate_up_half<BITS, 4>(pool, sorted, gr, hidden, stride, act, D, F, bx);
}

template <int BITS>
__device__ __forceinline__ void moe_wide_down(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                              const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                              const uint16_t* __restrict__ act, uint16_t* __restrict__ partials,
                                              uint32_t D, uint32_t F, uint32_t k, uint32_t bx, uint32_t by) {
    GroupedRows gr;
    if (!wide_rows(tiles, n_tiles, by, gr)) return;
    if (gr.count <= 32u) wide_down_half<BITS, 2>(pool, sorted, gr, act, partials, D, F, k, bx);
    else wide_down_half<BITS, 4>(pool, sorted, gr, act, partials, D, F, k, bx);
}

// One launch per projection runs both, so the stream's weight reads overlap
// the tile's matrix work: blocks 0 .. max_tiles·sx - 1 are the stream's
// (x = b mod sx, y = b / sx; sx blocks of rows), the rest the MFMA tile's
// (x = b' mod 2·max_tiles, y = b' / 2·max_tiles; ty blocks of outputs)
// (GroupedLaunch, abi_types.h). Either order measures the same on config 3.
static_assert(kGroupStreamThreads == kProjThreads, "one launch runs both roles");

template <int BITS>
__device__ __forceinline__ void moe_grouped_gate_up_launch(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                           const Tile* __restrict__ tiles,
                                                           const uint32_t* __restrict__ n_tiles,
                                                           const uint16_t* __restrict__ hidden, uint32_t stride,
                                                           uint16_t* __restrict__ act, uint32_t D, uint32_t F,
                                                           GroupedLaunch gl) {
    const uint32_t b = blockIdx.x, ns = gl.max_tiles * gl.sx;
    if (b < ns) moe_stream_gate_up<BITS>(pool, sorted, tiles, n_tiles, hidden, stride, act, D, F, b % gl.sx, b / gl.sx);
    else moe_wide_gate_up<BITS>(pool, sorted, tiles, n_tiles, hidden, stride, act, D, F, (b - ns) % gl.wx, (b - ns) / gl.wx);
}

template <int BITS>
__device__ __forceinline__ void moe_grouped_down_launch(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                        const Tile* __restrict__ tiles,
                                                        const uint32_t* __restrict__ n_tiles,
                                                        const uint16_t* __restrict__ act, uint16_t* __restrict__ partials,
                                                        uint32_t D, uint32_t F, uint32_t k, GroupedLaunch gl) {
    const uint32_t b = blockIdx.x, ns = gl.max_tiles * gl.sx;
    if (b < ns) moe_stream_down<BITS>(pool, sorted, tiles, n_tiles, act, partials, D, F, k, b % gl.sx, b / gl.sx);
    else moe_wide_down<BITS>(pool, sorted, tiles, n_tiles, act, partials, D, F, k, (b - ns) % gl.wx, (b - ns) / gl.wx);
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
