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
constexpr uint32_t kGroupStateWords = 4;       // TFQ_MOE_GROUP_STATE_WORDS
constexpr uint32_t kGroupSegments = 8;         // chunk segments of the per-expert scan
// status codes (the PrefillMoEGroupingError cases the device can detect)
constexpr uint32_t kGroupOk = 0;
constexpr uint32_t kGroupExpertOutOfRange = 8;
// grouping tiles of at most kGroupStreamMax pairs run as stream units, larger
// ones as wide units (see the grouped MoE units below)
constexpr uint32_t kGroupStreamMax = 32;

// threadIdx.x as an opaque value: the work units of a persistent launch read
// it through this, so the compiler rederives each unit's lane addresses
// inside the unit instead of hoisting them out of the unit loop, where they
// would stay live (in registers) across every other unit body.
__device__ __forceinline__ uint32_t unit_tid() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// dst[n .. n+3] = fp16(v[0..3]) as one 8-byte store when n < lim: n and
// lim are multiples of 4 (rows of d or f, multiples of 64, outputs in
// fours) and dst is 8-byte aligned (act and partials are 16-byte aligned).
__device__ __forceinline__ void store_f16x4(uint16_t* __restrict__ dst, uint32_t n, uint32_t lim, const float (&v)[4]) {
    if (n < lim)
        *reinterpret_cast<uint2*>(dst + n) = make_uint2((uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16),
                                                        (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16));
}

// Stable counting sort of the token-major pairs (token t, rank r) -> expert
// idx[t*k + r], one block of 1024 threads. Pairs come out ordered by
// (expert, token, rank) exactly as the reference's sort
// (PrefillMoEGrouping.swift:145-154 without sort keys): each wavefront
// ranks its 64 pairs among equal experts with ballots, a per-expert scan
// over the 64-pair chunks (in order) gives each chunk's base, and an
// exclusive scan over experts gives the offsets. Empty experts get offset
// 0xFFFFFFFF and count 0. The tile list cuts each expert's run into
// 128-row tiles. n_tiles is the grouping state (kGroupStateWords words):
// the tile count, then the grouped launches' work counters, zeroed here.
// On an out-of-range expert index nothing is grouped and
// *status = kGroupExpertOutOfRange.
__device__ __forceinline__ void moe_group(const uint32_t* __restrict__ idx, const uint16_t* __restrict__ w,
                                          uint32_t T, uint32_t k, uint32_t E, Pair* __restrict__ sorted,
                                          uint32_t* __restrict__ offsets, uint32_t* __restrict__ counts,
                                          Tile* __restrict__ tiles, uint32_t* __restrict__ n_tiles,
                                          uint32_t* __restrict__ status) {
    __shared__ uint16_t cnt[kGroupChunks][kGroupMaxExperts];
    __shared__ uint8_t rank_in_chunk[kGroupMaxPairs];
    __shared__ uint32_t base[kGroupMaxExperts], tot[kGroupMaxExperts], tile_base[kGroupMaxExperts + 1];
    __shared__ uint32_t seg_sum[kGroupSegments][kGroupMaxExperts];
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
        if (tid < kGroupStateWords) n_tiles[tid] = 0;
        if (tid == 0) *status = kGroupExpertOutOfRange;
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
    // per expert: exclusive scan over the chunks (in chunk order), in S
    // segments of chunks: thread (segment sg, expert e) sums its segment,
    // adds the sums of the segments before it and rewrites its counts as
    // offsets (lanes of a wavefront take consecutive experts of one segment)
    {
        const uint32_t ep = E > 1 ? 1u << (32 - __clz((int)(E - 1))) : 1u;   // E rounded up to a power of two
        const uint32_t S = kGroupThreads / ep < kGroupSegments ? kGroupThreads / ep : kGroupSegments;
        const uint32_t e = tid % ep, sg = tid / ep, per = (nchunks + S - 1) / S;
        const uint32_t c0 = sg * per, c1 = c0 + per < nchunks ? c0 + per : nchunks;
        const bool mine = e < E && sg < S;
        uint32_t part = 0;
        if (mine) {
            for (uint32_t c = c0; c < c1; ++c) part += cnt[c][e];
            seg_sum[sg][e] = part;
        }
        __syncthreads();
        if (mine) {
            uint32_t run = 0;
            for (uint32_t t = 0; t < sg; ++t) run += seg_sum[t][e];
            for (uint32_t c = c0; c < c1; ++c) {
                const uint32_t v = cnt[c][e];
                cnt[c][e] = (uint16_t)run;
                run += v;
            }
            if (sg == S - 1) tot[e] = run;
        }
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
        } else if (tid < kGroupStateWords) {
            n_tiles[tid] = 0;
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

// Rows of one work unit's pairs: a run of the sorted pairs of one expert.
struct GroupedRows {
    uint32_t first;   // index of the first pair in the sorted pairs
    uint32_t count;   // pairs (1..64 on the wide role, 1..32 on the stream)
    uint32_t expert;
};

// f(integral_constant<B>) ... f(<E-1>)
template <int B, int E, typename Fn>
__device__ __forceinline__ void sfor_w(Fn&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        sfor_w<B + 1, E>(f);
    }
}

// f(<B>), then f(<B+1>) only if f(<B>) returned true, ...: each call sits
// inside the branch of the one before, so the code after a call is reached
// only through it and the compiler's waits there count its loads exactly
// (independent branches would merge paths that issued different loads, and
// the wait after such a join covers every load).
template <int B, int E, typename Fn>
__device__ __forceinline__ void sfor_while(Fn&& f) {
    if constexpr (B < E) {
        if (f(std::integral_constant<int, B>{})) sfor_while<B + 1, E>(f);
    }
}


// ------------------------------------------------------ grouped MoE units ----
//
// The grouped projections run per unit: the pairs of one grouping tile (a
// 64-pair half of a tile of more than kGroupStreamMax pairs, or a whole
// smaller tile) times a block of weight rows. Each of the four wavefronts owns
// RT 16-row A operands of v_mfma_f32_16x16x32_f16 and the whole K loop; the
// pairs are NTT 16-pair B operands. Two shapes:
//   wide   (tiles of more than 32 pairs): RT 2, NTT 2 or 4, 128 rows per unit
//          (gate/up: 64 features, gate and up rows; down: 128 outputs);
//   stream (tiles of at most 32 pairs):   RT 4, NTT 1 or 2, 256 rows per unit
//          (gate/up: 128 features; down: 256 outputs).
// Under a skewed popularity most experts see a handful of tokens (config 3:
// 101 of 128 experts take at most 32 of the 4096 pairs, yet hold 80% of the
// active weights), so the stream shape spreads each activation k-tile over
// twice the rows. Lane l holds row l%16 of each A operand and the quarter
// q = l/16 of every 128-code k-tile (chunk 4m + q: one 16-byte load at 4 bits;
// word u feeds k-step u), dequantised from a DEPTH-deep register ring with the
// scale and bias of an LDS table (one word per row and group). The unit's
// activations are staged per k-tile into a double-buffered LDS tile
// [16·NTT pairs][128 codes + 8] in the unpack order, from a two-deep register
// ring, one barrier per k-tile; the B lane (pair l%16 of sub-tile j, quarter
// q) reads its 16 bytes of k-step u at column 32q + 8u. In a half-filled
// last k-tile the quarters past K dequantise with scale and bias 0 (exact
// zero weights) against activations staged from column 0 (finite), so they
// add nothing. Weights are dequantised as everywhere else (fp16(q·s + b),
// one rounding).
constexpr uint32_t kGroupWidePairs = 64;          // pairs of a wide unit (a half tile)
constexpr uint32_t kUnitStride = 128 + 8;         // halves per LDS activation row
constexpr uint32_t kUnitThreads = 256;            // four wavefronts

// LDS of a unit: two activation buffers of 16·NTT rows, then the scale/bias
// table of its 64·RT weight rows.
constexpr uint32_t unit_xbuf(int NTT) { return 16u * (uint32_t)NTT * kUnitStride; }   // halves
constexpr uint32_t unit_lds_bytes(int RT, int NTT, uint32_t K) {
    return 2u * unit_xbuf(NTT) * 2u + 4u * 64u * (uint32_t)RT * (K / 64u);
}

// A unit's scale/bias table staged through registers: the `count` scale and
// bias words of its rows (16-byte aligned, count % 8 == 0, count <=
// 8·U·kUnitThreads) loaded by issue() with unconditional, clamped loads
// before the unit's weight and activation loads, and written to LDS as
// (scale | bias << 16) words by store() once they arrive, so the wait for
// them covers nothing issued after them (copy_sb_to_lds loads and stores in
// one loop, whose waits covered the whole weight ring). Threads past the
// table rewrite its last 16-byte piece with the same words.
template <uint32_t U>
struct TableRegs {
    uint4 va[U], vb[U];
    __device__ __forceinline__ void issue(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                          uint32_t count, uint32_t tid) {
        const uint32_t n16 = count >> 3;
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = u * kUnitThreads + tid, c = i < n16 ? i : n16 - 1;
            va[u] = reinterpret_cast<const uint4*>(a)[c];
            vb[u] = reinterpret_cast<const uint4*>(b)[c];
        }
    }
    __device__ __forceinline__ void store(uint32_t* __restrict__ dst, uint32_t count, uint32_t tid) const {
        const uint32_t n16 = count >> 3;
        uint4* t = reinterpret_cast<uint4*>(dst);
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t i = u * kUnitThreads + tid, c = i < n16 ? i : n16 - 1;
            // v_perm: bytes 0-3 from the second operand, 4-7 from the first
            t[2 * c] = make_uint4(__builtin_amdgcn_perm(vb[u].x, va[u].x, 0x05040100u),
                                  __builtin_amdgcn_perm(vb[u].x, va[u].x, 0x07060302u),
                                  __builtin_amdgcn_perm(vb[u].y, va[u].y, 0x05040100u),
                                  __builtin_amdgcn_perm(vb[u].y, va[u].y, 0x07060302u));
            t[2 * c + 1] = make_uint4(__builtin_amdgcn_perm(vb[u].z, va[u].z, 0x05040100u),
                                      __builtin_amdgcn_perm(vb[u].z, va[u].z, 0x07060302u),
                                      __builtin_amdgcn_perm(vb[u].w, va[u].w, 0x05040100u),
                                      __builtin_amdgcn_perm(vb[u].w, va[u].w, 0x07060302u));
        }
    }
};

// Table words per 16-byte register piece of TableRegs: a unit of `rows`
// weight rows over K/64 groups fits U pieces per thread when rows·K/64 <=
// 8·U·kUnitThreads.
constexpr uint32_t table_regs_fit(uint32_t rows, uint32_t K, uint32_t U) { return rows * (K / 64u) <= 8u * U * kUnitThreads; }

// Global addresses are a block-uniform base (scalar registers) plus a 32-bit
// per-lane offset, the form that costs one vector register. acc[i][j]: row
// tile i, pair sub-tile j (16x16 D layout: column lane%16 = pair, rows
// 4·(lane/16) + r). wbase[i] + woff[i]: this lane's weight row in tile i.
// xbase + xoff(p) (halves): the activation row of pair p (< 16·NTT; past the
// unit's count: any valid row, not stored). sbt[i]: this lane's row of the
// scale/bias table, published by the barrier that `publish` runs once the
// first k-tiles' loads are in flight; `issue` runs first (the table's loads
// when it is staged through registers).
template <int BITS, int RT, int NTT, int DEPTH, typename XOff, typename Issue, typename Publish>
__device__ __forceinline__ void unit_rows_loop(const uint8_t* const (&wbase)[RT], const uint32_t (&woff)[RT],
                                               const uint32_t* const (&sbt)[RT], const uint16_t* __restrict__ xbase,
                                               XOff xoff, uint32_t K, _Float16* __restrict__ xs,
                                               f32x4 (&acc)[RT][NTT], Issue issue, Publish publish, uint32_t tid) {
    const uint32_t lane = tid & 63u, q = lane >> 4, r16 = lane & 15u;
    const uint32_t nch = K >> 5, nk = (nch + 3u) >> 2;
    constexpr uint32_t PIECES = NTT;                   // 16-byte activation pieces per thread (16·NTT rows x 16)
    constexpr uint32_t XB = unit_xbuf(NTT);
    const DequantConsts<BITS> dc = dequant_consts<BITS>();
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < NTT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // activation piece p of this thread: pair 16p + tid/16, 16-byte column tid % 16
    uint32_t xr_off[PIECES];
#pragma unroll
    for (uint32_t p = 0; p < PIECES; ++p) xr_off[p] = xoff(16u * p + (tid >> 4));
    const uint32_t xcol = tid & 15u;
    QChunk<BITS> wr[DEPTH][RT];
    uint4 xr[2][PIECES];
    auto load_w = [&](uint32_t m, QChunk<BITS> (&dst)[RT]) {
        const uint32_t c = 4u * m + q, cc = c < nch ? c : nch - 1;
#pragma unroll
        for (int i = 0; i < RT; ++i) dst[i] = ldg_chunk_at<BITS>(wbase[i], woff[i] + 4u * BITS * cc);
    };
    // columns past K load column 0 (in bounds; their weights are zero)
    auto load_x = [&](uint32_t m, uint4 (&dst)[PIECES]) {
        const uint32_t col = 128u * (m < nk ? m : nk - 1) + 8u * xcol;
        const uint32_t cc = col < K ? col : 0u;
#pragma unroll
        for (uint32_t p = 0; p < PIECES; ++p) dst[p] = *reinterpret_cast<const uint4*>(xbase + (xr_off[p] + cc));
    };
    auto store_x = [&](const uint4 (&src)[PIECES], _Float16* buf) {
#pragma unroll
        for (uint32_t p = 0; p < PIECES; ++p)
            *reinterpret_cast<h8*>(buf + (16u * p + (tid >> 4)) * kUnitStride + 8u * xcol) =
                unit_b_order<BITS>(__builtin_bit_cast(h8, src[p]));
    };
    // per k-step u: the NTT B operands read together, the RT A operands
    // dequantised from their block words, then RT·NTT MFMAs. A quarter past
    // K (a half-filled last k-tile) takes scale and bias 0: its weights are
    // exact zeros, and the (finite) activations staged there from column 0
    // add nothing.
    auto compute = [&](uint32_t m, const QChunk<BITS> (&w)[RT], const _Float16* buf) {
        const uint32_t c = 4u * m + q, g = (c < nch ? c : nch - 1) >> 1;
        uint32_t sb[RT];
#pragma unroll
        for (int i = 0; i < RT; ++i) sb[i] = c < nch ? sbt[i][g] : 0u;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            h8 b[NTT];
#pragma unroll
            for (int j = 0; j < NTT; ++j)
                b[j] = *reinterpret_cast<const h8*>(buf + (16u * j + r16) * kUnitStride + 32u * q + 8u * u);
            h8 a[RT];
#pragma unroll
            for (int i = 0; i < RT; ++i) a[i] = dequant_word_sb<BITS>(w[i], u, sb[i], dc);
#pragma unroll
            for (int j = 0; j < NTT; ++j)
#pragma unroll
                for (int i = 0; i < RT; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    // prologue: the table's loads (issue), weights of k-tiles 0..DEPTH-1,
    // activations of 0 and 1; stage 0
    issue();
    load_x(0, xr[0]);
    load_x(1, xr[1]);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load_w((uint32_t)d, wr[d]);
    publish();                                   // the scale/bias table (ends with a barrier)
    store_x(xr[0], xs);
    load_x(2, xr[0]);
    __syncthreads();
    // step m: k-tile m from buffer m%2 and ring stage m%DEPTH; stage k-tile
    // m+1 into the other buffer; refill the rings (weights m+DEPTH,
    // activations m+3)
    auto step = [&](uint32_t m, auto st_c, auto pa_c) {
        constexpr int ST = decltype(st_c)::value, PA = decltype(pa_c)::value;
        compute(m, wr[ST], xs + PA * XB);
        store_x(xr[PA ^ 1], xs + (PA ^ 1) * XB);
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
    sfor_while<0, U - 1>([&](auto c) {
        if (m + c.value >= nk) return false;
        step(m + c.value, std::integral_constant<int, c.value % DEPTH>{}, std::integral_constant<int, c.value & 1>{});
        return true;
    });
}

// ring depth of a shape: the 64-row waves hold four k-tiles of weights
template <int RT>
constexpr int unit_depth() { return RT == 2 ? 3 : 4; }

// Gate/up + GeGLU of one unit over 32·RT features (row block bx): wave w
// takes features f_blk + 16·(RT/2)·w + (0..16·RT/2-1), its gate rows as row
// tiles 0..RT/2-1 and its up rows as row tiles RT/2..RT-1, so each lane holds
// gate and up of the same (pair, feature). LDS table rows 0..NF-1: gate
// scales/biases, NF..2NF-1: up. TAB: the table staged through registers
// (TableRegs; 16-byte aligned scale/bias rows, table_regs_fit), else copied
// by copy_sb_to_lds.
template <int BITS, int RT, int NTT, bool TAB>
__device__ __forceinline__ void unit_gate_up(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                             const GroupedRows& gr, const uint16_t* __restrict__ hidden,
                                             uint32_t stride, uint16_t* __restrict__ act, uint32_t D, uint32_t F,
                                             uint32_t bx) {
    extern __shared__ __attribute__((aligned(16))) _Float16 unit_lds[];
    constexpr uint32_t NF = 32u * RT, HT = RT / 2;
    const uint32_t tid = unit_tid(), lane = tid & 63u, wave = tid >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t G = D >> 6, row_bytes = (D >> 3) * BITS;
    const uint32_t f_blk = bx * NF, fb = f_blk + 16u * HT * wave;
    const uint8_t* blob = pool.base + (uint64_t)gr.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    uint32_t* sb_lds = reinterpret_cast<uint32_t*>(unit_lds + 2u * unit_xbuf(NTT));
    const uint8_t* wbase[RT];
    uint32_t woff[RT];
    const uint32_t* sbt[RT];
#pragma unroll
    for (uint32_t i = 0; i < HT; ++i) {
        const uint32_t f = fb + 16u * i + r16, fc = f < F ? f : F - 1;   // features past F: clamped, not stored
        wbase[i] = blob + o.gate_w;
        wbase[HT + i] = blob + o.up_w;
        woff[i] = woff[HT + i] = fc * row_bytes;
        sbt[i] = sb_lds + (fc - f_blk) * G;
        sbt[HT + i] = sb_lds + (NF + fc - f_blk) * G;
    }
    f32x4 acc[RT][NTT];
    const uint32_t nf = F - f_blk < NF ? F - f_blk : NF;
    const uint16_t* gs = reinterpret_cast<const uint16_t*>(blob + o.gate_s) + (size_t)f_blk * G;
    const uint16_t* gb = reinterpret_cast<const uint16_t*>(blob + o.gate_b) + (size_t)f_blk * G;
    const uint16_t* us = reinterpret_cast<const uint16_t*>(blob + o.up_s) + (size_t)f_blk * G;
    const uint16_t* ub = reinterpret_cast<const uint16_t*>(blob + o.up_b) + (size_t)f_blk * G;
    TableRegs<TAB ? (RT == 4 ? 3u : 2u) : 1u> tg, tu;
    unit_rows_loop<BITS, RT, NTT, unit_depth<RT>()>(
        wbase, woff, sbt, hidden,
        [&](uint32_t p) { return sorted[gr.first + (p < gr.count ? p : 0u)].token * stride; }, D, unit_lds, acc,
        [&]() {
            if constexpr (TAB) {
                tg.issue(gs, gb, nf * G, tid);
                tu.issue(us, ub, nf * G, tid);
            }
        },
        [&]() {
            if constexpr (TAB) {
                tg.store(sb_lds, nf * G, tid);
                tu.store(sb_lds + NF * G, nf * G, tid);
            } else {
                copy_sb_to_lds<kUnitThreads, 2>(gs, gb, sb_lds, nf * G, tid);
                copy_sb_to_lds<kUnitThreads, 2>(us, ub, sb_lds + NF * G, nf * G, tid);
            }
            __syncthreads();
        },
        tid);
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        if (p >= gr.count) continue;
        uint16_t* dst = act + (size_t)(gr.first + p) * F;
#pragma unroll
        for (uint32_t i = 0; i < HT; ++i) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = gelu_tanh(acc[i][j][r]) * acc[HT + i][j][r];
            store_f16x4(dst, fb + 16u * i + 4u * q, F, v);
        }
    }
}

// Down projection of one unit over 64·RT outputs of D (row block bx): wave
// w takes rows d_blk + 16·RT·w + (0..16·RT-1). TAB as in unit_gate_up.
template <int BITS, int RT, int NTT, bool TAB>
__device__ __forceinline__ void unit_down(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                          const GroupedRows& gr, const uint16_t* __restrict__ act,
                                          uint16_t* __restrict__ partials, uint32_t D, uint32_t F, uint32_t k,
                                          uint32_t bx) {
    extern __shared__ __attribute__((aligned(16))) _Float16 unit_lds[];
    constexpr uint32_t NR = 64u * RT;
    const uint32_t tid = unit_tid(), lane = tid & 63u, wave = tid >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t G = F >> 6, row_bytes = (F >> 3) * BITS;
    const uint32_t d_blk = bx * NR, db = d_blk + 16u * RT * wave;
    const uint8_t* blob = pool.base + (uint64_t)gr.expert * pool.stride;
    const ExpertOffsets& o = pool.off;
    uint32_t* sb_lds = reinterpret_cast<uint32_t*>(unit_lds + 2u * unit_xbuf(NTT));
    const uint8_t* wbase[RT];
    uint32_t woff[RT];
    const uint32_t* sbt[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        const uint32_t d = db + 16u * i + r16, dc = d < D ? d : D - 1;   // rows past D: clamped, not stored
        wbase[i] = blob + o.down_w;
        woff[i] = dc * row_bytes;
        sbt[i] = sb_lds + (dc - d_blk) * G;
    }
    uint32_t dst_row[NTT];          // partials row of each pair, loaded before the K loop
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        const Pair pr = sorted[gr.first + (p < gr.count ? p : 0u)];
        dst_row[j] = pr.token * k + pr.rank;
    }
    f32x4 acc[RT][NTT];
    const uint32_t nd = D - d_blk < NR ? D - d_blk : NR;
    const uint16_t* ds = reinterpret_cast<const uint16_t*>(blob + o.down_s) + (size_t)d_blk * G;
    const uint16_t* dbv = reinterpret_cast<const uint16_t*>(blob + o.down_b) + (size_t)d_blk * G;
    TableRegs<TAB ? (RT == 4 ? 2u : 1u) : 1u> td;
    unit_rows_loop<BITS, RT, NTT, unit_depth<RT>()>(
        wbase, woff, sbt, act, [&](uint32_t p) { return (gr.first + (p < gr.count ? p : 0u)) * F; }, F, unit_lds, acc,
        [&]() {
            if constexpr (TAB) td.issue(ds, dbv, nd * G, tid);
        },
        [&]() {
            if constexpr (TAB) td.store(sb_lds, nd * G, tid);
            else copy_sb_to_lds<kUnitThreads, 2>(ds, dbv, sb_lds, nd * G, tid);
            __syncthreads();
        },
        tid);
#pragma unroll
    for (int j = 0; j < NTT; ++j) {
        const uint32_t p = 16u * j + r16;
        if (p >= gr.count) continue;
        uint16_t* dst = partials + (size_t)dst_row[j] * D;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            store_f16x4(dst, db + 16u * i + 4u * q, D, v);
        }
    }
}

// ------------------------------------------------ persistent unit schedule ----
//
// A grouped launch runs a grid of resident blocks (P = gridDim.x) over a work
// list that every block derives from the device tile list, so no block of
// the launch finds itself without work. A unit is (entry, row block): an
// entry is one 64-pair half of a tile of more than kGroupStreamMax pairs
// (wide role, wx row blocks) or one smaller tile (stream, sx row blocks).
// Entries come in four classes, dearest first: wide halves of more than 32
// pairs (NTT 4), the other wide halves (NTT 2), stream tiles of 17..32 pairs
// (NTT 2), then of at most 16 (NTT 1); tile order within a class, and the
// row blocks of an entry as consecutive units. Block b runs unit b first and
// then takes units P, P+1, ... in the order blocks ask for them (a counter in
// the grouping state, asked one unit ahead), so the dearest units start
// first and the cheap ones fill the gaps at the end. The last block to leave
// zeroes the counters for the next launch.
constexpr uint32_t kGroupMaxTiles = kGroupMaxPairs / kGemmBM + kGroupMaxExperts;   // bound of TFQ_MOE_MAX_TILES
static_assert(kGemmBM == 2 * kGroupWidePairs, "a grouping tile is two wide halves");
constexpr uint32_t kGroupMaxEntries = 2u * kGroupMaxTiles;
constexpr uint32_t kGroupNextUnit = 1, kGroupBlocksDone = 2;   // counter words of the grouping state

struct UnitPlan {
    uint32_t n_wide;      // wide entries (the first two classes)
    uint32_t n_entries;   // all entries
};

// Wavefront 0 writes the entries ({first pair, expert | count << 16}) of the
// first min(n_tiles[0], max_tiles) tiles into ent; ends with a barrier.
__device__ __forceinline__ UnitPlan plan_units(const Tile* __restrict__ tiles, const uint32_t* __restrict__ n_tiles,
                                               uint32_t max_tiles, uint2* ent) {
    __shared__ uint32_t plan_tot[2];
    constexpr uint32_t C = kGroupMaxTiles / 64u;          // tiles per lane
    static_assert(kGroupMaxTiles % 64u == 0, "whole wavefront passes");
    if (threadIdx.x < 64u) {
        const uint32_t lane = threadIdx.x;
        // the tile count and the tiles up to the launch bound in flight together
        const uint32_t nt = *n_tiles;
        const uint32_t mt = max_tiles < kGroupMaxTiles ? max_tiles : kGroupMaxTiles;
        Tile tl[C];
#pragma unroll
        for (uint32_t c = 0; c < C; ++c) {
            const uint32_t t = 64u * c + lane;
            tl[c] = t < mt ? tiles[t] : Tile{0u, 0u, 0u, 0u};
        }
        const uint32_t n = nt < mt ? nt : mt;
#pragma unroll
        for (uint32_t c = 0; c < C; ++c)
            if (64u * c + lane >= n) tl[c].count = 0;
        // per tile the entries of each class, two classes per word (16 bits
        // each: at most kGroupMaxEntries), scanned over the tiles in order
        uint32_t pre_w[C], pre_s[C], carry_w = 0, carry_s = 0;
#pragma unroll
        for (uint32_t c = 0; c < C; ++c) {
            const uint32_t cnt = tl[c].count;
            const uint32_t vw = ((cnt > 32u) + (cnt > 96u)) | ((uint32_t)(cnt > 64u && cnt <= 96u) << 16);
            const uint32_t vs = (uint32_t)(cnt > 16u && cnt <= 32u) | ((uint32_t)(cnt >= 1u && cnt <= 16u) << 16);
            uint32_t iw = vw, is = vs;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t uw = (uint32_t)__shfl_up((int)iw, o, kWave);
                const uint32_t us = (uint32_t)__shfl_up((int)is, o, kWave);
                if ((int)lane >= o) {
                    iw += uw;
                    is += us;
                }
            }
            pre_w[c] = carry_w + iw - vw;
            pre_s[c] = carry_s + is - vs;
            carry_w += (uint32_t)__shfl((int)iw, 63, kWave);
            carry_s += (uint32_t)__shfl((int)is, 63, kWave);
        }
        const uint32_t n0 = carry_w & 0xFFFFu, n1 = carry_w >> 16, n2 = carry_s & 0xFFFFu, n3 = carry_s >> 16;
#pragma unroll
        for (uint32_t c = 0; c < C; ++c) {
            const Tile t = tl[c];
            if (t.count > kGroupStreamMax) {
                const uint32_t p0 = pre_w[c] & 0xFFFFu;
                const uint32_t c0 = t.count < kGroupWidePairs ? t.count : kGroupWidePairs;
                ent[p0] = make_uint2(t.start, t.expert | (c0 << 16));
                if (t.count > kGroupWidePairs) {
                    const uint32_t left = t.count - kGroupWidePairs;
                    ent[left > 32u ? p0 + 1u : n0 + (pre_w[c] >> 16)] =
                        make_uint2(t.start + kGroupWidePairs, t.expert | (left << 16));
                }
            } else if (t.count > 16u) {
                ent[n0 + n1 + (pre_s[c] & 0xFFFFu)] = make_uint2(t.start, t.expert | (t.count << 16));
            } else if (t.count >= 1u) {
                ent[n0 + n1 + n2 + (pre_s[c] >> 16)] = make_uint2(t.start, t.expert | (t.count << 16));
            }
        }
        if (lane == 0) {
            plan_tot[0] = n0 + n1;
            plan_tot[1] = n0 + n1 + n2 + n3;
        }
    }
    __syncthreads();
    return {plan_tot[0], plan_tot[1]};
}

// The unit loop of one grouped launch: wide(rows, bx) / stream(rows, bx) run
// one unit each (block-uniform calls). Every unit starts after a barrier, so
// it may reuse the dynamic LDS of the one before. state: the grouping state
// (tile count, then the counters).
template <typename Wide, typename Stream>
__device__ __forceinline__ void run_units(const Tile* __restrict__ tiles, uint32_t* __restrict__ state,
                                          GroupedLaunch gl, Wide wide, Stream stream) {
    __shared__ uint2 ent[kGroupMaxEntries];
    __shared__ uint32_t next_unit;
    const UnitPlan pl = plan_units(tiles, state, gl.max_tiles, ent);
    const uint32_t P = gridDim.x, tid = threadIdx.x;
    const uint32_t n_wu = pl.n_wide * gl.wx, n_units = n_wu + (pl.n_entries - pl.n_wide) * gl.sx;
    uint32_t u = blockIdx.x;
    while (u < n_units) {
        // the next unit's number, asked for now and read after this unit
        uint32_t ask = 0;
        if (tid == 0) ask = atomicAdd(state + kGroupNextUnit, 1u);
        if (u < n_wu) {
            const uint2 e = ent[u / gl.wx];
            wide(GroupedRows{e.x, e.y >> 16, e.y & 0xFFFFu}, u % gl.wx);
        } else {
            const uint32_t v = u - n_wu;
            const uint2 e = ent[pl.n_wide + v / gl.sx];
            stream(GroupedRows{e.x, e.y >> 16, e.y & 0xFFFFu}, v % gl.sx);
        }
        if (tid == 0) next_unit = ask + P;
        __syncthreads();
        u = next_unit;
        __syncthreads();
    }
    // every block asks once more than it runs units: when the last one
    // leaves, no block of this launch touches the counters again
    if (tid == 0 && atomicAdd(state + kGroupBlocksDone, 1u) == P - 1u) {
        atomicExch(state + kGroupNextUnit, 0u);
        atomicExch(state + kGroupBlocksDone, 0u);
    }
}

static_assert(kUnitThreads == kProjThreads, "the grouped launches run kProjThreads threads");

// TAB: the units' scale/bias tables staged through registers (the host
// picks these launches for 16-byte aligned scale/bias offsets whose tables
// fit: d <= 3072 for gate/up, f <= 1024 for down).
template <int BITS, bool TAB = false>
__device__ __forceinline__ void moe_grouped_gate_up_launch(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                           const Tile* __restrict__ tiles, uint32_t* __restrict__ n_tiles,
                                                           const uint16_t* __restrict__ hidden, uint32_t stride,
                                                           uint16_t* __restrict__ act, uint32_t D, uint32_t F,
                                                           GroupedLaunch gl) {
    run_units(
        tiles, n_tiles, gl,
        [&](const GroupedRows& gr, uint32_t bx) {
            if (gr.count <= 32u) unit_gate_up<BITS, 2, 2, TAB>(pool, sorted, gr, hidden, stride, act, D, F, bx);
            else unit_gate_up<BITS, 2, 4, TAB>(pool, sorted, gr, hidden, stride, act, D, F, bx);
        },
        [&](const GroupedRows& gr, uint32_t bx) {
            if (gr.count <= 16u) unit_gate_up<BITS, 4, 1, TAB>(pool, sorted, gr, hidden, stride, act, D, F, bx);
            else unit_gate_up<BITS, 4, 2, TAB>(pool, sorted, gr, hidden, stride, act, D, F, bx);
        });
}

template <int BITS, bool TAB = false>
__device__ __forceinline__ void moe_grouped_down_launch(const ExpertPool& pool, const Pair* __restrict__ sorted,
                                                        const Tile* __restrict__ tiles, uint32_t* __restrict__ n_tiles,
                                                        const uint16_t* __restrict__ act, uint16_t* __restrict__ partials,
                                                        uint32_t D, uint32_t F, uint32_t k, GroupedLaunch gl) {
    run_units(
        tiles, n_tiles, gl,
        [&](const GroupedRows& gr, uint32_t bx) {
            if (gr.count <= 32u) unit_down<BITS, 2, 2, TAB>(pool, sorted, gr, act, partials, D, F, k, bx);
            else unit_down<BITS, 2, 4, TAB>(pool, sorted, gr, act, partials, D, F, k, bx);
        },
        [&](const GroupedRows& gr, uint32_t bx) {
            if (gr.count <= 16u) unit_down<BITS, 4, 1, TAB>(pool, sorted, gr, act, partials, D, F, k, bx);
            else unit_down<BITS, 4, 2, TAB>(pool, sorted, gr, act, partials, D, F, k, bx);
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

// moe_combine over 8 outputs per thread (16-byte loads and stores): D % 8 ==
// 0, partials and h2 16-byte aligned. Thread i: token i / (D/8), outputs
// 8·(i mod D/8) .. +7; the same rank-order fmas as moe_combine. Grid:
// ceil(T·D/8 / 256).
__device__ __forceinline__ void moe_combine_x8(const uint16_t* __restrict__ partials,
                                               const uint16_t* __restrict__ w, uint16_t* __restrict__ h2,
                                               uint32_t T, uint32_t k, uint32_t D) {
    const uint32_t n8 = D >> 3, i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= T * n8) return;
    const uint32_t t = i / n8, d = 8u * (i - t * n8);
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (k == 8) {
        // top-8 (the model's k): the eight rows' loads in flight together,
        // then the same fma chain in rank order (one memory round trip
        // instead of eight)
        h8 v[8];
        float wr[8];
#pragma unroll
        for (uint32_t r = 0; r < 8; ++r) {
            wr[r] = h2f(w[t * 8 + r]);
            v[r] = __builtin_bit_cast(h8, *reinterpret_cast<const uint4*>(partials + ((size_t)t * 8 + r) * D + d));
        }
#pragma unroll
        for (uint32_t r = 0; r < 8; ++r)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(wr[r], (float)v[r][e], acc[e]);
    } else {
        for (uint32_t r = 0; r < k; ++r) {
            const float wr = h2f(w[t * k + r]);
            const h8 v = __builtin_bit_cast(h8, *reinterpret_cast<const uint4*>(partials + ((size_t)t * k + r) * D + d));
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(wr, (float)v[e], acc[e]);
        }
    }
    h8 out;
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = (_Float16)acc[e];
    *reinterpret_cast<uint4*>(h2 + (size_t)t * D + d) = __builtin_bit_cast(uint4, out);
}

}  // namespace tfq
