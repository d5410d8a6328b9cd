// gemm.hpp — dequant-fused int4 GEMM tile on the matrix cores, used by the
// prefill projection GEMM and by the grouped MoE prefill:
//     C[j][n] = Σ_k X[row_j][k] · W_m[n][k]     (m = 0..NMAT-1 weight matrices)
// W affine int4 g64 with fp16 scale/bias, X fp16 (or bf16, converted),
// fp32 accumulate (S/Metal/TensorCore/tensorops.metal:13-105 and
// S/Metal/Prefill/prefill.metal:672-709 compute the same product).
//
// Block tile 128 rows x 128 outputs, one affine group (64 along K) per step,
// 8 wavefronts (two per SIMD, so one wave's loads and dequantisation overlap
// the other's MFMAs), each owning a 32x64 slice of the tile as 1x2
// v_mfma_f32_32x32x16_f16 tiles per matrix. Per step the block
//   * loads the X tile (16 B per load, coalesced; rows come from a caller
//     supplied row table, so gathered rows cost nothing extra) and each W
//     tile (8 B = 16 codes per thread) with its 128 scale/bias pairs, two
//     steps ahead of their use (two register stages),
//   * dequantises in registers: (0x6400 | q) - 1024 gives q exactly as fp16,
//     then v_pk_fma_f16(q, s, b) rounds q·s + b once to fp16 — the fp16
//     weight tile the reference's tensor-op kernel stages (tensorops.metal:57-80),
//   * writes the tiles to the other half of a double-buffered LDS while the
//     MFMAs consume the current half.
// Within every 8-element run along K the unpack yields element order
// (0,4,1,5,2,6,3,7); X is stored with the same permutation, so each MFMA
// k-slice pairs the right operands (a dot product is order-free).
// bf16 activations are converted to fp16 while staging; the conversion is
// exact for |x| in [2^-14, 65504] (the range of the reference's fp16 path).
#pragma once

#include <type_traits>

#include "common.hpp"

namespace tfq {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmBM = 128;
constexpr int kGemmBN = 128;
constexpr int kGemmBK = 64;
constexpr int kGemmLdsStride = kGemmBK + 8;       // halves per LDS row (16-byte pad)
constexpr int kGemmThreads = 512;
constexpr int kGemmTile = kGemmBM * kGemmLdsStride;

// Permute one 8-element run from natural order to (0,4,1,5,2,6,3,7).
__device__ __forceinline__ h8 perm_0415(h8 v) {
    return __builtin_shufflevector(v, v, 0, 4, 1, 5, 2, 6, 3, 7);
}

// 8 bf16 -> 8 fp16 (exact inside the fp16 normal range).
__device__ __forceinline__ h8 bf16x8_to_f16(uint4 raw) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    h8 out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = __builtin_bit_cast(float, w[i] << 16);
        const float hi = __builtin_bit_cast(float, w[i] & 0xFFFF0000u);
        out[2 * i] = (_Float16)lo;
        out[2 * i + 1] = (_Float16)hi;
    }
    return out;
}

// Dequantise the 32 codes of one 16-byte chunk into 4 runs of 8 fp16 weights
// (permuted order 0,4,1,5,2,6,3,7 inside each run).
__device__ __forceinline__ void dequant_chunk_f16(uint4 w, uint16_t s_bits, uint16_t b_bits, h8 (&out)[4]) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    const _Float16 s = __builtin_bit_cast(_Float16, s_bits);
    const _Float16 b = __builtin_bit_cast(_Float16, b_bits);
    const h2 s2 = {s, s}, b2 = {b, b};
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h8 run;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = ((ws[j] >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
            const h2 qh = __builtin_bit_cast(h2, q) - k1024;             // exact q pair
            const h2 wv = __builtin_elementwise_fma(qh, s2, b2);         // one rounding
            run[2 * i] = wv[0];
            run[2 * i + 1] = wv[1];
        }
        out[j] = run;
    }
}

// One int4 weight matrix as seen by a tile: row n of W starts at w + n*K/2.
struct Q4Tile {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
};

// LDS of one tile with NMAT weight matrices (double buffered).
template <int NMAT>
struct GemmLds {
    _Float16 x[2][kGemmTile];
    _Float16 w[NMAT][2][kGemmTile];
};

// Computes the 128x128 tile (rows: row_ptr[0..rows), outputs n0..n0+127 < N)
// and calls out(j, n, v[NMAT]) for every valid element. row_ptr holds the
// address of each X row (K elements). Must be called by all 512 threads.
template <bool X_BF16, int NMAT, typename Out>
__device__ __forceinline__ void gemm_tile(GemmLds<NMAT>& L, const uint16_t* const* row_ptr,
                                          uint32_t rows, const Q4Tile (&mats)[NMAT], uint32_t n0,
                                          uint32_t N, uint32_t K, Out out) {
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t groups = K >> 6;
    const uint32_t row_bytes = K >> 1;

    // global -> registers: X rows tid/8 and tid/8 + 64, 16-byte chunk tid%8
    // of the group; W row tid/4, 8-byte quarter tid%4 of the group's 32 bytes
    // (all 512 threads, no two loading the same bytes), with its scale and
    // bias. Every load is unconditional (groups past the end re-read the last
    // one, rows past `rows` read row 0, outputs past N read row N-1; none of
    // them is stored), so the number of loads per step is fixed and the
    // compiler waits for exactly the stage it consumes.
    const uint32_t xr = tid >> 3, xc = tid & 7u;
    const uint32_t wr = tid >> 2, wq = tid & 3u;
    uint4 xreg[2][2];
    uint2 wreg[2][NMAT];
    uint16_t sreg[2][NMAT], breg[2][NMAT];
    const size_t wn_row = (size_t)(n0 + wr < N ? n0 + wr : N - 1);
    auto load_global = [&](uint32_t g, int st) {
        const uint32_t gg = g < groups ? g : groups - 1;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t j = xr + 64u * p;
            xreg[st][p] = ldg16_global(row_ptr[j < rows ? j : 0u] + gg * 64u + 8u * xc);
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            wreg[st][m] = *reinterpret_cast<const uint2*>(mats[m].w + wn_row * row_bytes + gg * 32u + 8u * wq);
            sreg[st][m] = mats[m].s[wn_row * groups + gg];
            breg[st][m] = mats[m].b[wn_row * groups + gg];
        }
    };
    auto store_lds = [&](int st, int buf) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const h8 v = X_BF16 ? bf16x8_to_f16(xreg[st][p]) : __builtin_bit_cast(h8, xreg[st][p]);
            *reinterpret_cast<h8*>(&L.x[buf][(xr + 64u * p) * kGemmLdsStride + 8u * xc]) = perm_0415(v);
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            h8 runs[4];
            dequant_chunk_f16(make_uint4(wreg[st][m].x, wreg[st][m].y, 0u, 0u), sreg[st][m], breg[st][m], runs);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                *reinterpret_cast<h8*>(&L.w[m][buf][wr * kGemmLdsStride + 16u * wq + 8u * j]) = runs[j];
        }
    };

    f32x16 acc[NMAT][2];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[m][j][r] = 0.0f;

    // wave w: rows 32·(w/2) .. +31, outputs 64·(w%2) .. +63
    const uint32_t wm = (wave >> 1) * 32u, wn = (wave & 1u) * 64u;
    const uint32_t arow = lane & 31u, akoff = (lane >> 5) * 8u;

    auto mma_step = [&](int cur) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const h8 a = *reinterpret_cast<const h8*>(
                &L.x[cur][(wm + arow) * kGemmLdsStride + 16u * ks + akoff]);
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                h8 b[2];
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    b[j] = *reinterpret_cast<const h8*>(
                        &L.w[m][cur][(wn + 32u * j + arow) * kGemmLdsStride + 16u * ks + akoff]);
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[m][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b[j], acc[m][j], 0, 0, 0);
            }
        }
    };

    // one step: register stage and LDS buffer `cur` hold group g; refill the
    // stage with g+2, multiply, store the other stage (g+1) into the other
    // buffer. Stage indices are compile-time (the loop is unrolled by two),
    // so the register stages never go to scratch. The main loop runs whole
    // pairs of steps with no branch inside (past the end the steps re-read
    // and stage the last group, which nobody uses); an odd last group takes
    // a checked step after it.
    auto step = [&](uint32_t g, auto cur_c) {
        constexpr int cur = decltype(cur_c)::value;
        load_global(g + 2, cur);
        // keep the refill loads ahead of the MFMAs that follow
        __builtin_amdgcn_sched_barrier(0);
        mma_step(cur);
        store_lds(cur ^ 1, cur ^ 1);
        __syncthreads();
    };
    load_global(0, 0);
    load_global(1, 1);
    store_lds(0, 0);
    __syncthreads();
    uint32_t g = 0;
    for (; g + 2 <= groups; g += 2) {
        step(g, std::integral_constant<int, 0>{});
        step(g + 1, std::integral_constant<int, 1>{});
    }
    if (g < groups) step(g, std::integral_constant<int, 0>{});

    // D layout (32x32 tile): column = lane % 32, row = 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t col = n0 + wn + 32u * j + (lane & 31u);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t row = wm + 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3);
            if (row < rows) {
                float v[NMAT];
#pragma unroll
                for (int m = 0; m < NMAT; ++m) v[m] = acc[m][j][r];
                out(row, col, v);
            }
        }
    }
}

// ------------------------------------------------ projection GEMM tile ----
//
// The prefill projection Y = X·Wᵀ uses a second tile form in which the
// weights never pass through LDS: block tile 64 tokens x 256 outputs, four
// wavefronts, wave w owning outputs 64w..64w+63 for all 64 tokens as 2x2
// v_mfma_f32_32x32x16_f16 tiles. The MFMA B operand of a 32-output sub-tile
// is 8 consecutive k of one output row per lane, so each lane loads its own
// row's 16 bytes of a group (lane half h: bytes 16h..16h+15, k-step s uses
// word s) straight into registers, kProjDepth groups ahead (a register
// ring), and dequantises them into B operands just before its MFMAs; nothing
// else reads them, so they need no LDS and no barrier. The block's scales and
// biases (256 rows x K/64 groups each, one contiguous range per array) are
// copied to LDS once at the start. The activations, shared by all four
// waves, are converted (bf16 -> fp16) and permuted once per block into a
// double-buffered LDS tile (one barrier per group). Per group a wave issues
// 16 MFMAs and reads 8 KB of LDS.
//
// Every global load in the loop is unconditional (groups past the end
// re-read the last group, token rows past the end read row 0 and are zeroed
// when staged) and the ring holds only 16-byte registers: with a fixed load
// count per step the compiler waits for exactly the group it consumes.
// Copies `count` halves of two arrays into LDS: 16-byte loads when both
// sources are 16-byte aligned and count % 8 == 0 (else 2-byte loads), up to
// eight loads per thread and array issued before the first store, so the
// copy costs one memory latency per 8·NT chunks.
template <uint32_t NT>
__device__ __forceinline__ void copy_pair_to_lds(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                                 uint16_t* __restrict__ da, uint16_t* __restrict__ db,
                                                 uint32_t count) {
    constexpr uint32_t U = 8;
    if (((((uintptr_t)a) | ((uintptr_t)b)) & 15u) == 0 && (count & 7u) == 0) {
        const uint32_t n16 = count >> 3;
        const uint4* sa = reinterpret_cast<const uint4*>(a);
        const uint4* sb = reinterpret_cast<const uint4*>(b);
        uint4* ta = reinterpret_cast<uint4*>(da);
        uint4* tb = reinterpret_cast<uint4*>(db);
        for (uint32_t base = 0; base < n16; base += U * NT) {
            uint4 va[U], vb[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t i = base + u * NT + threadIdx.x;
                const uint32_t c = i < n16 ? i : n16 - 1;
                va[u] = sa[c];
                vb[u] = sb[c];
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t i = base + u * NT + threadIdx.x;
                if (i < n16) {
                    ta[i] = va[u];
                    tb[i] = vb[u];
                }
            }
        }
    } else {
        for (uint32_t base = 0; base < count; base += U * NT) {
            uint16_t va[U], vb[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t i = base + u * NT + threadIdx.x;
                const uint32_t c = i < count ? i : count - 1;
                va[u] = a[c];
                vb[u] = b[c];
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t i = base + u * NT + threadIdx.x;
                if (i < count) {
                    da[i] = va[u];
                    db[i] = vb[u];
                }
            }
        }
    }
}

constexpr uint32_t kProjBM = 64;
constexpr uint32_t kProjBN = 256;
constexpr uint32_t kProjThreads = 256;
constexpr uint32_t kProjDepth = 4;          // groups in flight per wave (register ring)
constexpr uint32_t kProjMaxK = 8192;        // scale/bias LDS: 2 x 256 x K/64 halves

// Dynamic LDS of the projection tile: X double buffer, then scales, biases.
constexpr uint32_t proj_lds_bytes(uint32_t K) {
    return 2u * kProjBM * kGemmLdsStride * 2u + 2u * kProjBN * (K / 64u) * 2u;
}

// Dequantises one 16-byte chunk like dequant_chunk_f16, with the fp16
// exponent pattern held in a VGPR so that each nibble pair costs one
// v_and_or_b32 (gfx9 VOP3 takes no literal and one scalar operand).
__device__ __forceinline__ void dequant_chunk_f16_v(uint4 w, uint16_t s_bits, uint16_t b_bits, uint32_t magic_v,
                                                    h8 (&out)[4]) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    const _Float16 s = __builtin_bit_cast(_Float16, s_bits);
    const _Float16 b = __builtin_bit_cast(_Float16, b_bits);
    const h2 s2 = {s, s}, b2 = {b, b};
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h8 run;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t q = ((ws[j] >> (4 * i)) & 0x000F000Fu) | magic_v;
            const h2 qh = __builtin_bit_cast(h2, q) - k1024;             // exact q pair
            const h2 wv = __builtin_elementwise_fma(qh, s2, b2);         // one rounding
            run[2 * i] = wv[0];
            run[2 * i + 1] = wv[1];
        }
        out[j] = run;
    }
}

template <bool X_BF16>
__device__ __forceinline__ void gemm_q4_proj(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                             const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
                                             uint16_t* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K) {
    extern __shared__ __attribute__((aligned(16))) _Float16 proj_lds[];
    _Float16* xs0 = proj_lds;
    _Float16* xs1 = proj_lds + kProjBM * kGemmLdsStride;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t G = K >> 6, row_bytes = K >> 1;
    const uint32_t n0 = blockIdx.x * kProjBN, m0 = blockIdx.y * kProjBM;
    const uint32_t h = lane >> 5, col = lane & 31u;
    uint16_t* s_lds = reinterpret_cast<uint16_t*>(proj_lds + 2 * kProjBM * kGemmLdsStride);
    uint16_t* b_lds = s_lds + kProjBN * G;
    uint32_t magic_v;
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic_v));

    // scales / biases of rows n0 .. n0+255 (clamped to N): contiguous in S and B
    {
        const uint32_t nrows = N - n0 < kProjBN ? N - n0 : kProjBN;
        copy_pair_to_lds<kProjThreads>(S + (size_t)n0 * G, B + (size_t)n0 * G, s_lds, b_lds, nrows * G);
    }

    const uint8_t* wp0;
    const uint8_t* wp1;
    uint32_t sidx0, sidx1;           // this lane's two rows in the LDS scale/bias table
    {
        const uint32_t na = n0 + 64u * wave + col, nb = na + 32u;
        const uint32_t ra = na < N ? na : N - 1, rb = nb < N ? nb : N - 1;
        wp0 = W + (size_t)ra * row_bytes + 16u * h;
        wp1 = W + (size_t)rb * row_bytes + 16u * h;
        sidx0 = (ra - n0) * G;
        sidx1 = (rb - n0) * G;
    }
    // activation staging: thread t covers token row t/4, halves 16·(t%4) .. +15
    // of a group. Rows past M read row 0: their results are never stored.
    const uint32_t xrow = tid >> 2, xq = tid & 3u;
    const uint16_t* xp = X + (size_t)(m0 + xrow < M ? m0 + xrow : 0u) * K + 16u * xq;

    uint4 w0[kProjDepth], w1[kProjDepth], xa[kProjDepth], xb[kProjDepth];
    auto load = [&](uint32_t g, auto st_c) {
        constexpr int ST = decltype(st_c)::value;
        const uint32_t gg = g < G ? g : G - 1;
        w0[ST] = ldg16(wp0 + 32u * gg);          // plain loads: the 8 token tiles of an
        w1[ST] = ldg16(wp1 + 32u * gg);          // output slice share it through L2
        xa[ST] = *reinterpret_cast<const uint4*>(xp + 64u * gg);
        xb[ST] = *reinterpret_cast<const uint4*>(xp + 64u * gg + 8u);
    };
    auto store_x = [&](const uint4 va, const uint4 vb, _Float16* buf) {
        const h8 ha = X_BF16 ? bf16x8_to_f16(va) : __builtin_bit_cast(h8, va);
        const h8 hb = X_BF16 ? bf16x8_to_f16(vb) : __builtin_bit_cast(h8, vb);
        *reinterpret_cast<h8*>(&buf[xrow * kGemmLdsStride + 16u * xq]) = perm_0415(ha);
        *reinterpret_cast<h8*>(&buf[xrow * kGemmLdsStride + 16u * xq + 8u]) = perm_0415(hb);
    };
    // B operands of one group: [sub-tile j][k-step s]; two buffers so that the
    // next group's dequantisation overlaps this group's MFMAs
    h8 bw[2][2][4];
    auto dequant = [&](uint32_t g, const uint4 wa, const uint4 wb, h8 (&dst)[2][4]) {
        const uint32_t gg = g < G ? g : G - 1;
        dequant_chunk_f16_v(wa, s_lds[sidx0 + gg], b_lds[sidx0 + gg], magic_v, dst[0]);
        dequant_chunk_f16_v(wb, s_lds[sidx1 + gg], b_lds[sidx1 + gg], magic_v, dst[1]);
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Step for group g (compile-time ring stage ST = g % kProjDepth): its B
    // operands are in bw[ST & 1] (dequantised during the previous step), its
    // activations in LDS buffer ST & 1. The step refills the ring stage with
    // group g + kProjDepth, runs the 16 MFMAs of group g interleaved with the
    // dequantisation of group g + 1 and the staging of the activations of
    // group g + 1 into the other LDS buffer, then synchronises the block.
    // The main loop runs whole rounds with no branch inside, so the wait
    // analysis keeps exact load counts; the last K/64 mod kProjDepth groups
    // take the checked steps after it. Groups past the end are clamped re-reads
    // whose results nobody uses.
    auto step = [&](uint32_t g, auto st_c) {
        constexpr int ST = decltype(st_c)::value;
        constexpr int NX = (ST + 1) % kProjDepth;
        constexpr int P = ST & 1;
        const _Float16* cur = P ? xs1 : xs0;
        h8 a[2][4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i][s] = *reinterpret_cast<const h8*>(&cur[(32u * i + col) * kGemmLdsStride + 32u * h + 8u * s]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i][s], bw[P][j][s], acc[i][j], 0, 0, 0);
        dequant(g + 1, w0[NX], w1[NX], bw[P ^ 1]);
        store_x(xa[NX], xb[NX], P ? xs0 : xs1);
        load(g + kProjDepth, st_c);
        // interleave: each MFMA followed by a share of the VALU work
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);    // VALU
        }
        // keep the refill loads in this step (the scheduler would otherwise
        // sink them toward their use and shorten the prefetch)
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };
    load(0, std::integral_constant<int, 0>{});
    load(1, std::integral_constant<int, 1>{});
    load(2, std::integral_constant<int, 2>{});
    load(3, std::integral_constant<int, 3>{});
    store_x(xa[0], xb[0], xs0);
    __syncthreads();                 // scale/bias table and the first activations
    dequant(0, w0[0], w1[0], bw[0]);
    uint32_t g = 0;
    for (; g + kProjDepth <= G; g += kProjDepth) {
        step(g, std::integral_constant<int, 0>{});
        step(g + 1, std::integral_constant<int, 1>{});
        step(g + 2, std::integral_constant<int, 2>{});
        step(g + 3, std::integral_constant<int, 3>{});
    }
    if (g < G) step(g, std::integral_constant<int, 0>{});
    if (g + 1 < G) step(g + 1, std::integral_constant<int, 1>{});
    if (g + 2 < G) step(g + 2, std::integral_constant<int, 2>{});

    // D layout (32x32 tile): column = lane % 32, row = 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t n = n0 + 64u * wave + 32u * j + col;
        if (n >= N) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t m = m0 + 32u * i + 8u * (r >> 2) + 4u * h + (r & 3);
                if (m < M) {
                    const float v = acc[i][j][r];
                    Y[(size_t)m * N + n] = X_BF16 ? __builtin_bit_cast(uint16_t, (__bf16)v) : f2h(v);
                }
            }
    }
}

// Prefill projection: Y[t][n] = X[t] · W[n] for tokens t < M.
template <bool X_BF16>
__device__ __forceinline__ void gemm_q4(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                        const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
                                        uint16_t* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K) {
    __shared__ __attribute__((aligned(16))) GemmLds<1> L;
    __shared__ const uint16_t* rows_ptr[kGemmBM];
    const uint32_t m0 = blockIdx.y * kGemmBM;
    const uint32_t rows = M - m0 < (uint32_t)kGemmBM ? M - m0 : (uint32_t)kGemmBM;
    if (threadIdx.x < kGemmBM) rows_ptr[threadIdx.x] = X + (size_t)(m0 + threadIdx.x) * K;
    __syncthreads();
    const Q4Tile mats[1] = {{W, S, B}};
    gemm_tile<X_BF16, 1>(L, rows_ptr, rows, mats, blockIdx.x * kGemmBN, N, K,
                         [&](uint32_t j, uint32_t n, const float* v) {
                             Y[(size_t)(m0 + j) * N + n] =
                                 X_BF16 ? __builtin_bit_cast(uint16_t, (__bf16)v[0]) : f2h(v[0]);
                         });
}

}  // namespace tfq
