// gemm_skinny.hpp — the prefill projection GEMM for a few tokens:
//     Y[t][n] = Σ_k X[t][k] · W[n][k],  t < M (small), W affine g64 (2/3/4-bit)
//
// The 64-token projection tile (gemm.hpp) gives every block 256 outputs and
// the whole K loop, so below a few hundred tokens most of the chip idles
// (N/256 blocks per token tile) and each block's per-group barriers set the
// pace. For few tokens the work is a weight stream instead: each weight is
// dequantised once and multiplied with at most 16 tokens, on the matrix
// cores with v_mfma_f32_16x16x32_f16 whose A operand is 16 weight rows and
// whose B operand is 16 tokens.
//
// Block: 8 wavefronts over the same 16·RT rows, wave w taking the 128-code
// tiles w, w+8, w+16, … of K (CNT = ceil(K/1024) tiles each) (a split of K inside the block, so a block's
// rows are finished in one pass over K/8 per wave and the grid has N/(16·RT)
// blocks of 8 independent streams). Lane l of a wave owns row l%16 of each
// of its RT 16-row MFMA tiles and the quarter q = l/16 of every 128-code
// tile: chunk 4T+q (32 codes, one 16-byte load at 4 bits). Word j of that
// chunk feeds k-step j of the tile; the unpack yields codes in the order
// (0,4,1,5,2,6,3,7) within each 8-code run, so the B lane (token l%16,
// quarter q) loads the matching 32 activations (64 bytes, L2-resident:
// every row block reads the same X) and permutes them the same way. The
// weights are dequantised exactly as in the projection tile
// (dequant_chunk_sb: fp16(q·s + b), one rounding), so both paths multiply
// the same fp16 weights. Nothing is staged in LDS except the final sum of
// the eight K-slices (fixed wave order: deterministic).
#pragma once

#include "gemm.hpp"

namespace tfq {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kSkinnyThreads = 512;   // 8 wavefronts per block
constexpr uint32_t kSkinnyWaves = kSkinnyThreads / 64;
constexpr uint32_t kSkinnyTok = 16;        // tokens per blockIdx.y (the MFMA's N)

// One 128-code tile of a lane: its chunk of each of the RT rows with the
// group's raw fp16 scale and bias (combined only where they are used, so no
// wait for them sits ahead of an earlier tile's work), the 32 activations of
// its token, and a mask that zeroes both operands of a chunk past the row end.
template <int RT, int BITS>
struct SkinnyStage {
    QChunk<BITS> w[RT];
    uint32_t s[RT], b[RT];
    uint4 x[4];
    uint32_t mask;
};

__device__ __forceinline__ h8 mask_h8(h8 v, uint32_t mask) {
    u32x4 u = __builtin_bit_cast(u32x4, v);
    u &= mask;
    return __builtin_bit_cast(h8, u);
}

// RT: 16-row MFMA tiles per wave (1 or 2); X_BF16: X and Y in bf16 (else
// fp16); rows of X and Y ldx and ldy halves apart; CNT: 128-code tiles per wave, ceil(K / 1024) (a compile-time count,
// so the loop unrolls and every wait names exactly the tile it needs).
template <bool X_BF16, int RT, int BITS, int CNT>
__device__ __forceinline__ void gemm_skinny(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                            const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
                                            uint16_t* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
                                            uint32_t ldx, uint32_t ldy) {
    __shared__ f32x4 red[kSkinnyWaves][RT][64];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t r16 = lane & 15u, q = lane >> 4;
    const uint32_t nch = K >> 5;                       // 32-code chunks per row
    const uint32_t G = K >> 6;
    const uint32_t row_bytes = (K >> 3) * BITS;
    const uint32_t n0 = blockIdx.x * (16u * RT);
    const uint32_t t0 = blockIdx.y * kSkinnyTok;

    const uint8_t* wrow[RT];
    const uint16_t* srow[RT];
    const uint16_t* brow[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        const uint32_t r = n0 + 16u * i + r16, rc = r < N ? r : N - 1;     // rows past N: clamped, not stored
        wrow[i] = W + (size_t)rc * row_bytes;
        srow[i] = S + (size_t)rc * G;
        brow[i] = B + (size_t)rc * G;
    }
    const uint32_t t = t0 + r16, tc = t < M ? t : M - 1;                  // tokens past M: clamped, not stored
    const uint16_t* xrow = X + (size_t)tc * ldx;

    const DequantConsts<BITS> dc = dequant_consts<BITS>();

    // tile m of this wave is tile wave + 8m of the row; a chunk past the row
    // end (the half-filled last tile, or a wave with fewer tiles) re-reads a
    // valid chunk and is masked to zero
    auto load = [&](uint32_t m, SkinnyStage<RT, BITS>& st) {
        const uint32_t c = 4u * (wave + kSkinnyWaves * m) + q;
        st.mask = c < nch ? 0xFFFFFFFFu : 0u;
        const uint32_t cc = c < nch ? c : nch - 1;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            st.w[i] = ldg_chunk<BITS, false>(wrow[i], cc);
            st.s[i] = srow[i][cc >> 1];
            st.b[i] = brow[i][cc >> 1];
        }
        const uint4* xp = reinterpret_cast<const uint4*>(xrow + 32u * cc);
#pragma unroll
        for (int j = 0; j < 4; ++j) st.x[j] = xp[j];
    };
    f32x4 acc[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const SkinnyStage<RT, BITS>& st) {
        h8 a[RT][4];
#pragma unroll
        for (int i = 0; i < RT; ++i) dequant_chunk_sb<BITS>(st.w[i], st.s[i] | (st.b[i] << 16), dc, a[i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const h8 xv = X_BF16 ? bf16x8_to_f16(st.x[j]) : __builtin_bit_cast(h8, st.x[j]);
            const h8 b = mask_h8(unit_b_order<BITS>(xv), st.mask);
#pragma unroll
            for (int i = 0; i < RT; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(mask_h8(a[i][j], st.mask), b, acc[i], 0, 0, 0);
        }
    };
    // up to four tiles in flight: tile m + D is requested as soon as tile m
    // has been consumed
    constexpr int D = CNT < 4 ? CNT : 4;
    SkinnyStage<RT, BITS> st[D];
#pragma unroll
    for (int m = 0; m < D; ++m) load(m, st[m]);
    // keep every load ahead of the first use (the scheduler would otherwise
    // sink later tiles' loads into the first tile's compute)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < CNT; ++m) {
        compute(st[m % D]);
        if (m + D < CNT) load(m + D, st[m % D]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // sum of the eight K-slices, in wave order
#pragma unroll
    for (int i = 0; i < RT; ++i) red[wave][i][lane] = acc[i];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
        f32x4 v = red[0][i][lane];
#pragma unroll
        for (uint32_t w = 1; w < kSkinnyWaves; ++w) v += red[w][i][lane];
        // D layout of the 16x16 MFMA: column = lane % 16 (token), rows 4·(lane/16) + r
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t n = n0 + 16u * i + 4u * q + r;
            if (n < N && t < M)
                Y[(size_t)t * ldy + n] = X_BF16 ? __builtin_bit_cast(uint16_t, (__bf16)v[r]) : f2h(v[r]);
        }
    }
}

}  // namespace tfq
