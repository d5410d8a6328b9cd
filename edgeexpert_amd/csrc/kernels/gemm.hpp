// gemm.hpp — dequant-fused int4 GEMM tile on the matrix cores, used by the
// prefill projection GEMM and by the grouped MoE prefill:
//     Y[t][n] = Σ_k X[t][k] · W[n][k]
// W affine int4 g64 with fp16 scale/bias, X fp16 (or bf16, converted),
// fp32 accumulate (S/Metal/TensorCore/tensorops.metal:13-105 and
// S/Metal/Prefill/prefill.metal:672-709 compute the same product). The
// 3-bit and 2-bit rows (prefill.metal:711-757,1223-1450) run the same tiles
// with the chunk load and unpack of common.hpp (template parameter BITS).
//
// Weights are dequantised in registers to fp16(q·s + b) with one rounding
// (v_pk_fma_f16 of the exact code q, the scale and the bias) — the fp16
// weight tile the reference's tensor-op kernel stages
// (tensorops.metal:57-80); dequant_word_sb gives the code order inside each
// 8-element run along K (4 bits: (0,2,1,3,4,6,5,7), through the gfx950 FP8
// conversion; 2 and 3 bits: (0,4,1,5,2,6,3,7)), and X is stored with the
// same permutation (unit_b_order), so each MFMA k-slice pairs the right
// operands (a dot product is order-free).
// bf16 activations are converted to fp16 while staging; the conversion is
// exact for |x| in [2^-14, 65504] (the range of the reference's fp16 path).
#pragma once

#include <type_traits>

#include "common.hpp"

namespace tfq {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmBM = 128;                      // rows of a grouped-MoE tile (grouping granule)
constexpr int kGemmBK = 64;
constexpr int kGemmLdsStride = kGemmBK + 8;       // halves per LDS row (16-byte pad)

// Permute one 8-element run from natural order to (0,4,1,5,2,6,3,7).
__device__ __forceinline__ h8 perm_0415(h8 v) {
    return __builtin_shufflevector(v, v, 0, 4, 1, 5, 2, 6, 3, 7);
}

// Permute one 8-element run from natural order to (0,2,1,3,4,6,5,7).
__device__ __forceinline__ h8 perm_0213(h8 v) {
    return __builtin_shufflevector(v, v, 0, 2, 1, 3, 4, 6, 5, 7);
}

// ------------------------------------------------------ projection tile ----
//
// The weights never pass through LDS: each lane loads its own row's 16 bytes
// of a group (the MFMA B operand of a 32-output sub-tile is 8 consecutive k
// of one output row per lane; lane half h: bytes 16h..16h+15, k-step s uses
// word s) straight into a register ring kProjDepth groups ahead, and
// dequantises them into B operands just before its MFMAs. The block's scales
// and biases are copied to LDS once at the start; the activations, shared
// by all waves, are converted (bf16 -> fp16) and permuted once per block
// into LDS. Every global load in the loop is unconditional (groups past the
// end re-read the last group, token rows past the end read row 0 and are
// not stored), so the compiler waits for exactly the group it consumes.
constexpr uint32_t kProjBM = 64;
constexpr uint32_t kProjBN = 256;
constexpr uint32_t kProjThreads = 256;
constexpr uint32_t kProjGemmThreads = 512;   // the prefill GEMM's eight-wave tile
constexpr uint32_t kProjDepth = 4;          // weight groups in flight per wave (register ring)
constexpr uint32_t kProjMaxK = 8192;        // scale/bias LDS: 256 rows x K/64 words

// What one lane of the projection tile streams: its two weight rows (the
// wave's 32-output sub-tiles 0 and 1; the lane's 16-byte half of each
// group already applied) and their rows in the block's LDS scale/bias table.
struct ProjLanes {
    const uint8_t* wp0;
    const uint8_t* wp1;
    uint32_t sidx0;
    uint32_t sidx1;
};

// ------------------------------------------- pipelined projection tile ----
//
// Every LDS round trip is off the group's critical path: three activation
// buffers, so that a group's A operands are read
// into registers one step before its MFMAs, and a scale/bias table of one
// word per (row, group) (scale | bias << 16) read two groups ahead. The only
// wait left in a step is its closing barrier, by which time the step's own
// LDS traffic has long completed. Step g: read A(g+1) and the scale/bias
// words of group g+2, run the 16 MFMAs of group g interleaved with the
// dequantisation of group g+1 (its B operands), stage the activations of
// group g+2, refill the rings, barrier.

// Dynamic LDS of the pipelined tile: three activation buffers, then the
// scale/bias table (kProjBN rows x K/64 words).
constexpr uint32_t proj_pl_lds_bytes(uint32_t K) {
    return 3u * kProjBM * kGemmLdsStride * 2u + 4u * kProjBN * (K / 64u);
}

// dst[i] = a[i] | b[i] << 16 for i < count, into LDS (16-byte loads and
// stores when the sources are 16-byte aligned and count % 8 == 0; U loads
// per thread and array in flight). tid: the thread's index in the block.
template <uint32_t NT, uint32_t U = 8>
__device__ __forceinline__ void copy_sb_to_lds(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                               uint32_t* __restrict__ dst, uint32_t count,
                                               uint32_t tid = threadIdx.x) {
    if (((((uintptr_t)a) | ((uintptr_t)b)) & 15u) == 0 && (count & 7u) == 0) {
        const uint32_t n16 = count >> 3;
        const uint4* sa = reinterpret_cast<const uint4*>(a);
        const uint4* sbp = reinterpret_cast<const uint4*>(b);
        uint4* t = reinterpret_cast<uint4*>(dst);
        for (uint32_t base = 0; base < n16; base += U * NT) {
            uint4 va[U], vb[U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t i = base + u * NT + tid;
                const uint32_t c = i < n16 ? i : n16 - 1;
                va[u] = sa[c];
                vb[u] = sbp[c];
            }
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
                const uint32_t i = base + u * NT + tid;
                if (i < n16) {
                    // v_perm: bytes 0-3 from the second operand, 4-7 from the first
                    t[2 * i] = make_uint4(__builtin_amdgcn_perm(vb[u].x, va[u].x, 0x05040100u),
                                          __builtin_amdgcn_perm(vb[u].x, va[u].x, 0x07060302u),
                                          __builtin_amdgcn_perm(vb[u].y, va[u].y, 0x05040100u),
                                          __builtin_amdgcn_perm(vb[u].y, va[u].y, 0x07060302u));
                    t[2 * i + 1] = make_uint4(__builtin_amdgcn_perm(vb[u].z, va[u].z, 0x05040100u),
                                              __builtin_amdgcn_perm(vb[u].z, va[u].z, 0x07060302u),
                                              __builtin_amdgcn_perm(vb[u].w, va[u].w, 0x05040100u),
                                              __builtin_amdgcn_perm(vb[u].w, va[u].w, 0x07060302u));
                }
            }
        }
    } else {
        for (uint32_t i = tid; i < count; i += NT) dst[i] = (uint32_t)a[i] | ((uint32_t)b[i] << 16);
    }
}

// Field i of a block word (codes 8j+i in the low half, 8j+i+4 in the high
// half, BITS bits each) read without a shift where it lies inside the fp16
// mantissa: OR-ed into the exponent of 2^(10-o) (o: the field's bit offset
// after an optional 8-bit shift of the word) it reads as 2^(10-o) + q, and
// one subtraction leaves q exactly. 4 bits: offsets 0, 4, 0, 4 (the upper
// two after a shift by 8); 3 bits: 0, 3, 6, then 1 after a shift; 2 bits: 0,
// 2, 4, 6.
template <int BITS>
struct DqField {
    static constexpr uint32_t shift(int i) { return (BITS == 4 && i >= 2) || (BITS == 3 && i == 3) ? 8u : 0u; }
    static constexpr uint32_t offset(int i) {
        return BITS == 4 ? 4u * (uint32_t)(i & 1) : BITS == 3 ? (i == 3 ? 1u : 3u * (uint32_t)i) : 2u * (uint32_t)i;
    }
    static constexpr uint32_t mask(int i) { return (((1u << BITS) - 1u) << offset(i)) * 0x00010001u; }
    static constexpr uint32_t magic(int i) { return ((25u - offset(i)) << 10) * 0x00010001u; }   // 2^(10-o) pairs
    static constexpr float base(int i) { return (float)(1u << (10u - offset(i))); }
};

// The magic pairs in VGPRs (v_and_or_b32 takes one scalar operand, the mask):
// fields with equal offsets share one register.
template <int BITS>
struct DequantConsts {
    uint32_t magic[4];
};

template <int BITS>
__device__ __forceinline__ DequantConsts<BITS> dequant_consts() {
    DequantConsts<BITS> dc;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (BITS == 4) {
            dc.magic[i] = 0;                 // the 4-bit path converts through FP8
        } else {
            uint32_t v;
            asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "i"(DqField<BITS>::magic(i)));
            dc.magic[i] = v;
        }
    }
    return dc;
}

// Word j of a chunk (codes 8j..8j+7) dequantised as fp16(q·s + b) with one
// rounding, s and b from one table word (scale | bias << 16). 4 bits: each
// code lands in the low nibble of a byte (word & 0x0F0F0F0F and its shift by
// 4), which read as an FP8 E4M3 number is q·2^-9 exactly (q < 8: subnormal
// q·2^-9; q >= 8: exponent field 1, (8 + (q-8))·2^-9); the gfx950
// conversion v_cvt_scalef32_pk_f16_fp8 with scale 2^9 turns two of them
// into the fp16 pair q exactly, in the code order (0,2,1,3,4,6,5,7)
// (unit_b_order). 2 and 3 bits: the fields of DqField, in the order
// (0,4,1,5,2,6,3,7).
template <int BITS>
__device__ __forceinline__ h8 dequant_word_sb(const QChunk<BITS>& w, int j, uint32_t sb, const DequantConsts<BITS>& dc) {
    const h2 s2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(sb, sb, 0x01000100u));
    const h2 b2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(sb, sb, 0x03020302u));
    uint32_t t = block_word<BITS>(w, j);
    h8 run;
    if constexpr (BITS == 4) {
        const uint32_t lo = t & 0x0F0F0F0Fu, hi = (t >> 4) & 0x0F0F0F0Fu;
        const h2 q[4] = {__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false),   // codes 0, 2
                         __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false),   // 1, 3
                         __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true),    // 4, 6
                         __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true)};   // 5, 7
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const h2 wv = __builtin_elementwise_fma(q[i], s2, b2);             // one rounding
            run[2 * i] = wv[0];
            run[2 * i + 1] = wv[1];
        }
    } else {
        asm("" : "+v"(t));
        const uint32_t t8 = t >> 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            using F = DqField<BITS>;
            const uint32_t src = F::shift(i) ? t8 : t;
            const uint32_t q = (src & F::mask(i)) | dc.magic[i];
            const h2 base = {(_Float16)F::base(i), (_Float16)F::base(i)};
            const h2 wv = __builtin_elementwise_fma(__builtin_bit_cast(h2, q) - base, s2, b2);   // exact q, one rounding
            run[2 * i] = wv[0];
            run[2 * i + 1] = wv[1];
        }
    }
    return run;
}

// The activation order that matches dequant_word_sb's code order.
template <int BITS>
__device__ __forceinline__ h8 unit_b_order(h8 v) {
    if constexpr (BITS == 4) return perm_0213(v);
    else return perm_0415(v);
}

// A chunk's four words dequantised with the scale and bias of one table word
// (dequant_word_sb per word: 4 bits in the code order of unit_b_order<4>).
template <int BITS>
__device__ __forceinline__ void dequant_chunk_sb(const QChunk<BITS>& w, uint32_t sb, const DequantConsts<BITS>& dc,
                                                 h8 (&out)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = dequant_word_sb<BITS>(w, j, sb, dc);
}

// The K loop of the pipelined tile. J = 32-output sub-tiles per wave: J = 2
// runs four waves; J = 1 runs eight waves (two per SIMD, so one wave's
// MFMAs overlap another's dequantisation and staging; a single wave does
// not overlap its own). With J = 1 a wave keeps two
// accumulator sets per token sub-tile (even and odd k-steps, summed at the
// end): a 32x32 MFMA chain on one accumulator issues at half rate, four
// independent chains per wave keep the matrix core busy; its A operands are
// then read at the start of each step (the other wave on the SIMD covers
// that wait) to stay within 256 registers. acc[i][j]: token sub-tile i, the
// wave's output sub-tile j; pl.wp0/sidx0 (and wp1/sidx1 for J = 2) index
// sb_lds, the table of `tcount` words tS[i] | tB[i] << 16 copied in here
// once the first groups' weight and activation loads are issued (so that the
// table's latency overlaps theirs) and published by the first barrier; xp:
// this thread's activation row (token row
// tid / (64/XH) of the block, clamped to a valid row) + XH·(tid % (64/XH))
// halves, XH = halves it stages per group. lds: the three activation buffers.
template <bool X_BF16, int J, int BITS = 4>
__device__ __forceinline__ void proj_core_pl(f32x16 (&acc)[2][J], _Float16* lds, uint32_t* sb_lds,
                                             const ProjLanes& pl, const uint16_t* __restrict__ xp, uint32_t G,
                                             const uint16_t* __restrict__ tS, const uint16_t* __restrict__ tB,
                                             uint32_t tcount) {
    constexpr uint32_t T = kProjBM * kGemmLdsStride;         // halves per activation buffer
    constexpr uint32_t NT = 64u * (8u / J);                  // threads of the block
    constexpr uint32_t XH = kProjBM * 64u / NT;              // activation halves staged per thread (16 or 8)
    constexpr uint32_t XV = XH / 8u;                         // of them, 16-byte pieces
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t h = lane >> 5, col = lane & 31u;
    const uint32_t xrow = tid / (64u / XH), xq = tid % (64u / XH);
    const DequantConsts<BITS> dc = dequant_consts<BITS>();

    constexpr int KS = J == 1 ? 2 : 1;                        // accumulator sets (k-step parity)
    constexpr int AB = J == 1 ? 1 : 2;                        // A-operand buffers
    QChunk<BITS> wr[J][kProjDepth];
    uint4 xr[2][XV];
    h8 a[AB][2][4];         // [group parity][token sub-tile][k-step]
    f32x16 accs[2][J][KS];
    h8 bw[2][J][4];         // [group parity][output sub-tile][k-step]
    uint32_t sbw[2][J];     // [group parity][output sub-tile]
    auto load_w = [&](uint32_t g, auto st_c) {
        constexpr int ST = decltype(st_c)::value;
        const uint32_t gg = g < G ? g : G - 1;
        wr[0][ST] = ldg_chunk<BITS, false>(pl.wp0, 2u * gg);
        if constexpr (J == 2) wr[J - 1][ST] = ldg_chunk<BITS, false>(pl.wp1, 2u * gg);
    };
    auto load_x = [&](uint32_t g, auto sl_c) {
        constexpr int SL = decltype(sl_c)::value;
        const uint32_t gg = g < G ? g : G - 1;
#pragma unroll
        for (uint32_t v = 0; v < XV; ++v) xr[SL][v] = ldg16_global(xp + 64u * gg + 8u * v);
    };
    auto buf = [&](uint32_t g) { return lds + (g % 3u) * T; };
    auto store_x = [&](const uint4 (&v)[XV], _Float16* dst) {
#pragma unroll
        for (uint32_t u = 0; u < XV; ++u) {
            const h8 hv = X_BF16 ? bf16x8_to_f16(v[u]) : __builtin_bit_cast(h8, v[u]);
            *reinterpret_cast<h8*>(&dst[xrow * kGemmLdsStride + XH * xq + 8u * u]) = unit_b_order<BITS>(hv);
        }
    };
    auto read_a = [&](const _Float16* src, h8 (&dst)[2][4]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
                dst[i][s] = *reinterpret_cast<const h8*>(&src[(32u * i + col) * kGemmLdsStride + 32u * h + 8u * s]);
    };
    auto read_sb = [&](uint32_t g, uint32_t (&dst)[J]) {
        const uint32_t gg = g < G ? g : G - 1;
        dst[0] = sb_lds[pl.sidx0 + gg];
        if constexpr (J == 2) dst[J - 1] = sb_lds[pl.sidx1 + gg];
    };
    auto dequant = [&](int st, const uint32_t (&sw)[J], h8 (&dst)[J][4]) {
#pragma unroll
        for (int j = 0; j < J; ++j) dequant_chunk_sb<BITS>(wr[j][st], sw[j], dc, dst[j]);
    };

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int k = 0; k < KS; ++k)
#pragma unroll
                for (int r = 0; r < 16; ++r) accs[i][j][k][r] = 0.0f;

    // Step g (compile-time weight-ring stage ST = g % kProjDepth, parity P =
    // ST & 1; the activation ring slot of group g + 2 is P as well).
    auto step = [&](uint32_t g, auto st_c) {
        constexpr int ST = decltype(st_c)::value;
        constexpr int NW = (ST + 1) % kProjDepth;
        constexpr int P = ST & 1;
        constexpr int PA = AB == 2 ? P : 0;
        if constexpr (AB == 2) read_a(buf(g + 1), a[P ^ 1]);
        else read_a(buf(g), a[0]);
        read_sb(g + 2, sbw[P]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < J; ++j)
                    accs[i][j][s % KS] =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(a[PA][i][s], bw[P][j][s], accs[i][j][s % KS], 0, 0, 0);
        dequant(NW, sbw[P ^ 1], bw[P ^ 1]);
        store_x(xr[P], buf(g + 2));
        load_w(g + kProjDepth, st_c);
        load_x(g + 4, std::integral_constant<int, P>{});
        __builtin_amdgcn_sched_group_barrier(0x100, 8 + J, 0);    // LDS reads first
#pragma unroll
        for (int m = 0; m < 8 * J; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);     // VALU
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };
    load_x(0, std::integral_constant<int, 0>{});
    load_x(1, std::integral_constant<int, 1>{});
    load_w(0, std::integral_constant<int, 0>{});
    load_w(1, std::integral_constant<int, 1>{});
    load_w(2, std::integral_constant<int, 2>{});
    load_w(3, std::integral_constant<int, 3>{});
    copy_sb_to_lds<NT, 3>(tS, tB, sb_lds, tcount);
    store_x(xr[0], buf(0));
    store_x(xr[1], buf(1));
    load_x(2, std::integral_constant<int, 0>{});
    load_x(3, std::integral_constant<int, 1>{});
    __syncthreads();                 // scale/bias table and the first two activation groups
    read_sb(0, sbw[0]);
    read_sb(1, sbw[1]);
    if constexpr (AB == 2) read_a(buf(0), a[0]);
    dequant(0, sbw[0], bw[0]);
    // no LDS read may be pending at the loop head, or the wait analysis keeps
    // waiting for the prologue's reads in every iteration (lgkmcnt(0))
    __builtin_amdgcn_s_waitcnt(0xC07F);
    uint32_t g = 0;
    for (; g + kProjDepth <= G; g += kProjDepth) {
        step(g, std::integral_constant<int, 0>{});
        step(g + 1, std::integral_constant<int, 1>{});
        step(g + 2, std::integral_constant<int, 2>{});
        step(g + 3, std::integral_constant<int, 3>{});
    }
    // the remaining groups nested (each step inside the branch of the one
    // before), so that their waits count the ring's loads exactly
    if (g < G) {
        step(g, std::integral_constant<int, 0>{});
        if (g + 1 < G) {
            step(g + 1, std::integral_constant<int, 1>{});
            if (g + 2 < G) step(g + 2, std::integral_constant<int, 2>{});
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j) {
            acc[i][j] = accs[i][j][0];
#pragma unroll
            for (int k = 1; k < KS; ++k) acc[i][j] += accs[i][j][k];
        }
}

// Calls fn(m, n, v) for every element of the tile held by this lane:
// m = token row in the block (0..63), n = output in the block (the wave's
// 32·J-output slice), per the 32x32 MFMA D layout (column = lane % 32,
// row = 8*(r/4) + 4*(lane/32) + r%4).
template <int J, int MI, typename Fn>
__device__ __forceinline__ void proj_for_each(const f32x16 (&acc)[MI][J], Fn fn) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                fn(32u * i + 8u * (r >> 2) + 4u * (lane >> 5) + (r & 3), 32u * J * wave + 32u * j + (lane & 31u),
                   acc[i][j][r]);
}

// Lanes of a wave over the outputs n_base + 32·J·wave_in_mat + 32j + lane%32
// (j < J) of a matrix with `nrows` outputs (clamped to the last one), rows of
// row_bytes (K·BITS/8), the table rows of those outputs starting at
// table_base. The lane's half h of each 64-code group is chunk 2g + h.
template <int J, int BITS = 4>
__device__ __forceinline__ ProjLanes proj_lanes(const uint8_t* W, uint32_t row_bytes, uint32_t n_base,
                                                uint32_t wave_in_mat, uint32_t nrows, uint32_t table_base,
                                                uint32_t G) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t h = lane >> 5, col = lane & 31u;
    ProjLanes pl;
    const uint32_t na = n_base + 32u * J * wave_in_mat + col, nb = na + 32u;
    const uint32_t ra = na < nrows ? na : nrows - 1, rb = nb < nrows ? nb : nrows - 1;
    pl.wp0 = W + (size_t)ra * row_bytes + 4u * BITS * h;
    pl.wp1 = W + (size_t)rb * row_bytes + 4u * BITS * h;
    pl.sidx0 = (table_base + ra - n_base) * G;
    pl.sidx1 = (table_base + rb - n_base) * G;
    return pl;
}

// Eight waves (kProjGemmThreads), one 32-output sub-tile each; BITS-bit rows.
// Row t of X starts at X + t·ldx, row t of Y at Y + t·ldy (halves).
template <bool X_BF16, int BITS = 4>
__device__ __forceinline__ void gemm_q4_proj(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                             const uint16_t* __restrict__ S, const uint16_t* __restrict__ B,
                                             uint16_t* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
                                             uint32_t ldx, uint32_t ldy) {
    extern __shared__ __attribute__((aligned(16))) _Float16 proj_lds[];
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    const uint32_t G = K >> 6;
    const uint32_t n0 = blockIdx.x * kProjBN, m0 = blockIdx.y * kProjBM;
    uint32_t* sb_lds = reinterpret_cast<uint32_t*>(proj_lds + 3 * kProjBM * kGemmLdsStride);
    // scales / biases of rows n0 .. n0+255 (clamped to N): contiguous in S and B
    const uint32_t nrows = N - n0 < kProjBN ? N - n0 : kProjBN;
    const ProjLanes pl = proj_lanes<1, BITS>(W, (K >> 3) * BITS, n0, wave, N, 0, G);
    // token rows past M read row 0: their results are never stored
    const uint32_t xrow = tid >> 3;
    const uint16_t* xp = X + (size_t)(m0 + xrow < M ? m0 + xrow : 0u) * ldx + 8u * (tid & 7u);
    f32x16 acc[2][1];
    proj_core_pl<X_BF16, 1, BITS>(acc, proj_lds, sb_lds, pl, xp, G, S + (size_t)n0 * G, B + (size_t)n0 * G,
                                  nrows * G);
    proj_for_each<1>(acc, [&](uint32_t m, uint32_t n, float v) {
        if (m0 + m < M && n0 + n < N)
            Y[(size_t)(m0 + m) * ldy + n0 + n] = X_BF16 ? __builtin_bit_cast(uint16_t, (__bf16)v) : f2h(v);
    });
}

}  // namespace tfq
