// common.hpp — shared device helpers for the gfx950 quantized-matmul kernels.
//
// Wave64 throughout: a "segment" is a power-of-two group of SEG lanes inside
// one wavefront that cooperates on one output row; several segments share a
// wave when a row needs fewer than 64 lanes.
//
// Block sizes are compile-time constants (template parameter NT, default
// kThreads): reading blockDim.x costs a load from the dispatch's implicit
// arguments, and the wait for it would sit in front of every kernel's first
// weight load.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "abi_types.h"

namespace tfq {

constexpr int kGroup = 64;        // affine group size along the reduction axis
constexpr int kWave = 64;         // CDNA wavefront width
constexpr uint32_t kThreads = 256;     // threads per block of every GEMV-family kernel

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// fp32 -> fp16, round to nearest even (v_cvt_f16_f32 under the default mode).
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float bf2f(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
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

// Cross-lane reductions on the VALU (DPP row permutations and the gfx950
// permlane swaps) instead of LDS permutes: a few cycles per step rather than
// an LDS round trip. Every lane receives the result; the pairing is fixed, so
// results are deterministic (and commutative pairs make them equal in every
// lane). Row = 16 aligned lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppRowMirror = 0x140;       // lane i <-> 15 - i
constexpr int kDppRowHalfMirror = 0x141;   // lane i <-> 7 - i within each 8
constexpr int kDppQuadSwap2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppQuadSwap1 = 0xB1;        // quad_perm [1,0,3,2]

// After the mirror and half-mirror steps lane i of a row holds the sum of
// lanes {i, 7-i, 8+i, 15-i} (mod the row); the two quad swaps add the four
// disjoint such sets of a quad together.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<kDppRowMirror>(v);
    v += dpp_mov<kDppRowHalfMirror>(v);
    v += dpp_mov<kDppQuadSwap2>(v);
    v += dpp_mov<kDppQuadSwap1>(v);
    return v;
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t row16_sum_u32(uint32_t v) {
    v += dpp_mov_u32<kDppRowMirror>(v);
    v += dpp_mov_u32<kDppRowHalfMirror>(v);
    v += dpp_mov_u32<kDppQuadSwap2>(v);
    v += dpp_mov_u32<kDppQuadSwap1>(v);
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_mov<kDppRowMirror>(v));
    v = fmaxf(v, dpp_mov<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_mov<kDppQuadSwap2>(v));
    v = fmaxf(v, dpp_mov<kDppQuadSwap1>(v));
    return v;
}

// v_permlane16_swap with both operands = x leaves (row0, row0, row2, row2) in
// one result and (row1, row1, row3, row3) in the other; v_permlane32_swap does
// the same for the two 32-lane halves. Applied to row-uniform values they
// combine rows pairwise, then halves.
template <bool MAX>
__device__ __forceinline__ float rows_combine(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const auto p = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const float x0 = __builtin_bit_cast(float, (uint32_t)p[0]), x1 = __builtin_bit_cast(float, (uint32_t)p[1]);
    v = MAX ? fmaxf(x0, x1) : x0 + x1;
    const uint32_t c = __builtin_bit_cast(uint32_t, v);
    const auto q = __builtin_amdgcn_permlane32_swap(c, c, false, false);
    const float y0 = __builtin_bit_cast(float, (uint32_t)q[0]), y1 = __builtin_bit_cast(float, (uint32_t)q[1]);
    return MAX ? fmaxf(y0, y1) : y0 + y1;
}
__device__ __forceinline__ float wave_sum(float v) { return rows_combine<false>(row16_sum(v)); }
__device__ __forceinline__ float wave_max(float v) { return rows_combine<true>(row16_max(v)); }

// Sum over the SEG lanes of a segment (SEG a power of two, aligned); every
// lane of the segment receives the total, bit-identical in every lane. The
// steps stay inside the segment, so segments of one wave may hold different
// rows (or have left a loop the others continue), and the order of additions
// is fixed (deterministic).
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
    static_assert(SEG == 1 || SEG == 2 || SEG == 4 || SEG == 8 || SEG == 16 || SEG == 32 || SEG == 64,
                  "segment of 1..64 lanes");
    if constexpr (SEG == 16) {
        return row16_sum(v);
    } else if constexpr (SEG == 32) {
        const uint32_t b = __builtin_bit_cast(uint32_t, row16_sum(v));
        const auto p = __builtin_amdgcn_permlane16_swap(b, b, false, false);
        return __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
    } else if constexpr (SEG == 64) {
        return wave_sum(v);
    } else {
        if constexpr (SEG >= 8) v += dpp_mov<kDppRowHalfMirror>(v);
        if constexpr (SEG >= 4) v += dpp_mov<kDppQuadSwap2>(v);
        if constexpr (SEG >= 2) v += dpp_mov<kDppQuadSwap1>(v);
        return v;
    }
}

// gelu_pytorch_tanh with the inner argument clamped to ±20
// (S/Metal/MoE/moe.metal:53-60; the clamp is exact at fp32 saturation).
// GELU, tanh form: 0.5·x·(1 + tanh(z)), z = sqrt(2/pi)·(x + 0.044715·x^3),
// evaluated as x / (1 + e^(-2z)) (the same function: 0.5·(1 + tanh z) is
// the logistic of 2z) with the hardware exp2 and reciprocal, ~1e-7
// relative. Large negative x: e^(-2z) overflows to inf and the result is
// -0; large positive x: x.
__device__ __forceinline__ float gelu_tanh(float x) {
    constexpr float kC = -2.0f * 0.7978845608028654f * 1.4426950408889634f;   // -2·sqrt(2/pi)·log2(e)
    constexpr float kC3 = kC * 0.044715f;
    const float e = __builtin_amdgcn_exp2f(x * fmaf(kC3, x * x, kC));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ uint4 ldg16(const uint8_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

// 16-byte load through a pointer the compiler cannot prove global (one read
// from LDS, say): naming the global address space makes it a global_load,
// counted by vmcnt only, instead of a flat load, whose completion every LDS
// wait (lgkmcnt) would also have to wait for.
typedef __attribute__((address_space(1))) const uint4 global_uint4;
__device__ __forceinline__ uint4 ldg16_global(const void* p) {
    return *reinterpret_cast<global_uint4*>(reinterpret_cast<uintptr_t>(p));
}

// 128-bit load of weights that are read once per token: non-temporal, so the
// stream does not evict the activations and small vectors the caches hold.
__device__ __forceinline__ uint4 ldg16_stream(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ------------------------------------------------------------ int4 chunk ----
//
// A chunk is 16 bytes of a weight row: 32 int4 codes, four 32-bit words, code
// 8j+i in bits 4i..4i+3 of word j. Masking a word with 0x000F000F keeps codes
// 8j (low half) and 8j+4 (high half) in mantissa bits 0-3 of two fp16
// lanes; OR-ing 0x6400 makes them the exact fp16 values 1024 + q. Masking
// with 0x00F000F0 keeps codes 8j+1 / 8j+5 in mantissa bits 4-7: 1024 + 16q,
// also exact. The word shifted right by 8 gives codes 8j+2 / 8j+6 and
// 8j+3 / 8j+7 the same way. So a word costs 5 bit operations for its 8
// codes; v_dot2_f32_f16 multiplies each fp16 pair with the matching
// activation pair (exact products) and accumulates in fp32, into accA for
// the 1024 + q form and accB for the 1024 + 16q form. The offsets are
// removed per chunk with the activation sums of the two position classes:
//     Σ q·x = (accA − 1024·SA) + (accB − 1024·SB) / 16.
// The activations of a chunk are therefore held as 16 fp16 pairs
// xp[4j+i] = (x[8j+i], x[8j+i+4]).

struct XChunk {
    h2 p[16];
    float sum;      // Σ of the 32 activations (fp32)
    float ca;       // 1024 · Σ of the activations at positions 8j+{0,2,4,6}
    float cb;       // 1024 · Σ of the activations at positions 8j+{1,3,5,7}
};

// The activations of the int4 dot as the dot consumes them, in LDS (so the
// x values need no registers of their own across the row loop, which keeps
// the GEMV kernels' register count, and with it their occupancy, in check).
// Chunk c (32 values) is stored as 4 planes of 16 bytes, plane j holding the
// pairs (v[8j+i], v[8j+i+4]) for i = 0..3 at byte 16·(j·nch + c): lanes that
// read consecutive chunks read consecutive 16-byte slots. sums[c] holds the
// chunk's (sum, ca, cb, 0).
struct XPairs {
    const uint4* planes;
    const float4* sums;
    uint32_t nch;
};

// The per-16-byte part of a chunk's sums: Σ of the 8 values and of the 4 at
// even / odd positions, in element order.
__device__ __forceinline__ void h8_sums(const h8 v, float& s, float& sa, float& sb) {
    s = 0.0f;
    sa = 0.0f;
    sb = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        s += (float)v[e];
        if (e & 1) sb += (float)v[e];
        else sa += (float)v[e];
    }
}

__device__ __forceinline__ uint4 h8_pairs(const h8 v) {
    return make_uint4(__builtin_bit_cast(uint32_t, __builtin_shufflevector(v, v, 0, 4)),
                      __builtin_bit_cast(uint32_t, __builtin_shufflevector(v, v, 1, 5)),
                      __builtin_bit_cast(uint32_t, __builtin_shufflevector(v, v, 2, 6)),
                      __builtin_bit_cast(uint32_t, __builtin_shufflevector(v, v, 3, 7)));
}

// The chunk sums of 16-byte piece q (= 4c + j) combine over the four pieces of
// chunk c as (p0 + p1) + (p2 + p3).
// Lane ^ 1, then lane ^ 2 inside the quad (the same sums either way): on DPP
// quad permutations, or (DPP == false) on LDS permutes, which measured
// faster where the staging holds four pieces per thread (routed phase 2).
template <bool DPP = true>
__device__ __forceinline__ float4 chunk_sums(const float s, const float sa, const float sb) {
    auto x1 = [](float v) { return DPP ? dpp_mov<kDppQuadSwap1>(v) : __shfl_xor(v, 1, kWave); };
    auto x2 = [](float v) { return DPP ? dpp_mov<kDppQuadSwap2>(v) : __shfl_xor(v, 2, kWave); };
    float t = s + x1(s);
    float ta = sa + x1(sa);
    float tb = sb + x1(sb);
    t += x2(t);
    ta += x2(ta);
    tb += x2(tb);
    return make_float4(t, 1024.0f * ta, 1024.0f * tb, 0.0f);
}

// Builds the paired copy of the n staged halves at lds_xh into the LDS that
// follows them (layout of xpairs_lds_bytes): one 16-byte piece per thread and
// step, the four pieces of a chunk in four consecutive lanes. Every thread of
// the block calls it after staging; it ends with a barrier.
template <uint32_t NT = kThreads>
__device__ __forceinline__ XPairs build_xpairs(uint16_t* lds_xh, uint32_t n) {
    const uint32_t nch = n >> 5, npc = n >> 3;
    uint4* planes = reinterpret_cast<uint4*>(lds_xh + n);
    float4* sums = reinterpret_cast<float4*>(planes + 4 * nch);
    for (uint32_t base = 0; base < npc; base += NT) {
        const uint32_t q = base + threadIdx.x;      // npc is a multiple of 8: a chunk's pieces are all live or all not
        const h8 v = q < npc ? reinterpret_cast<const h8*>(lds_xh)[q] : h8{};
        float s, sa, sb;
        h8_sums(v, s, sa, sb);
        const float4 cs = chunk_sums(s, sa, sb);
        if (q < npc) {
            planes[(q & 3u) * nch + (q >> 2)] = h8_pairs(v);
            if ((q & 3u) == 0) sums[q >> 2] = cs;
        }
    }
    __syncthreads();
    return {planes, sums, nch};
}

__device__ __forceinline__ void read_xpairs(const XPairs& xp, uint32_t c, XChunk& xc) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 v = xp.planes[j * xp.nch + c];
        xc.p[4 * j + 0] = __builtin_bit_cast(h2, v.x);
        xc.p[4 * j + 1] = __builtin_bit_cast(h2, v.y);
        xc.p[4 * j + 2] = __builtin_bit_cast(h2, v.z);
        xc.p[4 * j + 3] = __builtin_bit_cast(h2, v.w);
    }
    const float4 s = xp.sums[c];
    xc.sum = s.x;
    xc.ca = s.y;
    xc.cb = s.z;
}

// ------------------------------------------------- 2-, 3- and 4-bit chunks ----
//
// The 32 codes of activation chunk c (positions 32c..32c+31) take 4·BITS
// bytes of a BITS-bit row, codes packed from the least significant bit up
// (S/Infrastructure/ModelIO/Quantization.swift:198-201,296-320): 16 bytes at
// 4 bits, 12 at 3 bits (code i of the chunk in bits 3i..3i+2 of the 96-bit
// little-endian value), 8 at 2 bits. Chunk c of a row starts at byte
// 4·BITS·c, so a lane's chunk is one 128-, 96- or 64-bit load.
template <int BITS>
struct QChunk {
    uint32_t w[BITS];
};

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Non-temporal load of chunk c of a row (4-byte aligned for every BITS: rows
// of n codes start at multiples of n·BITS/8, a multiple of 8 bytes for n %
// 64 == 0, and chunks at multiples of 4·BITS). Three separate words at 3
// bits: a 3-wide vector load may be widened to 16 bytes, past the row.
// STREAM: non-temporal (weights read once per token); plain loads where
// several token tiles share the rows through L2 (the prefill tiles).
template <int BITS, bool STREAM = true>
__device__ __forceinline__ QChunk<BITS> ldg_chunk(const uint8_t* row, uint32_t c) {
    QChunk<BITS> q;
    const uint8_t* p = row + 4u * BITS * c;
    if constexpr (BITS == 4) {
        const uint4 v = STREAM ? ldg16_stream(p) : ldg16(p);
        q.w[0] = v.x;
        q.w[1] = v.y;
        q.w[2] = v.z;
        q.w[3] = v.w;
    } else if constexpr (BITS == 2) {
        const u32x2* vp = reinterpret_cast<const u32x2*>(p);
        const u32x2 v = STREAM ? __builtin_nontemporal_load(vp) : *vp;
        q.w[0] = v.x;
        q.w[1] = v.y;
    } else {
        static_assert(BITS == 3, "2, 3 or 4 bits");
        const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
        for (int i = 0; i < 3; ++i) q.w[i] = STREAM ? __builtin_nontemporal_load(w + i) : w[i];
    }
    return q;
}

// Plain load of the chunk at byte offset off of a block-uniform base: the
// 32-bit offset keeps the address in one vector register over the scalar
// base (the scalar-base form of global_load).
template <int BITS>
__device__ __forceinline__ QChunk<BITS> ldg_chunk_at(const uint8_t* __restrict__ base, uint32_t off) {
    QChunk<BITS> q;
    if constexpr (BITS == 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(base + off);
        q.w[0] = v.x;
        q.w[1] = v.y;
        q.w[2] = v.z;
        q.w[3] = v.w;
    } else if constexpr (BITS == 2) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(base + off);
        q.w[0] = v.x;
        q.w[1] = v.y;
    } else {
        static_assert(BITS == 3, "2, 3 or 4 bits");
        // one pointer for the three words, so that they merge into one
        // 12-byte load (three 32-bit offsets could wrap apart)
        const uint32_t* w = reinterpret_cast<const uint32_t*>(base + off);
#pragma unroll
        for (int i = 0; i < 3; ++i) q.w[i] = w[i];
    }
    return q;
}

// Codes 8j..8j+7 of a chunk in the int4 word form: a word whose low half
// holds codes 8j..8j+3 and whose high half holds 8j+4..8j+7, at BITS-bit
// spacing from bit 0 and bit 16 (bits between or above the codes may hold
// anything; the dot masks them off).
template <int BITS>
__device__ __forceinline__ uint32_t block_word(const QChunk<BITS>& q, int j) {
    if constexpr (BITS == 4) {
        return q.w[j];
    } else if constexpr (BITS == 2) {
        // byte 2(j&1) -> byte 0, byte 2(j&1)+1 -> byte 2 of the result
        const uint32_t w = q.w[j >> 1];
        return __builtin_amdgcn_perm(w, w, (j & 1) ? 0x03030202u : 0x01010000u);
    } else {
        // the 24 bits of codes 8j..8j+7 start at bit 24j of the 96-bit chunk
        // (v_alignbit_b32 on 32-bit halves: a 64-bit shift of the words lets
        // the compiler fuse their reads into one 64-bit access, which keeps
        // the chunk arrays in scratch memory)
        uint32_t u;
        if (j == 0) u = q.w[0];
        else if (j == 1) u = __builtin_amdgcn_alignbit(q.w[1], q.w[0], 24);
        else if (j == 2) u = __builtin_amdgcn_alignbit(q.w[2], q.w[1], 16);
        else u = q.w[2] >> 8;
        // codes 4..7 (bits 12..23) move up to bits 16..27
        return (u & 0x0000FFFFu) | ((u << 4) & 0xFFFF0000u);
    }
}

// Σ_k q_k x_k over the 32 codes of a BITS-bit chunk (fp32 accumulate), the
// int4 dot generalised: with t = block_word(j) and M = 2^BITS − 1 in both
// halves, (t & M) | 0x6400 pairs give codes 8j, 8j+4 as 1024 + q and
// (t & M<<BITS) | 0x6400 gives 8j+1, 8j+5 as 1024 + 2^BITS·q (all exact
// fp16); t >> 2·BITS gives 8j+2, 8j+6 and 8j+3, 8j+7 the same way. The
// activation pairs and offsets are the int4 chunk's, so
//     Σ q·x = (accA − ca) + (accB − cb) / 2^BITS.
// MAGIC_V: the magic 0x64006400 sits in a VGPR. gfx950's VOP3 encodings
// take no literal, so with both the mask and the magic as literals each pair
// costs a v_and_b32 and a v_or_b32; with the mask in an SGPR and the magic in
// a VGPR it is one v_and_or_b32 (which kernel runs faster with which form is
// measured, not assumed: the schedules differ).
template <int BITS, bool MAGIC_V = true>
__device__ __forceinline__ float dot_chunk(const QChunk<BITS>& q, const XChunk& xc) {
    constexpr uint32_t M = (1u << BITS) - 1u;
    constexpr uint32_t MA = M | (M << 16);
    constexpr uint32_t MB = MA << BITS;
    uint32_t magic = 0x64006400u;
    if constexpr (MAGIC_V) asm("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    float acc_a = 0.0f, acc_b = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t t = block_word<BITS>(q, j);
        // opaque to the optimiser: otherwise it distributes the masks below
        // over the shifts and merges that built t (3-bit: ~50% more bit ops
        // than the one v_and_or_b32 per pair)
        if constexpr (BITS != 4) asm("" : "+v"(t));
        const uint32_t t2 = t >> (2 * BITS);
        const h2 q0 = __builtin_bit_cast(h2, (t & MA) | magic);
        const h2 q1 = __builtin_bit_cast(h2, (t & MB) | magic);
        const h2 q2 = __builtin_bit_cast(h2, (t2 & MA) | magic);
        const h2 q3 = __builtin_bit_cast(h2, (t2 & MB) | magic);
        acc_a = __builtin_amdgcn_fdot2(q0, xc.p[4 * j + 0], acc_a, false);
        acc_b = __builtin_amdgcn_fdot2(q1, xc.p[4 * j + 1], acc_b, false);
        acc_a = __builtin_amdgcn_fdot2(q2, xc.p[4 * j + 2], acc_a, false);
        acc_b = __builtin_amdgcn_fdot2(q3, xc.p[4 * j + 3], acc_b, false);
    }
    return fmaf(acc_b - xc.cb, 1.0f / (float)(1u << BITS), acc_a - xc.ca);
}

// Σ_i q_i * x_i over the 16 int8 codes of one 16-byte chunk, fp32 operands.
__device__ __forceinline__ float dot16_q8(const uint4 w, const float* x) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) d = fmaf((float)((ws[i] >> (8 * b)) & 0xFFu), x[4 * i + b], d);
    }
    return d;
}

// Sum of v over the block (every thread receives it); wave sums first, then
// the per-wave totals in wave order (deterministic).
template <uint32_t NT = kThreads>
__device__ __forceinline__ float block_sum(float v) {
    __shared__ float part[16];
    v = seg_sum<kWave>(v);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) part[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < NT / 64; ++i) t += part[i];
    return t;
}

// block_sums for a call site that runs once per kernel (TAG names its LDS
// array): no barrier is needed before the partials are written.
template <int N, uint32_t NT, int TAG>
__device__ __forceinline__ void block_sums_once(float (&v)[N]) {
    __shared__ float partn[16][N];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = seg_sum<kWave>(v[k]);
    if (lane == 0)
#pragma unroll
        for (int k = 0; k < N; ++k) partn[wave][k] = v[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < N; ++k) {
        float t = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < NT / 64; ++i) t += partn[i][k];
        v[k] = t;
    }
}

// N independent block sums at once (one pair of barriers for all of them).
template <int N, uint32_t NT = kThreads>
__device__ __forceinline__ void block_sums(float (&v)[N]) {
    __shared__ float partn[16][N];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = seg_sum<kWave>(v[k]);
    __syncthreads();
    if (lane == 0)
#pragma unroll
        for (int k = 0; k < N; ++k) partn[wave][k] = v[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < N; ++k) {
        float t = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < NT / 64; ++i) t += partn[i][k];
        v[k] = t;
    }
}

// 1/sqrt(mean(x^2) + eps) of an fp16 vector held in LDS
// (V/Reference/Primitives/RmsNorm.swift:18-22 in the reference checkout).
template <uint32_t NT = kThreads>
__device__ __forceinline__ float lds_inv_rms(const uint16_t* __restrict__ lds, uint32_t n, float eps) {
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += NT) {
        const float v = h2f(lds[i]);
        ss = fmaf(v, v, ss);
    }
    const float total = block_sum<NT>(ss);
    return 1.0f / sqrtf(total / (float)n + eps);
}

// Copies n fp16 values to LDS (16-byte transfers when x is 16-byte aligned;
// each thread issues up to four loads before its first store, so a copy of
// up to 4·8·NT values costs one memory latency). The loads use clamped
// (always valid) chunk indices and plain scalars, so the compiler keeps them
// in registers and in flight together.
template <uint32_t NT = kThreads>
__device__ __forceinline__ void copy_to_lds(const uint16_t* __restrict__ x, uint16_t* __restrict__ lds,
                                            uint32_t n) {
    if ((((uintptr_t)x) & 15u) == 0 && (n & 7u) == 0) {
        const uint4* src = reinterpret_cast<const uint4*>(x);
        uint4* dst = reinterpret_cast<uint4*>(lds);
        const uint32_t nch = n >> 3;
        if (nch == 0) return;
        for (uint32_t base = threadIdx.x; base < nch; base += 4 * NT) {
            const uint32_t c1 = base + NT, c2 = base + 2 * NT, c3 = base + 3 * NT;
            const uint4 v0 = src[base];
            const uint4 v1 = src[c1 < nch ? c1 : base];
            const uint4 v2 = src[c2 < nch ? c2 : base];
            const uint4 v3 = src[c3 < nch ? c3 : base];
            dst[base] = v0;
            if (c1 < nch) dst[c1] = v1;
            if (c2 < nch) dst[c2] = v2;
            if (c3 < nch) dst[c3] = v3;
        }
    } else {
        for (uint32_t i = threadIdx.x; i < n; i += NT) lds[i] = x[i];
    }
}

// lds[i] <- fp16(lds[i] * w[i] * r(lds)) in place (w == null: no scale);
// RmsNorm.swift:14-43 forms the product x·w first, then applies the scale.
template <uint32_t NT = kThreads>
__device__ __forceinline__ void rmsnorm_lds(uint16_t* __restrict__ lds, uint32_t n,
                                            const uint16_t* __restrict__ w, float eps) {
    const float inv = lds_inv_rms<NT>(lds, n, eps);
    for (uint32_t i = threadIdx.x; i < n; i += NT) {
        const float xw = w ? h2f(lds[i]) * h2f(w[i]) : h2f(lds[i]);
        lds[i] = f2h(xw * inv);
    }
    __syncthreads();
}

// Scalar form of the staging (any alignment, any n): the fp16 activation
// vector as NormArg describes, into lds[0..n).
template <uint32_t NT = kThreads>
__device__ __forceinline__ void stage_act_scalar(const uint16_t* __restrict__ x, uint16_t* __restrict__ lds,
                                                 uint32_t n, const NormArg& na) {
    copy_to_lds<NT>(x, lds, n);
    __syncthreads();
    if (na.mode == kStageTail) {
        float s3[3] = {0.0f, 0.0f, 0.0f};
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const float a = h2f(na.attn[i]), u = h2f(na.h1[i]), v = h2f(na.h2[i]);
            s3[0] = fmaf(a, a, s3[0]);
            s3[1] = fmaf(u, u, s3[1]);
            s3[2] = fmaf(v, v, s3[2]);
        }
        block_sums<3, NT>(s3);
        const float inv_a = 1.0f / sqrtf(s3[0] / (float)n + na.eps);
        const float inv_1 = 1.0f / sqrtf(s3[1] / (float)n + na.eps);
        const float inv_2 = 1.0f / sqrtf(s3[2] / (float)n + na.eps);
        auto h12_at = [&](uint32_t i) {
            const uint16_t a1 = f2h(h2f(na.h1[i]) * h2f(na.h1_w[i]) * inv_1);
            const uint16_t a2 = f2h(h2f(na.h2[i]) * h2f(na.h2_w[i]) * inv_2);
            return f2h(h2f(a1) + h2f(a2));
        };
        float s12 = 0.0f;
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const uint16_t an = f2h(h2f(na.attn[i]) * h2f(na.attn_w[i]) * inv_a);
            lds[i] = f2h(h2f(lds[i]) + h2f(an));
            const float h12 = h2f(h12_at(i));
            s12 = fmaf(h12, h12, s12);
        }
        const float inv_12 = 1.0f / sqrtf(block_sum<NT>(s12) / (float)n + na.eps);
        const float sc = (float)(_Float16)na.scalar;
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const uint16_t f2 = f2h(h2f(h12_at(i)) * h2f(na.ffn_w[i]) * inv_12);
            lds[i] = f2h(h2f(f2h(h2f(lds[i]) + h2f(f2))) * sc);
            if (na.export_h && blockIdx.x == 0) na.export_h[i] = lds[i];
        }
        __syncthreads();
        rmsnorm_lds<NT>(lds, n, na.w, na.eps);
        return;
    }
    if (na.mode == kStageBf16) {
        for (uint32_t i = threadIdx.x; i < n; i += NT) lds[i] = f2h(bf2f(lds[i]));
        __syncthreads();
        return;
    }
    if (na.mode == kStageScaled) {
        const float inv = *na.inv;
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const float xw = na.w ? h2f(lds[i]) * h2f(na.w[i]) : h2f(lds[i]);
            lds[i] = f2h(xw * inv);
        }
        __syncthreads();
        return;
    }
    if (na.mode == kStagePostAttn || na.mode == kStageResidual) {
        float ss = 0.0f;
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const float v = h2f(na.attn[i]);
            ss = fmaf(v, v, ss);
        }
        const float inv = 1.0f / sqrtf(block_sum<NT>(ss) / (float)n + na.eps);
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const uint16_t an = f2h(h2f(na.attn[i]) * h2f(na.attn_w[i]) * inv);
            lds[i] = f2h(h2f(lds[i]) + h2f(an));
        }
        __syncthreads();
    }
    if (na.mode == kStagePostAttn && na.export_h) {
        // h and r(h) for later kernels (kStageScaled), then the norm with that r(h)
        const float inv = lds_inv_rms<NT>(lds, n, na.eps);
        if (blockIdx.x == 0) {
            for (uint32_t i = threadIdx.x; i < n; i += NT) na.export_h[i] = lds[i];
            if (threadIdx.x == 0) *na.export_inv = inv;
        }
        for (uint32_t i = threadIdx.x; i < n; i += NT) {
            const float xw = na.w ? h2f(lds[i]) * h2f(na.w[i]) : h2f(lds[i]);
            lds[i] = f2h(xw * inv);
        }
        __syncthreads();
        return;
    }
    if (na.mode == kStageNorm || na.mode == kStagePostAttn) rmsnorm_lds<NT>(lds, n, na.w, na.eps);
}

__device__ __forceinline__ uint4 ld16h(const uint16_t* p, uint32_t chunk) {
    return reinterpret_cast<const uint4*>(p)[chunk];
}

// Staging of a kernel's activation vector in two steps, so that the loads of
// x (and of the norm inputs) are in flight together with the weight loads
// the kernel issues between the two:
//   load()   issues the 16-byte loads of every input chunk the thread owns
//            (chunks t, t + NT, …, CH per thread; vector path only);
//   pairs()  forms the vector as NormArg says (attention-output norm and
//            residual add, fused_post_attn_setup, S/Metal/Fusions/
//            fused.metal:199-231; RMSNorm) in registers and writes it to
//            LDS directly in the paired layout the int4 dot reads
//            (XPairs), plus the plain fp16 copy when `plain` is set;
//   plain()  the same, writing only the plain fp16 copy.
// Both end with a block barrier. Inputs that are not 16-byte aligned, or
// longer than 8·CH·NT halves, take the scalar path instead (two passes).
// NORM == false compiles the copy-only form (NormArg ignored).
// TAIL: the kStageTail form (its five extra input vectors in registers).
// FIXED >= 0: the staging mode, known at compile time, with the vector path's
// conditions guaranteed by the caller (16-byte aligned inputs, n a multiple
// of 8, n <= 8·CH·NT). No load then sits under a branch: a load under a
// branch makes the compiler's wait for it at the join cover every load
// issued after it, the weights included, which serialised the staging
// behind the weight stream (config 0's GEMV: 4.05 against 3.60 us).
template <uint32_t NT, uint32_t CH, bool NORM = true, bool DPP_SUMS = true, bool TAIL = false, int FIXED = -1>
struct XStage {
    static constexpr uint32_t TC = TAIL ? CH : 1;
    __device__ static __forceinline__ uint32_t md(const NormArg& na) {
        return FIXED >= 0 ? (uint32_t)FIXED : na.mode;
    }
    h8 xv[CH], av[CH], awv[CH], wv[CH];
    h8 t1[TC], t1w[TC], t2[TC], t2w[TC], tfw[TC];   // kStageTail: h1, its norm weight, h2, its, post-FFN norm
    float inv_in;      // kStageScaled: r(h), loaded with the chunks
    bool vec;

    __device__ __forceinline__ void load(const uint16_t* __restrict__ x, uint32_t n, const NormArg& na) {
        const uint32_t nch = n >> 3;
        const bool tail = TAIL && NORM && md(na) == kStageTail;
        uintptr_t align =
            (uintptr_t)x | (uintptr_t)na.w | (uintptr_t)na.attn | (uintptr_t)na.attn_w | (uintptr_t)na.export_h;
        if (tail)
            align |= (uintptr_t)na.h1 | (uintptr_t)na.h1_w | (uintptr_t)na.h2 | (uintptr_t)na.h2_w | (uintptr_t)na.ffn_w;
        vec = FIXED >= 0 || (((NORM ? align : (uintptr_t)x) & 15u) == 0 && (n & 7u) == 0 && nch != 0 &&
                             nch <= CH * NT);
        if (!vec) return;
        const bool post = NORM && (md(na) == kStagePostAttn || md(na) == kStageResidual || tail);
        const bool norm = NORM && (md(na) == kStageNorm || md(na) == kStagePostAttn || md(na) == kStageScaled || tail);
        if (tail) {
#pragma unroll
            for (uint32_t i = 0; i < TC; ++i) {
                const uint32_t c0 = threadIdx.x + i * NT;
                const uint32_t c = c0 < nch ? c0 : nch - 1;
                t1[i] = __builtin_bit_cast(h8, ld16h(na.h1, c));
                t1w[i] = __builtin_bit_cast(h8, ld16h(na.h1_w, c));
                t2[i] = __builtin_bit_cast(h8, ld16h(na.h2, c));
                t2w[i] = __builtin_bit_cast(h8, ld16h(na.h2_w, c));
                tfw[i] = __builtin_bit_cast(h8, ld16h(na.ffn_w, c));
            }
        }
        if (NORM && md(na) == kStageScaled) inv_in = *na.inv;
        // clamped chunk indices: every load is valid and unconditional (chunks
        // past the end are loaded twice and never stored or counted)
#pragma unroll
        for (uint32_t i = 0; i < CH; ++i) {
            const uint32_t c0 = threadIdx.x + i * NT;
            const uint32_t c = c0 < nch ? c0 : nch - 1;
            xv[i] = __builtin_bit_cast(h8, ld16h(x, c));
            if (post) {
                av[i] = __builtin_bit_cast(h8, ld16h(na.attn, c));
                awv[i] = __builtin_bit_cast(h8, ld16h(na.attn_w, c));
            }
            if (FIXED >= 0 && norm) wv[i] = __builtin_bit_cast(h8, ld16h(na.w ? na.w : x, c));
            else if (norm && na.w) wv[i] = __builtin_bit_cast(h8, ld16h(na.w, c));
        }
    }

    // Applies the NormArg transform to the loaded chunks (vector path).
    __device__ __forceinline__ void transform(uint32_t n, const NormArg& na) {
        if (!NORM) return;
        const uint32_t nch = n >> 3;
        const bool post = md(na) == kStagePostAttn || md(na) == kStageResidual;
        const bool norm = md(na) == kStageNorm || md(na) == kStagePostAttn || (TAIL && md(na) == kStageTail);
        if (md(na) == kStageBf16) {
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i) xv[i] = bf16x8_to_f16(__builtin_bit_cast(uint4, xv[i]));
            return;
        }
        if (TAIL && md(na) == kStageTail) {
            // the previous layer's tail, as layer_tail computes it (same
            // rounding points), then its output's RMSNorm; waves past the
            // vector skip the arithmetic (their chunks are never stored)
            const uint32_t wave_base = threadIdx.x & ~63u;
            float s3[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
                if (threadIdx.x + i * NT < nch)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        s3[0] = fmaf((float)av[i][e], (float)av[i][e], s3[0]);
                        s3[1] = fmaf((float)t1[i][e], (float)t1[i][e], s3[1]);
                        s3[2] = fmaf((float)t2[i][e], (float)t2[i][e], s3[2]);
                    }
            block_sums_once<3, NT, 0>(s3);
            const float inv_a = 1.0f / sqrtf(s3[0] / (float)n + na.eps);
            const float inv_1 = 1.0f / sqrtf(s3[1] / (float)n + na.eps);
            const float inv_2 = 1.0f / sqrtf(s3[2] / (float)n + na.eps);
            float s12[1] = {0.0f};
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
                if (wave_base + i * NT < nch)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const _Float16 an = (_Float16)((float)av[i][e] * (float)awv[i][e] * inv_a);
                        xv[i][e] = (_Float16)((float)xv[i][e] + (float)an);
                        const _Float16 a1 = (_Float16)((float)t1[i][e] * (float)t1w[i][e] * inv_1);
                        const _Float16 a2 = (_Float16)((float)t2[i][e] * (float)t2w[i][e] * inv_2);
                        t1[i][e] = (_Float16)((float)a1 + (float)a2);
                        if (threadIdx.x + i * NT < nch) s12[0] = fmaf((float)t1[i][e], (float)t1[i][e], s12[0]);
                    }
            block_sums_once<1, NT, 1>(s12);
            const float inv_12 = 1.0f / sqrtf(s12[0] / (float)n + na.eps);
            const float sc = (float)(_Float16)na.scalar;
            float ss[1] = {0.0f};
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
                if (wave_base + i * NT < nch)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const _Float16 f2 = (_Float16)((float)t1[i][e] * (float)tfw[i][e] * inv_12);
                        const _Float16 r = (_Float16)((float)xv[i][e] + (float)f2);
                        xv[i][e] = (_Float16)((float)r * sc);
                        if (threadIdx.x + i * NT < nch) ss[0] = fmaf((float)xv[i][e], (float)xv[i][e], ss[0]);
                    }
            if (na.export_h && blockIdx.x == 0)
#pragma unroll
                for (uint32_t i = 0; i < CH; ++i)
                    if (threadIdx.x + i * NT < nch) reinterpret_cast<h8*>(na.export_h)[threadIdx.x + i * NT] = xv[i];
            // the input RMSNorm of out
            block_sums_once<1, NT, 2>(ss);
            const float inv = 1.0f / sqrtf(ss[0] / (float)n + na.eps);
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
                if (wave_base + i * NT < nch)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float xw = na.w ? (float)xv[i][e] * (float)wv[i][e] : (float)xv[i][e];
                        xv[i][e] = (_Float16)(xw * inv);
                    }
            return;
        }
        if (md(na) == kStageScaled) {
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float xw = na.w ? (float)xv[i][e] * (float)wv[i][e] : (float)xv[i][e];
                    xv[i][e] = (_Float16)(xw * inv_in);
                }
            return;
        }
        if (post) {
            float ss = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
                if (threadIdx.x + i * NT < nch)
#pragma unroll
                    for (int e = 0; e < 8; ++e) ss = fmaf((float)av[i][e], (float)av[i][e], ss);
            const float inv = 1.0f / sqrtf(block_sum<NT>(ss) / (float)n + na.eps);
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const _Float16 an = (_Float16)((float)av[i][e] * (float)awv[i][e] * inv);
                    xv[i][e] = (_Float16)((float)xv[i][e] + (float)an);
                }
        }
        if (norm) {
            float ss = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
                if (threadIdx.x + i * NT < nch)
#pragma unroll
                    for (int e = 0; e < 8; ++e) ss = fmaf((float)xv[i][e], (float)xv[i][e], ss);
            const float inv = 1.0f / sqrtf(block_sum<NT>(ss) / (float)n + na.eps);
            if (post && na.export_h && blockIdx.x == 0) {
#pragma unroll
                for (uint32_t i = 0; i < CH; ++i)
                    if (threadIdx.x + i * NT < nch)
                        reinterpret_cast<h8*>(na.export_h)[threadIdx.x + i * NT] = xv[i];
                if (threadIdx.x == 0) *na.export_inv = inv;
            }
#pragma unroll
            for (uint32_t i = 0; i < CH; ++i)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float xw = na.w ? (float)xv[i][e] * (float)wv[i][e] : (float)xv[i][e];
                    xv[i][e] = (_Float16)(xw * inv);
                }
        }
    }

    // LDS layout: xpairs_lds_bytes(n) at lds (plain copy, planes, sums).
    __device__ __forceinline__ XPairs pairs(const uint16_t* __restrict__ x, uint16_t* __restrict__ lds,
                                            uint32_t n, const NormArg& na, bool plain = false) {
        if (!vec) {
            stage_act_scalar<NT>(x, lds, n, NORM ? na : NormArg{nullptr, nullptr, nullptr, 0.0f, kStageCopy});
            return build_xpairs<NT>(lds, n);
        }
        transform(n, na);
        const uint32_t npc = n >> 3, nch = n >> 5;
        uint4* planes = reinterpret_cast<uint4*>(lds + n);
        float4* sums = reinterpret_cast<float4*>(planes + 4 * nch);
#pragma unroll
        for (uint32_t i = 0; i < CH; ++i) {
            const uint32_t q = threadIdx.x + i * NT;     // npc is a multiple of 8: all four pieces of a chunk agree
            const h8 v = q < npc ? xv[i] : h8{};
            float s, sa, sb;
            h8_sums(v, s, sa, sb);
            const float4 cs = chunk_sums<DPP_SUMS>(s, sa, sb);
            if (q < npc) {
                planes[(q & 3u) * nch + (q >> 2)] = h8_pairs(v);
                if ((q & 3u) == 0) sums[q >> 2] = cs;
                if (plain) reinterpret_cast<h8*>(lds)[q] = v;
            }
        }
        __syncthreads();
        return {planes, sums, nch};
    }

    __device__ __forceinline__ void plain(const uint16_t* __restrict__ x, uint16_t* __restrict__ lds, uint32_t n,
                                          const NormArg& na) {
        if (!vec) {
            stage_act_scalar<NT>(x, lds, n, NORM ? na : NormArg{nullptr, nullptr, nullptr, 0.0f, kStageCopy});
            return;
        }
        transform(n, na);
        const uint32_t nch = n >> 3;
#pragma unroll
        for (uint32_t i = 0; i < CH; ++i) {
            const uint32_t q = threadIdx.x + i * NT;
            if (TAIL) {
                if (q < nch) reinterpret_cast<h8*>(lds)[q] = xv[i];
            } else {
                // a chunk past the end holds the last chunk (clamped load, the
                // same transform) and is stored there again: the store stays
                // unconditional, so the compiler cannot sink the chunk's load
                // under a branch, whose join would wait for every load issued
                // before it (the weight stream included)
                reinterpret_cast<h8*>(lds)[q < nch ? q : nch - 1] = xv[i];
            }
        }
        __syncthreads();
    }
};

constexpr uint32_t kStageChunks = 2;     // 16-byte chunks per thread of the GEMV-family staging (n <= 4096)

// One-call staging of the fp16 vector (no pairs): lds[0..n).
template <uint32_t NT = kThreads>
__device__ __forceinline__ void stage_act(const uint16_t* __restrict__ x, uint16_t* __restrict__ lds,
                                          uint32_t n, const NormArg& na) {
    XStage<NT, kStageChunks> st;
    st.load(x, n, na);
    st.plain(x, lds, n, na);
}

// Plain staging (no normalisation).
template <uint32_t NT = kThreads>
__device__ __forceinline__ void stage_xh(const uint16_t* __restrict__ x, uint16_t* __restrict__ lds,
                                         uint32_t n) {
    copy_to_lds<NT>(x, lds, n);
    __syncthreads();
}

}  // namespace tfq
