// common.hpp — shared device helpers for the gfx950 quantized-matmul kernels.
//
// Wave64 throughout: a "segment" is a power-of-two group of SEG lanes inside
// one wavefront that cooperates on one output row; several segments share a
// wave when a row needs fewer than 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tfq {

constexpr int kGroup = 64;       // affine group size along the reduction axis
constexpr int kWave = 64;        // CDNA wavefront width

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

// Sum over the SEG lanes of a segment; every lane of the segment receives the
// total. The xor butterfly stays inside the segment, so segments of one wave
// may hold different rows, and the order of additions is fixed (deterministic).
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
#pragma unroll
    for (int m = SEG / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// gelu_pytorch_tanh with the inner argument clamped to ±20
// (S/Metal/MoE/moe.metal:53-60; the clamp is exact at fp32 saturation).
__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = 0.7978845608028654f;
    const float k3 = 0.044715f;
    float inner = c * (x + k3 * x * x * x);
    inner = fminf(fmaxf(inner, -20.0f), 20.0f);
    return 0.5f * x * (1.0f + tanhf(inner));
}

// Σ_i q_i * x_i over the 32 int4 codes of one 16-byte chunk (8 codes per
// 32-bit word, element 8j+i in bits 4i..4i+3 of word j), fp32 FMA chain in
// element order.
__device__ __forceinline__ float dot32_q4(const uint4 w, const float* x) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = ws[i] & 0x0F0F0F0Fu;
        const uint32_t hi = (ws[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            d = fmaf((float)((lo >> (8 * b)) & 0xFFu), x[8 * i + 2 * b], d);
            d = fmaf((float)((hi >> (8 * b)) & 0xFFu), x[8 * i + 2 * b + 1], d);
        }
    }
    return d;
}

// Σ_i q_i * x_i over the 16 int8 codes of one 16-byte chunk.
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

__device__ __forceinline__ uint4 ldg16(const uint8_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

}  // namespace tfq
