// gemv.hpp — decode-side GEMVs: int4 g64 (plain and fused QKV), int8 g64,
// the int8 router with its in-kernel top-k, and the BF16 -> fp16 converter.
//
// Mapping (all GEMVs): one 16-byte chunk of a weight row per lane, so every
// weight byte arrives through a 128-bit load and a segment's lanes read one
// contiguous run of the row. A row of n codes has n/32 (int4) or n/16 (int8)
// chunks; a segment of SEG lanes walks them with stride SEG (P chunks per
// lane). Lane ↔ chunk is fixed for the whole kernel, so each lane keeps the
// fp32 activations of its P chunks in registers (staged once through LDS) and
// the per-chunk activation sum needed by the affine factoring
//     Σ_k (q_k·s + b)·x_k = s·Σ q_k x_k + b·Σ x_k        (per group of 64)
// (S/Metal/Quant/dequant_int4.metal:14-17). Rows are then streamed with only
// weight, scale and bias loads; a segment butterfly reduces the partials.
#pragma once

#include "abi_types.h"
#include "common.hpp"

namespace tfq {

__device__ __forceinline__ void stage_f16_as_f32(const uint16_t* __restrict__ x,
                                                 float* __restrict__ lds, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) lds[i] = h2f(x[i]);
    __syncthreads();
}

// Load the 32 fp32 activations of chunk c (int4 layout) and their sum.
__device__ __forceinline__ void load_x32(const float* __restrict__ lds, uint32_t c, float* xr,
                                         float& xs) {
    const float4* src = reinterpret_cast<const float4*>(lds + 32u * c);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 v = src[i];
        xr[4 * i + 0] = v.x;
        xr[4 * i + 1] = v.y;
        xr[4 * i + 2] = v.z;
        xr[4 * i + 3] = v.w;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) s += xr[i];
    xs = s;
}

// int4 GEMV over 1..3 matrices with a shared x. Dynamic LDS: n floats.
template <int SEG, int P>
__device__ __forceinline__ void q4_gemv_multi(const Q4Multi& mats, const uint16_t* __restrict__ x,
                                              uint32_t n) {
    extern __shared__ float lds_x[];
    stage_f16_as_f32(x, lds_x, n);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = n >> 5;              // 16-byte chunks per row
    const uint32_t row_bytes = n >> 1;
    const uint32_t ngroups = n >> 6;

    float xr[P][32];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_x32(lds_x, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }

    constexpr uint32_t spw = kWave / SEG;     // segments (rows in flight) per wave
    const uint32_t rstride = gridDim.x * nwaves * spw;
    for (uint32_t row = (blockIdx.x * nwaves + wave) * spw + lane / SEG; row < mats.total_rows;
         row += rstride) {
        uint32_t r = row;
        int mi = 0;
        if (mats.nmat > 1 && r >= mats.m[0].rows) { r -= mats.m[0].rows; mi = 1; }
        if (mats.nmat > 2 && mi == 1 && r >= mats.m[1].rows) { r -= mats.m[1].rows; mi = 2; }
        const Q4Mat& m = mats.m[mi];
        const uint8_t* wrow = m.w + (size_t)r * row_bytes;
        const uint16_t* srow = m.s + (size_t)r * ngroups;
        const uint16_t* brow = m.b + (size_t)r * ngroups;
        uint4 wv[P];
        float sv[P], bv[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t c = sl + p * SEG;
            if (c < lpr) {
                wv[p] = ldg16(wrow + 16u * c);
                sv[p] = h2f(srow[c >> 1]);
                bv[p] = h2f(brow[c >> 1]);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t c = sl + p * SEG;
            if (c < lpr) {
                const float d = dot32_q4(wv[p], xr[p]);
                acc = fmaf(sv[p], d, acc);
                acc = fmaf(bv[p], xs[p], acc);
            }
        }
        acc = seg_sum<SEG>(acc);
        if (sl == 0) m.y[r] = f2h(acc);
    }
}

// ---------------------------------------------------------------- int8 ----

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

// Rows [row0 .. M) of an int8 GEMV whose x already sits in LDS as fp32;
// emits fp32 results through `out(row, value)` from lane 0 of each segment.
template <int SEG, int P, typename Out>
__device__ __forceinline__ void q8_rows(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                        const uint16_t* __restrict__ B, const float* __restrict__ lds_x,
                                        uint32_t M, uint32_t n, Out out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = n >> 4;
    const uint32_t ngroups = n >> 6;
    float xr[P][16];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_x16(lds_x, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }
    constexpr uint32_t spw = kWave / SEG;
    const uint32_t rstride = gridDim.x * nwaves * spw;
    for (uint32_t row = (blockIdx.x * nwaves + wave) * spw + lane / SEG; row < M; row += rstride) {
        const uint8_t* wrow = W + (size_t)row * n;
        uint4 wv[P];
        float sv[P], bv[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t c = sl + p * SEG;
            if (c < lpr) {
                wv[p] = ldg16(wrow + 16u * c);
                sv[p] = h2f(S[(size_t)row * ngroups + (c >> 2)]);
                bv[p] = h2f(B[(size_t)row * ngroups + (c >> 2)]);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t c = sl + p * SEG;
            if (c < lpr) {
                const float d = dot16_q8(wv[p], xr[p]);
                acc = fmaf(sv[p], d, acc);
                acc = fmaf(bv[p], xs[p], acc);
            }
        }
        acc = seg_sum<SEG>(acc);
        if (sl == 0) out(row, acc);
    }
}

template <int SEG, int P>
__device__ __forceinline__ void q8_gemv(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                        const uint16_t* __restrict__ B, const uint16_t* __restrict__ x,
                                        uint16_t* __restrict__ y, uint32_t M, uint32_t n) {
    extern __shared__ float lds_x[];
    stage_f16_as_f32(x, lds_x, n);
    q8_rows<SEG, P>(W, S, B, lds_x, M, n, [&](uint32_t row, float v) { y[row] = f2h(v); });
}

// -------------------------------------------------------------- router ----

// Workspace layout (bytes): [0, 4) arrival counter; [1024, 2048) logits fp32.
constexpr uint32_t kRouterCounterOffset = 0;
constexpr uint32_t kRouterLogitsOffset = 1024;
constexpr uint32_t kRouterMaxExperts = 256;
constexpr uint32_t kRouterMaxTopK = 64;

// Top-k of `E` logits by (value desc, index asc), run by one wavefront.
// Writes the selected indices / values into LDS arrays (lane 0).
__device__ __forceinline__ void wave_topk(const float* logits, uint32_t E, uint32_t k,
                                          uint32_t* sel_idx, float* sel_val) {
    const uint32_t lane = threadIdx.x & 63u;
    constexpr uint32_t NONE = 0xFFFFFFFFu;
    float v[4];
    uint32_t id[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t e = lane + 64u * j;
        v[j] = e < E ? logits[e] : -INFINITY;
        id[j] = e < E ? e : NONE;
    }
    for (uint32_t r = 0; r < k; ++r) {
        float bv = -INFINITY;
        uint32_t bi = NONE;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (id[j] != NONE && (bi == NONE || v[j] > bv || (v[j] == bv && id[j] < bi))) {
                bv = v[j];
                bi = id[j];
            }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, kWave);
            const uint32_t oi = (uint32_t)__shfl_xor((int)bi, m, kWave);
            if (oi != NONE && (bi == NONE || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (id[j] == bi) id[j] = NONE;
        if (lane == 0) {
            sel_idx[r] = bi;
            sel_val[r] = bv;
        }
    }
}

// Router GEMV (h ⊙ eff through the int8 rows, fp32 logits) then, in the last
// block to finish, top-k + softmax over the k + per-expert gain
// (S/Metal/MoE/moe.metal:78-185). Dynamic LDS: d floats.
template <int SEG, int P>
__device__ __forceinline__ void router_topk(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                            const uint16_t* __restrict__ B, const uint16_t* __restrict__ h,
                                            const uint16_t* __restrict__ eff,
                                            const uint16_t* __restrict__ gain,
                                            uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w,
                                            float* __restrict__ out_wf, float* __restrict__ out_logits,
                                            uint32_t E, uint32_t d, uint32_t k, uint8_t* __restrict__ ws) {
    extern __shared__ float lds_x[];
    for (uint32_t i = threadIdx.x; i < d; i += blockDim.x) {
        const float hv = h2f(h[i]);
        lds_x[i] = eff ? hv * h2f(eff[i]) : hv;
    }
    __syncthreads();

    float* logits = reinterpret_cast<float*>(ws + kRouterLogitsOffset);
    uint32_t* counter = reinterpret_cast<uint32_t*>(ws + kRouterCounterOffset);
    q8_rows<SEG, P>(W, S, B, lds_x, E, d, [&](uint32_t row, float v) {
        logits[row] = v;
        if (out_logits) out_logits[row] = v;
    });

    // Last-arriving block selects (no spin: every block exits on its own).
    __shared__ uint32_t is_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        is_last = (prev == gridDim.x - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();

    __shared__ uint32_t sel_idx[kRouterMaxTopK];
    __shared__ float sel_val[kRouterMaxTopK];
    if (threadIdx.x < 64) {
        // logits written by other blocks: read through the coherent path
        float lv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = threadIdx.x + 64u * j;
            lv[j] = e < E ? __hip_atomic_load(&logits[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : 0.0f;
        }
        float* stage = lds_x;   // reuse LDS for the gathered logits
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t e = threadIdx.x + 64u * j;
            if (e < E) stage[e] = lv[j];
        }
        wave_topk(stage, E, k, sel_idx, sel_val);
        if (threadIdx.x == 0) {
            const float vmax = sel_val[0];
            float sum = 0.0f;
            for (uint32_t r = 0; r < k; ++r) sum += expf(sel_val[r] - vmax);
            for (uint32_t r = 0; r < k; ++r) {
                const uint32_t e = sel_idx[r];
                const float wgt = expf(sel_val[r] - vmax) / sum * (gain ? h2f(gain[e]) : 1.0f);
                out_idx[r] = e;
                out_w[r] = f2h(wgt);
                if (out_wf) out_wf[r] = wgt;
            }
            __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------- convert ----

__device__ __forceinline__ void convert_bf16_to_f16(const uint16_t* __restrict__ src,
                                                    uint16_t* __restrict__ dst, uint64_t n,
                                                    uint32_t* __restrict__ inexact) {
    uint32_t bad = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float v = bf2f(src[i]);
        const uint16_t hbits = f2h(v);
        dst[i] = hbits;
        const float back = h2f(hbits);
        if (!(back == v) && !(v != v)) ++bad;   // NaN passes through as NaN
    }
    if (inexact && bad) atomicAdd(inexact, bad);
}

}  // namespace tfq
