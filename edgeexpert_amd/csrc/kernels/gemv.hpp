// gemv.hpp — decode-side GEMVs: int4 g64 (plain and fused QKV), int8 g64,
// the int8 router logits + top-k selection, and the BF16 -> fp16 converter.
//
// Mapping (all GEMVs): one 16-byte chunk of a weight row per lane, so every
// weight byte arrives through a 128-bit load and a segment's lanes read one
// contiguous run of the row. A row of n codes has n/32 (int4) or n/16 (int8)
// chunks; a segment of SEG lanes walks them with stride SEG (P chunks per
// lane). Lane <-> chunk is fixed for the whole kernel, so each lane keeps the
// activations of its P chunks in registers (staged once through LDS) together
// with the per-chunk activation sum needed by the affine factoring
//     Σ_k (q_k·s + b)·x_k = s·Σ q_k x_k + b·Σ x_k        (per group of 64)
// (S/Metal/Quant/dequant_int4.metal:14-17).
//
// Latency: the kernels are HBM-latency bound at decode sizes, so every
// segment issues the weight/scale/bias loads of its first R rows *before*
// staging x, and each later group of R rows is requested while the previous
// group's partial sums are being reduced and stored.
#pragma once

#include "abi_types.h"
#include "common.hpp"

namespace tfq {

// Row r of a multi-matrix launch -> (weights row, scales row, biases row, y slot).
struct Q4Row {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint16_t* y;
};

__device__ __forceinline__ Q4Row resolve_row(const Q4Multi& mats, uint32_t row, uint32_t row_bytes,
                                             uint32_t ngroups) {
    uint32_t r = row;
    const uint8_t* w = mats.m[0].w;
    const uint16_t* s = mats.m[0].s;
    const uint16_t* b = mats.m[0].b;
    uint16_t* y = mats.m[0].y;
    if (mats.nmat > 1 && r >= mats.m[0].rows) {
        r -= mats.m[0].rows;
        w = mats.m[1].w; s = mats.m[1].s; b = mats.m[1].b; y = mats.m[1].y;
        if (mats.nmat > 2 && r >= mats.m[1].rows) {
            r -= mats.m[1].rows;
            w = mats.m[2].w; s = mats.m[2].s; b = mats.m[2].b; y = mats.m[2].y;
        }
    }
    return {w + (size_t)r * row_bytes, s + (size_t)r * ngroups, b + (size_t)r * ngroups, y + r};
}

// int4 GEMV over 1..3 matrices with a shared x. Dynamic LDS: n halves.
template <int SEG, int P, int R>
__device__ __forceinline__ void q4_gemv_multi(const Q4Multi& mats, const uint16_t* __restrict__ x,
                                              uint32_t n) {
    extern __shared__ uint16_t lds_xh[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = n >> 5;              // 16-byte chunks per row
    const uint32_t row_bytes = n >> 1;
    const uint32_t ngroups = n >> 6;
    constexpr uint32_t spw = kWave / SEG;     // segments per wave
    const uint32_t seg_id = (blockIdx.x * nwaves + wave) * spw + lane / SEG;
    const uint32_t seg_total = gridDim.x * nwaves * spw;
    const uint32_t total = mats.total_rows;

    uint4 wv[R][P];
    float sv[R][P], bv[R][P];
    auto issue = [&](uint32_t grp) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = seg_id + (grp * R + r) * seg_total;
            if (row < total) {
                const Q4Row q = resolve_row(mats, row, row_bytes, ngroups);
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c = sl + p * SEG;
                    if (c < lpr) {
                        wv[r][p] = ldg16(q.w + 16u * c);
                        sv[r][p] = h2f(q.s[c >> 1]);
                        bv[r][p] = h2f(q.b[c >> 1]);
                    }
                }
            }
        }
    };
    issue(0);
    stage_xh(x, lds_xh, n);
    XChunk xc[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_xchunk(lds_xh, c, xc[p]);
    }

    for (uint32_t grp = 0; seg_id + grp * R * seg_total < total; ++grp) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c = sl + p * SEG;
                if (c < lpr) {
                    const float d = dot_q4_chunk(wv[r][p], xc[p]);
                    acc[r] = fmaf(sv[r][p], d, acc[r]);
                    acc[r] = fmaf(bv[r][p], xc[p].sum, acc[r]);
                }
            }
        }
        issue(grp + 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = seg_sum<SEG>(acc[r]);
            const uint32_t row = seg_id + (grp * R + r) * seg_total;
            if (sl == 0 && row < total) *resolve_row(mats, row, row_bytes, ngroups).y = f2h(v);
        }
    }
}

// ---------------------------------------------------------------- int8 ----
//
// The int8 paths (router logits, DequantInt8GEMV) keep fp32 activations:
// the router multiplies h by the effective scale in fp32 before the dot,
// and its top-k ordering must not see an extra fp16 rounding.

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

// Rows of an int8 GEMV. `stage()` must fill lds_x (fp32, n values) and
// synchronise; it runs after the first row group's loads are in flight.
// Emits fp32 results through `out(row, value)` from lane 0 of each segment.
template <int SEG, int P, int R, typename Stage, typename Out>
__device__ __forceinline__ void q8_rows(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                        const uint16_t* __restrict__ B, float* __restrict__ lds_x,
                                        uint32_t M, uint32_t n, Stage stage, Out out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = n >> 4;
    const uint32_t ngroups = n >> 6;
    constexpr uint32_t spw = kWave / SEG;
    const uint32_t seg_id = (blockIdx.x * nwaves + wave) * spw + lane / SEG;
    const uint32_t seg_total = gridDim.x * nwaves * spw;

    uint4 wv[R][P];
    float sv[R][P], bv[R][P];
    auto issue = [&](uint32_t grp) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = seg_id + (grp * R + r) * seg_total;
            if (row < M) {
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const uint32_t c = sl + p * SEG;
                    if (c < lpr) {
                        wv[r][p] = ldg16(W + (size_t)row * n + 16u * c);
                        sv[r][p] = h2f(S[(size_t)row * ngroups + (c >> 2)]);
                        bv[r][p] = h2f(B[(size_t)row * ngroups + (c >> 2)]);
                    }
                }
            }
        }
    };
    issue(0);
    stage();
    float xr[P][16];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_x16(lds_x, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }
    for (uint32_t grp = 0; seg_id + grp * R * seg_total < M; ++grp) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            acc[r] = 0.0f;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c = sl + p * SEG;
                if (c < lpr) {
                    const float d = dot16_q8(wv[r][p], xr[p]);
                    acc[r] = fmaf(sv[r][p], d, acc[r]);
                    acc[r] = fmaf(bv[r][p], xs[p], acc[r]);
                }
            }
        }
        issue(grp + 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float v = seg_sum<SEG>(acc[r]);
            const uint32_t row = seg_id + (grp * R + r) * seg_total;
            if (sl == 0 && row < M) out(row, v);
        }
    }
}

template <int SEG, int P, int R>
__device__ __forceinline__ void q8_gemv(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                        const uint16_t* __restrict__ B, const uint16_t* __restrict__ x,
                                        uint16_t* __restrict__ y, uint32_t M, uint32_t n) {
    extern __shared__ float lds_x[];
    q8_rows<SEG, P, R>(
        W, S, B, lds_x, M, n,
        [&]() {
            for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) lds_x[i] = h2f(x[i]);
            __syncthreads();
        },
        [&](uint32_t row, float v) { y[row] = f2h(v); });
}

// -------------------------------------------------------------- router ----

constexpr uint32_t kRouterMaxExperts = 256;
constexpr uint32_t kRouterMaxTopK = 64;

// logits[e] = Σ_g s·Σ q·(h⊙eff) + b·Σ(h⊙eff), fp32 (S/Metal/MoE/moe.metal:78-116).
// Dynamic LDS: d floats.
template <int SEG, int P>
__device__ __forceinline__ void router_logits(const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                              const uint16_t* __restrict__ B, const uint16_t* __restrict__ h,
                                              const uint16_t* __restrict__ eff,
                                              float* __restrict__ logits, uint32_t E, uint32_t d) {
    extern __shared__ float lds_x[];
    q8_rows<SEG, P, 1>(
        W, S, B, lds_x, E, d,
        [&]() {
            for (uint32_t i = threadIdx.x; i < d; i += blockDim.x) {
                const float hv = h2f(h[i]);
                lds_x[i] = eff ? hv * h2f(eff[i]) : hv;
            }
            __syncthreads();
        },
        [&](uint32_t row, float v) { logits[row] = v; });
}

// Top-k of E logits by (value desc, index asc) in one wavefront.
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

// One wavefront (block of 64): top-k, softmax over the k, × per-expert gain
// (S/Metal/MoE/moe.metal:135-185; ties to the lower index as at :157).
__device__ __forceinline__ void router_select(const float* __restrict__ logits,
                                              const uint16_t* __restrict__ gain,
                                              uint32_t* __restrict__ out_idx, uint16_t* __restrict__ out_w,
                                              float* __restrict__ out_wf, uint32_t E, uint32_t k) {
    __shared__ float stage[kRouterMaxExperts];
    __shared__ uint32_t sel_idx[kRouterMaxTopK];
    __shared__ float sel_val[kRouterMaxTopK];
    for (uint32_t e = threadIdx.x; e < E; e += blockDim.x) stage[e] = logits[e];
    __syncthreads();
    wave_topk(stage, E, k, sel_idx, sel_val);
    __syncthreads();
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
