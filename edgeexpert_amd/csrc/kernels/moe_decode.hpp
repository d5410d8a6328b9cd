// moe_decode.hpp — routed top-k MoE decode block and the int4 shared expert.
//
// The routed experts of a layer live in one HBM pool: expert e's blob is
// pool + e*stride, holding [gateW gateS gateB upW upS upB downW downS downB]
// at fixed offsets (S/Kernels/MoE/MoE.swift:4-29). The kernels read the
// router's index buffer and form the blob address on the device; there is no
// host round trip between routing and the expert GEMVs.
//
// Phase 1 (S/Metal/MoE/moe.metal:248-369): one segment per (slot, f) row,
//   gate and up rows share the x registers; acts[slot][f] = gelu(g)·u in fp32.
// Phase 2 (moe.metal:189-244,475-511): one wavefront per output d; its eight
//   8-lane segments each own one slot's down row d, so the eight expert dot
//   products finish inside one wave and lane 0 adds
//   residual + Σ_slot w[slot]·dot[slot] in fixed slot order.
#pragma once

#include "gemv.hpp"

namespace tfq {

// Two int4 rows (gate f, up f) of one expert against the same x registers.
template <int SEG, int P>
__device__ __forceinline__ float2 gate_up_row(const uint8_t* __restrict__ gw, const uint16_t* __restrict__ gs,
                                              const uint16_t* __restrict__ gb, const uint8_t* __restrict__ uw,
                                              const uint16_t* __restrict__ us, const uint16_t* __restrict__ ub,
                                              uint32_t sl, uint32_t lpr, const float (&xr)[P][32],
                                              const float (&xs)[P]) {
    uint4 gv[P], uv[P];
    float gsv[P], gbv[P], usv[P], ubv[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) {
            gv[p] = ldg16(gw + 16u * c);
            uv[p] = ldg16(uw + 16u * c);
            gsv[p] = h2f(gs[c >> 1]);
            gbv[p] = h2f(gb[c >> 1]);
            usv[p] = h2f(us[c >> 1]);
            ubv[p] = h2f(ub[c >> 1]);
        }
    }
    float ga = 0.0f, ua = 0.0f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) {
            const float gd = dot32_q4(gv[p], xr[p]);
            const float ud = dot32_q4(uv[p], xr[p]);
            ga = fmaf(gsv[p], gd, ga);
            ga = fmaf(gbv[p], xs[p], ga);
            ua = fmaf(usv[p], ud, ua);
            ua = fmaf(ubv[p], xs[p], ua);
        }
    }
    return make_float2(seg_sum<SEG>(ga), seg_sum<SEG>(ua));
}

// Phase 1 over n_active slots (active_slots == nullptr: slots 0..n_active-1).
template <int SEG, int P>
__device__ __forceinline__ void moe_phase1(const ExpertPool& pool, const uint32_t* __restrict__ indices,
                                           const uint32_t* __restrict__ active_slots, uint32_t n_active,
                                           uint32_t top_k, const uint16_t* __restrict__ x,
                                           float* __restrict__ acts, uint32_t D, uint32_t F) {
    extern __shared__ float lds_x[];
    stage_f16_as_f32(x, lds_x, D);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = D >> 5;
    const uint32_t row_bytes = D >> 1;
    const uint32_t ngroups = D >> 6;
    float xr[P][32];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_x32(lds_x, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }
    constexpr uint32_t spw = kWave / SEG;
    const uint32_t total = n_active * F;
    const uint32_t rstride = gridDim.x * nwaves * spw;
    for (uint32_t row = (blockIdx.x * nwaves + wave) * spw + lane / SEG; row < total;
         row += rstride) {
        const uint32_t a = row / F;
        const uint32_t f = row - a * F;
        const uint32_t slot = active_slots ? active_slots[a] : a;
        if (slot >= top_k) continue;                    // moe.metal:387 semantics
        const uint32_t e = indices[slot];
        float act;
        if (e < pool.num_experts) {
            const uint8_t* blob = pool.base + (uint64_t)e * pool.stride;
            const ExpertOffsets& o = pool.off;
            const float2 gu = gate_up_row<SEG, P>(
                blob + o.gate_w + (size_t)f * row_bytes,
                reinterpret_cast<const uint16_t*>(blob + o.gate_s) + (size_t)f * ngroups,
                reinterpret_cast<const uint16_t*>(blob + o.gate_b) + (size_t)f * ngroups,
                blob + o.up_w + (size_t)f * row_bytes,
                reinterpret_cast<const uint16_t*>(blob + o.up_s) + (size_t)f * ngroups,
                reinterpret_cast<const uint16_t*>(blob + o.up_b) + (size_t)f * ngroups, sl, lpr, xr,
                xs);
            act = gelu_tanh(gu.x) * gu.y;
        } else {
            act = __builtin_nanf("");                   // invalid expert index: poison loudly
        }
        if (sl == 0) acts[(size_t)slot * F + f] = act;
    }
}

// Phase 2: P chunks of 32 per lane over F (F <= 256*P). Dynamic LDS: top_k*F floats.
template <int P>
__device__ __forceinline__ void moe_phase2(const ExpertPool& pool, const uint32_t* __restrict__ indices,
                                           const float* __restrict__ acts,
                                           const uint16_t* __restrict__ rw,
                                           const uint16_t* __restrict__ residual,
                                           uint16_t* __restrict__ y, uint32_t D, uint32_t F,
                                           uint32_t top_k) {
    constexpr int SEG = 8;
    extern __shared__ float lds_a[];
    for (uint32_t i = threadIdx.x; i < top_k * F; i += blockDim.x) lds_a[i] = acts[i];
    __syncthreads();

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t slot = lane >> 3;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = F >> 5;
    const uint32_t row_bytes = F >> 1;
    const uint32_t ngroups = F >> 6;
    const bool live = slot < top_k;
    const uint32_t e = live ? indices[slot] : 0u;
    const bool valid = live && e < pool.num_experts;

    float xr[P][32];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (live && c < lpr) load_x32(lds_a + (size_t)slot * F, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }
    const uint8_t* blob = pool.base + (uint64_t)(valid ? e : 0u) * pool.stride;
    const uint8_t* dw = blob + pool.off.down_w;
    const uint16_t* ds = reinterpret_cast<const uint16_t*>(blob + pool.off.down_s);
    const uint16_t* db = reinterpret_cast<const uint16_t*>(blob + pool.off.down_b);
    const float w_slot = live ? h2f(rw[slot]) : 0.0f;

    for (uint32_t d = blockIdx.x * nwaves + wave; d < D; d += gridDim.x * nwaves) {
        float acc = 0.0f;
        if (valid) {
            uint4 wv[P];
            float sv[P], bv[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c = sl + p * SEG;
                if (c < lpr) {
                    wv[p] = ldg16(dw + (size_t)d * row_bytes + 16u * c);
                    sv[p] = h2f(ds[(size_t)d * ngroups + (c >> 1)]);
                    bv[p] = h2f(db[(size_t)d * ngroups + (c >> 1)]);
                }
            }
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint32_t c = sl + p * SEG;
                if (c < lpr) {
                    const float dd = dot32_q4(wv[p], xr[p]);
                    acc = fmaf(sv[p], dd, acc);
                    acc = fmaf(bv[p], xs[p], acc);
                }
            }
        } else if (live) {
            acc = __builtin_nanf("");
        }
        acc = seg_sum<SEG>(acc);
        const float part = w_slot * acc;              // partial[slot] = w·value (moe.metal:499)
        float out = residual ? h2f(residual[d]) : 0.0f;
#pragma unroll
        for (uint32_t s = 0; s < 8; ++s) {
            const float ps = __shfl(part, (int)(s * SEG), kWave);
            if (s < top_k) out += ps;                 // fixed slot order (moe.metal:505-509)
        }
        if (lane == 0) y[d] = f2h(out);
    }
}

// Shared-expert gate/up/act: act[i] = fp16(gelu(gate[i]·x) · (up[i]·x)).
template <int SEG, int P>
__device__ __forceinline__ void q4_gate_up_act(const uint8_t* __restrict__ gw, const uint16_t* __restrict__ gs,
                                               const uint16_t* __restrict__ gb, const uint8_t* __restrict__ uw,
                                               const uint16_t* __restrict__ us, const uint16_t* __restrict__ ub,
                                               const uint16_t* __restrict__ x, uint16_t* __restrict__ act,
                                               uint32_t D, uint32_t F) {
    extern __shared__ float lds_x[];
    stage_f16_as_f32(x, lds_x, D);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t sl = lane & (SEG - 1);
    const uint32_t lpr = D >> 5;
    const uint32_t row_bytes = D >> 1;
    const uint32_t ngroups = D >> 6;
    float xr[P][32];
    float xs[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t c = sl + p * SEG;
        if (c < lpr) load_x32(lds_x, c, xr[p], xs[p]);
        else xs[p] = 0.0f;
    }
    constexpr uint32_t spw = kWave / SEG;
    const uint32_t rstride = gridDim.x * nwaves * spw;
    for (uint32_t f = (blockIdx.x * nwaves + wave) * spw + lane / SEG; f < F; f += rstride) {
        const float2 gu = gate_up_row<SEG, P>(gw + (size_t)f * row_bytes, gs + (size_t)f * ngroups,
                                              gb + (size_t)f * ngroups, uw + (size_t)f * row_bytes,
                                              us + (size_t)f * ngroups, ub + (size_t)f * ngroups, sl,
                                              lpr, xr, xs);
        if (sl == 0) act[f] = f2h(gelu_tanh(gu.x) * gu.y);
    }
}

}  // namespace tfq
