// attention.hpp — single-token GQA decode attention over an fp16 KV cache
// (split-K over the keys), the Gemma 4 q/k/v epilogue fused into it, and the
// decode layer's tail.
//
// Cache layout [capacity][num_kv_heads][HD] fp16 for K and for V (the
// reference's, S/Metal/Attention/attention.metal:316-580). Keys
// [kv_start, seq_len) are cut into kAttnChunk-key chunks; block (chunk, kv head)
// computes, for each of the G query heads sharing that kv head,
//     m = max_j s_j,  l = Σ_j e^{s_j - m},  O[d] = Σ_j e^{s_j - m} V[j][d],
// s_j = scale · q·k_j (fp32 accumulate of exact fp16 products), and stores
// (m, l, O) in fp32. A second kernel merges the chunks of each query head:
//     out[d] = fp16(Σ_c e^{m_c - M} O_c[d] / Σ_c e^{m_c - M} l_c),  M = max_c m_c,
// which is the exact softmax of AttentionRef.apply
// (V/Reference/Attention/Attention.swift:14-104) regrouped by chunk.
//
// Mapping inside a block (256 threads): for q·k, 16 lanes own one key (each
// lane HD/128 16-byte pieces of the row, so one load instruction covers
// 2048/HD whole rows); for p·V, HD/8 threads own one key row with 16-byte
// loads and 2048/HD groups of them split the chunk's keys, reduced through
// LDS in group order. The chunk's K loads are issued first, its V loads after
// the q/k/v epilogue. A block serves GB of the G query heads of its kv head
// (GB = G up to head_dim 256; at head_dim 512, the full-attention layers'
// 16 q / 2 kv heads, two blocks of 4 heads each per (chunk, kv head), which
// keeps the query registers to 64 per lane and gives 256 blocks at 4096 keys).
#pragma once

#include "common.hpp"

namespace tfq {

constexpr uint32_t kAttnThreads = 256;
constexpr uint32_t kLayerTailThreads = 1024;     // threads of the one-block layer tail
constexpr uint32_t kAttnKeyLanes = 16;          // one DPP row per key (row16_sum)
static_assert(kAttnChunk == kWave, "chunk softmax: one key per lane of a wavefront");

// NeoX rotation of pair i at `pos`: angle = pos · theta^(-2i/HD)
// (fused.metal:58-72; V/Reference/Attention/RoPE.swift:70-110). The inverse
// frequency 2^(-(2i/HD)·log2 theta) and the angle are formed in fp64 and the
// angle is reduced to a fraction of a turn there, so no fp32 error grows with
// the position; sine and cosine of the reduced angle are taken in fp32
// (sincospi of 2·turns, ~1e-7 absolute).
__device__ __forceinline__ void rope_table(float* __restrict__ c, float* __restrict__ s, uint32_t pairs,
                                           uint32_t hd, uint32_t pos, double log2_theta) {
    constexpr double kInvTwoPi = 0.15915494309189533577;
    for (uint32_t i = threadIdx.x; i < pairs; i += kAttnThreads) {
        const double inv_freq = exp2(-(2.0 * (double)i / (double)hd) * log2_theta);
        const double turns = (double)pos * inv_freq * kInvTwoPi;
        float sv, cv;
        sincospif((float)(2.0 * (turns - floor(turns))), &sv, &cv);
        c[i] = cv;
        s[i] = sv;
    }
}

// Per-head RMSNorm of one fp16 vector of HD values by one wavefront:
// dst[i] = fp16(src[i] * w[i] * r(src)) (w == null: no scale).
template <int HD>
__device__ __forceinline__ void wave_head_norm(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                               const uint16_t* __restrict__ w, float eps) {
    const uint32_t lane = threadIdx.x & 63u;
    constexpr int PER = HD / 64;
    float v[PER];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        v[i] = h2f(src[lane + 64 * i]);
        ss = fmaf(v[i], v[i], ss);
    }
    ss = seg_sum<kWave>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const uint32_t e = lane + 64 * i;
        const float xw = w ? v[i] * h2f(w[e]) : v[i];
        dst[e] = f2h(xw * inv);
    }
}

template <int HD, int GB>
struct AttnLds {
    uint16_t q[GB][HD];
    uint16_t wn[2][HD];       // q and k norm weights
    uint16_t kp[HD];
    uint16_t vp[HD];
    float rc[HD / 2];
    float rs[HD / 2];
    float p[GB][kAttnChunk];
    float ml[GB][2];
    float red[2048 / HD][GB][HD];
};

// One (chunk, kv head, query-head subset) block: blockIdx = (chunk, kv head h,
// subset z), query heads h·G + z·GB + [0, GB). q: fp16 [num_q_heads][HD] (raw
// projection when the epilogue is on); part_o: fp32
// [num_q_heads][nchunks][HD]; part_ml: fp32 [num_q_heads][nchunks][2].
// With GB < G every subset block of the new token's chunk runs the k/v
// epilogue on the staged raw rows (epi.k_raw / v_raw) and writes the same
// words into the cache slot; nothing reads that slot from the caches.
template <int HD, int G, int GB = G>
__device__ __forceinline__ void attn_partial(const uint16_t* __restrict__ q, uint16_t* __restrict__ kc,
                                             uint16_t* __restrict__ vc, uint32_t nkv, uint32_t seq_len,
                                             uint32_t kv_start, float scale, const AttnEpilogue& epi,
                                             float* __restrict__ part_o, float* __restrict__ part_ml) {
    static_assert(HD == 128 || HD == 256 || HD == 512, "head_dim 128, 256 or 512");
    static_assert(GB >= 1 && G % GB == 0, "query heads split evenly over blocks");
    constexpr uint32_t CPL = HD / 128;                 // 16-byte pieces per lane per key (q·k)
    constexpr uint32_t TPR = HD / 8;                   // threads per V row
    constexpr uint32_t VGROUPS = kAttnThreads / TPR;
    constexpr uint32_t KPG = kAttnChunk / VGROUPS;     // keys per V group
    constexpr uint32_t KSTEPS = kAttnChunk / (kAttnThreads / kAttnKeyLanes);
    __shared__ __attribute__((aligned(16))) AttnLds<HD, GB> L;

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t chunk = blockIdx.x, h = blockIdx.y, nchunks = gridDim.x;
    const uint32_t qh0 = h * G + (GB < G ? blockIdx.z * GB : 0u);       // first query head of the block
    const uint32_t c0 = kv_start + chunk * kAttnChunk;
    const uint32_t n = seq_len - c0 < kAttnChunk ? seq_len - c0 : kAttnChunk;
    const size_t row = (size_t)nkv * HD;               // halves between consecutive positions
    const uint16_t* kbase = kc + (size_t)c0 * row + (size_t)h * HD;
    const uint16_t* vbase = vc + (size_t)c0 * row + (size_t)h * HD;
    const bool epi_on = epi.q_norm != nullptr;
    const uint32_t pos = seq_len - 1;                  // the new token
    const bool own_pos = epi_on && pos >= c0 && pos < c0 + n;

    // 1. loads, in the order they are waited for: the queries (16-byte
    // chunks; G*HD/8 <= 256 of them), the norm weights and, in the block that
    // owns it, the new token's raw k and v rows; then the chunk's K rows (its
    // V rows follow the epilogue). No load is predicated (rows past the
    // chunk's end re-read its last row and are masked afterwards, threads
    // past the queries re-read the last chunk, blocks without the new token
    // re-read the queries), so each wait covers exactly the loads before it:
    // the epilogue runs while K streams in, the scores while V does.
    constexpr uint32_t QCH = GB * HD / 8;
    constexpr uint32_t KVCH = 2 * (HD / 8);
    static_assert(QCH <= kAttnThreads && KVCH <= kAttnThreads, "one chunk per thread");
    const uint4 qraw = reinterpret_cast<const uint4*>(q + (size_t)qh0 * HD)[tid < QCH ? tid : QCH - 1];
    const uint32_t kvi = tid % KVCH;
    const uint16_t* kvsrc = !own_pos ? q
                            : epi.k_raw ? (kvi < HD / 8 ? epi.k_raw : epi.v_raw) + (size_t)h * HD
                                        : (kvi < HD / 8 ? kc : vc) + (size_t)pos * row + (size_t)h * HD;
    const uint4 kvraw = reinterpret_cast<const uint4*>(kvsrc)[kvi % (HD / 8)];
    const uint16_t* wsrc = epi_on ? (kvi < HD / 8 ? epi.q_norm : epi.k_norm) : q;
    const uint4 wraw = reinterpret_cast<const uint4*>(wsrc)[kvi % (HD / 8)];

    const uint32_t sl = lane & (kAttnKeyLanes - 1);
    uint4 kr[KSTEPS][CPL];
#pragma unroll
    for (uint32_t st = 0; st < KSTEPS; ++st) {
        const uint32_t j = st * (kAttnThreads / kAttnKeyLanes) + (tid >> 4);
        const uint32_t jr = j < n ? j : n - 1;
#pragma unroll
        for (uint32_t cc = 0; cc < CPL; ++cc)
            kr[st][cc] = *reinterpret_cast<const uint4*>(kbase + jr * row + 8u * (sl + 16u * cc));
    }
    // 2. queries (and the new token's k/v) through the epilogue
    if (tid < QCH) reinterpret_cast<uint4*>(&L.q[0][0])[tid] = qraw;
    if (epi_on) {
        rope_table(L.rc, L.rs, epi.rotated_pairs, HD, pos, epi.log2_theta);
        if (tid < KVCH) {
            reinterpret_cast<uint4*>(&L.wn[0][0])[tid] = wraw;
            if (own_pos) reinterpret_cast<uint4*>(tid < HD / 8 ? L.kp : L.vp)[tid % (HD / 8)] = kvraw;
        }
        __syncthreads();
        const uint32_t nvec = GB + (own_pos ? 2u : 0u);
        for (uint32_t v = wave; v < nvec; v += kAttnThreads / 64) {
            uint16_t* buf = v < GB ? L.q[v] : (v == GB ? L.kp : L.vp);
            const uint16_t* w = v < GB ? L.wn[0] : (v == GB ? L.wn[1] : nullptr);
            wave_head_norm<HD>(buf, buf, w, epi.eps);
        }
        __syncthreads();
        const uint32_t nrot = GB + (own_pos ? 1u : 0u);
        for (uint32_t i = tid; i < nrot * epi.rotated_pairs; i += kAttnThreads) {
            const uint32_t v = i / epi.rotated_pairs, pr = i % epi.rotated_pairs;
            uint16_t* buf = v < GB ? L.q[v] : L.kp;
            const float x0 = h2f(buf[pr]), x1 = h2f(buf[pr + HD / 2]);
            buf[pr] = f2h(x0 * L.rc[pr] - x1 * L.rs[pr]);
            buf[pr + HD / 2] = f2h(x0 * L.rs[pr] + x1 * L.rc[pr]);
        }
        __syncthreads();
        if (own_pos && tid < 2 * (HD / 8)) {   // the cache keeps the processed k/v of the new token
            uint16_t* dst = (tid < HD / 8 ? kc : vc) + (size_t)pos * row + (size_t)h * HD;
            reinterpret_cast<uint4*>(dst)[tid % (HD / 8)] =
                reinterpret_cast<const uint4*>(tid < HD / 8 ? L.kp : L.vp)[tid % (HD / 8)];
        }
    } else {
        __syncthreads();
    }

    // the chunk's V rows, issued after the epilogue: a wave stalls while the
    // memory pipeline backs up under its loads, so the epilogue runs under
    // the K stream (which alone keeps HBM busy) instead of after both
    const uint32_t vg = tid / TPR, vl = tid % TPR;
    uint4 vr[KPG];
#pragma unroll
    for (uint32_t i = 0; i < KPG; ++i) {
        const uint32_t j = vg * KPG + i;
        vr[i] = *reinterpret_cast<const uint4*>(vbase + (j < n ? j : n - 1) * row + 8u * vl);
    }

    // 3. scores
    h2 qv[GB][CPL][4];
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
        for (uint32_t cc = 0; cc < CPL; ++cc) {
            const uint4 raw = *reinterpret_cast<const uint4*>(&L.q[g][8u * (sl + 16u * cc)]);
            qv[g][cc][0] = __builtin_bit_cast(h2, raw.x);
            qv[g][cc][1] = __builtin_bit_cast(h2, raw.y);
            qv[g][cc][2] = __builtin_bit_cast(h2, raw.z);
            qv[g][cc][3] = __builtin_bit_cast(h2, raw.w);
        }
#pragma unroll
    for (uint32_t st = 0; st < KSTEPS; ++st) {
        const uint32_t j = st * (kAttnThreads / kAttnKeyLanes) + (tid >> 4);
        float acc[GB];
#pragma unroll
        for (int g = 0; g < GB; ++g) acc[g] = 0.0f;
#pragma unroll
        for (uint32_t cc = 0; cc < CPL; ++cc) {
            uint4 kk = kr[st][cc];
            if (own_pos && c0 + j == pos) kk = *reinterpret_cast<const uint4*>(&L.kp[8u * (sl + 16u * cc)]);
            const h2 k4[4] = {__builtin_bit_cast(h2, kk.x), __builtin_bit_cast(h2, kk.y),
                              __builtin_bit_cast(h2, kk.z), __builtin_bit_cast(h2, kk.w)};
#pragma unroll
            for (int g = 0; g < GB; ++g)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[g] = __builtin_amdgcn_fdot2(k4[e], qv[g][cc][e], acc[g], false);
        }
#pragma unroll
        for (int g = 0; g < GB; ++g) {
            const float sdot = row16_sum(acc[g]);
            if (sl == 0) L.p[g][j] = j < n ? sdot * scale : -__builtin_inff();
        }
    }
    __syncthreads();

    // 4. chunk softmax statistics, one wavefront per query head
    for (uint32_t g = wave; g < (uint32_t)GB; g += kAttnThreads / 64) {
        const float sv = lane < kAttnChunk ? L.p[g][lane] : -__builtin_inff();
        const float m = wave_max(sv);
        const float e = lane < n ? expf(sv - m) : 0.0f;
        const float l = wave_sum(e);
        if (lane < kAttnChunk) L.p[g][lane] = e;
        if (lane == 0) {
            L.ml[g][0] = m;
            L.ml[g][1] = l;
        }
    }
    __syncthreads();

    // 5. p·V
    float o[GB][8];
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < KPG; ++i) {
        const uint32_t j = vg * KPG + i;
        uint4 vv = vr[i];
        if (own_pos && c0 + j == pos) vv = *reinterpret_cast<const uint4*>(&L.vp[8u * vl]);
        const h8 v8 = __builtin_bit_cast(h8, vv);
#pragma unroll
        for (int g = 0; g < GB; ++g) {
            const float pj = L.p[g][j];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pj, (float)v8[e], o[g][e]);
        }
    }
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) L.red[vg][g][8u * vl + e] = o[g][e];
    __syncthreads();
    for (uint32_t i = tid; i < GB * HD; i += kAttnThreads) {
        const uint32_t g = i / HD, d = i % HD;
        float s = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < VGROUPS; ++r) s += L.red[r][g][d];
        const size_t qh = (size_t)qh0 + g;
        part_o[(qh * nchunks + chunk) * HD + d] = s;
    }
    if (tid < (uint32_t)GB) {
        const size_t qh = (size_t)qh0 + tid;
        part_ml[(qh * nchunks + chunk) * 2 + 0] = L.ml[tid][0];
        part_ml[(qh * nchunks + chunk) * 2 + 1] = L.ml[tid][1];
    }
}

// Merge of the chunks of query head blockIdx.x, head dims
// [64·blockIdx.y, 64·blockIdx.y + 64). Thread (cg, d4) accumulates float4 d4
// of the chunks c ≡ cg (mod 16); its first four loads are issued before the
// weights are formed (rows past the last chunk re-read it and get weight 0),
// so the block waits for one memory round trip, not two. The 16 partial sums
// are added through LDS in cg order.
template <int HD>
__device__ __forceinline__ void attn_combine(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                             uint16_t* __restrict__ out, uint32_t nchunks) {
    static_assert(HD % kAttnCombineDims == 0, "head dims split in 64s");
    constexpr uint32_t NV = kAttnCombineDims / 4;               // float4 columns per block
    constexpr uint32_t NG = kAttnCombineThreads / NV;           // chunk groups
    constexpr uint32_t PRE = 4;
    __shared__ float wgt[kAttnMaxChunks];
    __shared__ float tot;
    __shared__ float4 red[NG][NV];
    const uint32_t qh = blockIdx.x, tid = threadIdx.x, d4 = tid % NV, cg = tid / NV;
    const float4* po = reinterpret_cast<const float4*>(part_o + (size_t)qh * nchunks * HD +
                                                       (size_t)blockIdx.y * kAttnCombineDims) + d4;
    float4 pre[PRE];
#pragma unroll
    for (uint32_t i = 0; i < PRE; ++i) {
        const uint32_t c = cg + NG * i;
        pre[i] = po[(size_t)(c < nchunks ? c : nchunks - 1) * (HD / 4)];
    }
    const float* ml = part_ml + (size_t)qh * nchunks * 2;
    if (tid < kWave) {
        float m = -__builtin_inff();
        float l = 0.0f;
        if (nchunks <= kWave) {
            // one chunk per lane: its (m, l) pair loaded once, unconditionally
            // (clamped), so it shares the partials' memory round trip; the
            // same values and operations as the loops below
            const bool own = tid < nchunks;
            const float2 v = reinterpret_cast<const float2*>(ml)[own ? tid : nchunks - 1];
            m = wave_max(own ? v.x : -__builtin_inff());
            const float w = expf(v.x - m);
            // unguarded (slots past nchunks are never read): no branch that
            // the compiler could sink the pair's second half under
            wgt[tid] = own ? w : 0.0f;
            l = wave_sum(own ? fmaf(w, v.y, 0.0f) : 0.0f);
        } else {
            for (uint32_t c = tid; c < nchunks; c += kWave) m = fmaxf(m, ml[2 * c]);
            m = wave_max(m);
            for (uint32_t c = tid; c < nchunks; c += kWave) {
                const float w = expf(ml[2 * c] - m);
                wgt[c] = w;
                l = fmaf(w, ml[2 * c + 1], l);
            }
            l = wave_sum(l);
        }
        if (tid == 0) tot = l;
    }
    __syncthreads();
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (uint32_t i = 0; i < PRE; ++i) {
        const uint32_t c = cg + NG * i;
        const float w = c < nchunks ? wgt[c] : 0.0f;
        acc.x = fmaf(w, pre[i].x, acc.x);
        acc.y = fmaf(w, pre[i].y, acc.y);
        acc.z = fmaf(w, pre[i].z, acc.z);
        acc.w = fmaf(w, pre[i].w, acc.w);
    }
    for (uint32_t c = cg + NG * PRE; c < nchunks; c += NG) {
        const float w = wgt[c];
        const float4 v = po[(size_t)c * (HD / 4)];
        acc.x = fmaf(w, v.x, acc.x);
        acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z);
        acc.w = fmaf(w, v.w, acc.w);
    }
    red[cg][d4] = acc;
    __syncthreads();
    if (tid < kAttnCombineDims) {
        const float* r = reinterpret_cast<const float*>(&red[0][0]) + tid;
        float s = 0.0f;
#pragma unroll
        for (uint32_t g = 0; g < NG; ++g) s += r[g * kAttnCombineDims];
        out[(size_t)qh * HD + (size_t)blockIdx.y * kAttnCombineDims + tid] = f2h(s / tot);
    }
}

// Decode-layer tail (one block): recomputes the post-attention residual
// stream h = fp16(hidden + fp16(attn·w_post_attn·r(attn))), normalises the
// shared-expert output h1 (post_feedforward_layernorm_1) and the routed output
// h2 (post_feedforward_layernorm_2), adds them, normalises the sum
// (post_feedforward_layernorm), adds it to h and scales by the layer scalar:
//     out = fp16(fp16(h + fp16(h12·w_post_ffn·r(h12))) · fp16(layer_scalar)),
//     h12 = fp16(fp16(h1·w_sp·r(h1)) + fp16(h2·w_pf2·r(h2)))
// (fused_post_attn_setup / rmsnorm / fused_layer_tail,
// S/Metal/Fusions/fused.metal:199-231,270-375). Each thread owns one 16-byte
// chunk of every vector and loads all eight at once; requires D % 8 == 0,
// D <= 8·kLayerTailThreads and 16-byte aligned vectors (the host checks).
__device__ __forceinline__ void layer_tail(const uint16_t* __restrict__ hidden, const uint16_t* __restrict__ attn,
                                           const uint16_t* __restrict__ w_post_attn,
                                           const uint16_t* __restrict__ h1, const uint16_t* __restrict__ w_sp,
                                           const uint16_t* __restrict__ h2, const uint16_t* __restrict__ w_pf2,
                                           const uint16_t* __restrict__ w_pf, float eps, float layer_scalar,
                                           uint16_t* __restrict__ out, uint32_t D) {
    const uint32_t c = threadIdx.x;
    const bool live = c < (D >> 3);
    h8 hv{}, av{}, paw{}, h1v{}, spw{}, h2v{}, pf2w{}, pfw{};
    if (live) {
        hv = __builtin_bit_cast(h8, ld16h(hidden, c));
        av = __builtin_bit_cast(h8, ld16h(attn, c));
        paw = __builtin_bit_cast(h8, ld16h(w_post_attn, c));
        h1v = __builtin_bit_cast(h8, ld16h(h1, c));
        spw = __builtin_bit_cast(h8, ld16h(w_sp, c));
        h2v = __builtin_bit_cast(h8, ld16h(h2, c));
        pf2w = __builtin_bit_cast(h8, ld16h(w_pf2, c));
        pfw = __builtin_bit_cast(h8, ld16h(w_pf, c));
    }
    const float n = (float)D;
    float ss[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        ss[0] = fmaf((float)av[e], (float)av[e], ss[0]);
        ss[1] = fmaf((float)h1v[e], (float)h1v[e], ss[1]);
        ss[2] = fmaf((float)h2v[e], (float)h2v[e], ss[2]);
    }
    block_sums<3, kLayerTailThreads>(ss);
    const float inv_a = 1.0f / sqrtf(ss[0] / n + eps);
    const float inv_1 = 1.0f / sqrtf(ss[1] / n + eps);
    const float inv_2 = 1.0f / sqrtf(ss[2] / n + eps);
    h8 h12;
    float s12[1] = {0.0f};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const _Float16 an = (_Float16)((float)av[e] * (float)paw[e] * inv_a);
        hv[e] = (_Float16)((float)hv[e] + (float)an);
        const _Float16 a1 = (_Float16)((float)h1v[e] * (float)spw[e] * inv_1);
        const _Float16 a2 = (_Float16)((float)h2v[e] * (float)pf2w[e] * inv_2);
        h12[e] = (_Float16)((float)a1 + (float)a2);
        s12[0] = fmaf((float)h12[e], (float)h12[e], s12[0]);
    }
    if (!live) s12[0] = 0.0f;
    block_sums<1, kLayerTailThreads>(s12);
    const float inv_12 = 1.0f / sqrtf(s12[0] / n + eps);
    const float sc = (float)(_Float16)layer_scalar;
    h8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const _Float16 t2 = (_Float16)((float)h12[e] * (float)pfw[e] * inv_12);
        const _Float16 r = (_Float16)((float)hv[e] + (float)t2);
        o[e] = (_Float16)((float)r * sc);
    }
    if (live) reinterpret_cast<h8*>(out)[c] = o;
}

}  // namespace tfq
