// tfq_moe.hip — routed decode phase 2 (down + fixed-order weighted sum), the int4
// shared expert's fused gate/up/act, the prefill GeGLU and the token-major combine.
#include "entry_points.hpp"

TFQ_PHASE2(1)
TFQ_PHASE2(2)
TFQ_PHASE2(3)
TFQ_PHASE2(4)
TFQ_Q4_TABLE(TFQ_GATE_UP)

extern "C" __global__ __launch_bounds__(256) void tfq_gelu_mul_f16(const uint16_t* g, const uint16_t* u,
                                                                   uint16_t* act, uint64_t n) {
    gelu_mul_f16(g, u, act, n);
}

extern "C" __global__ __launch_bounds__(256) void tfq_moe_combine(const uint16_t* partials,
                                                                  const uint16_t* w, uint16_t* h2,
                                                                  uint32_t T, uint32_t k, uint32_t D) {
    moe_combine(partials, w, h2, T, k, D);
}

extern "C" __global__ __launch_bounds__(256) void tfq_moe_combine_x8(const uint16_t* partials,
                                                                     const uint16_t* w, uint16_t* h2,
                                                                     uint32_t T, uint32_t k, uint32_t D) {
    moe_combine_x8(partials, w, h2, T, k, D);
}
