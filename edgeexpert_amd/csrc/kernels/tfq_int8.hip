// tfq_int8.hip — int8 GEMV, the int8 shared expert's fused gate/up/act, the router
// (decode and prefill) logits and top-k selection.
#include "entry_points.hpp"

TFQ_Q8_TABLE(TFQ_Q8_GEMV)
TFQ_Q8_TABLE(TFQ_Q8_GATE_UP)
TFQ_Q8_TABLE(TFQ_ROUTER)
TFQ_Q8_TABLE(TFQ_PREFILL_ROUTER)

extern "C" __global__ __launch_bounds__(256) void tfq_router_select(const float* logits,
                                                                    const uint16_t* gain,
                                                                    uint32_t* out_idx,
                                                                    uint16_t* out_w,
                                                                    float* out_wf, uint32_t E,
                                                                    uint32_t k) {
    router_select(logits, gain, out_idx, out_w, out_wf, E, k);
}

// Per-token selection for a prefill chunk: one block per token.
extern "C" __global__ __launch_bounds__(256) void tfq_prefill_select(const float* logits,
                                                                     const uint16_t* gain,
                                                                     uint32_t* out_idx,
                                                                     uint16_t* out_w,
                                                                     float* out_wf, uint32_t E,
                                                                     uint32_t k) {
    const size_t t = blockIdx.x;
    router_select(logits + t * E, gain, out_idx + t * k, out_w + t * k, out_wf ? out_wf + t * k : nullptr,
                  E, k);
}
