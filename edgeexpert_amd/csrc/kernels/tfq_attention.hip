// tfq_attention.hip — split-K GQA decode attention (with the Gemma 4 q/k/v epilogue), its
// combine, and the decoder layer's tail.
#include "entry_points.hpp"

TFQ_ATTN(128, 1)
TFQ_ATTN(128, 2)
TFQ_ATTN(128, 4)
TFQ_ATTN(256, 1)
TFQ_ATTN(256, 2)
TFQ_ATTN(256, 4)
TFQ_ATTN(512, 1)
TFQ_ATTN(512, 2)
TFQ_ATTN(512, 4)
TFQ_ATTN_GB(512, 8, 4)
TFQ_ATTN_COMBINE(128)
TFQ_ATTN_COMBINE(256)
TFQ_ATTN_COMBINE(512)

extern "C" __global__ __launch_bounds__(kLayerTailThreads) void tfq_layer_tail(
    const uint16_t* hidden, const uint16_t* attn, const uint16_t* w_post_attn, const uint16_t* h1,
    const uint16_t* w_sp, const uint16_t* h2, const uint16_t* w_pf2, const uint16_t* w_pf, float eps,
    float layer_scalar, uint16_t* out, uint32_t D) {
    layer_tail(hidden, attn, w_post_attn, h1, w_sp, h2, w_pf2, w_pf, eps, layer_scalar, out, D);
}
