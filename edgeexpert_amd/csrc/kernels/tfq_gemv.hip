// tfq_gemv.hip — int4/3-bit GEMV (plain, fused QKV, norm-staged forms), the greedy
// LM head, the HBM read probe and the BF16 -> fp16 converter.
#include "entry_points.hpp"

TFQ_Q4_TABLE(TFQ_Q4_GEMV)
TFQ_Q4_TABLE(TFQ_Q4_GEMV_TAIL)
TFQ_Q4_TABLE(TFQ_Q4_GEMV_WIDE)
TFQ_Q4_TABLE(TFQ_Q3_GEMV)
TFQ_Q4_TABLE(TFQ_LM_HEAD)

extern "C" __global__ __launch_bounds__(256) void tfq_lm_head_reduce(const uint64_t* summaries, uint32_t n,
                                                                     uint32_t* out_token) {
    lm_head_greedy_reduce(summaries, n, out_token);
}

extern "C" __global__ __launch_bounds__(256) void tfq_read_ceiling(const uint4* src, uint64_t n16,
                                                                     uint32_t* sink) {
    read_ceiling<4>(src, n16, sink);
}

extern "C" __global__ __launch_bounds__(256) void tfq_convert_bf16_f16(const uint16_t* src,
                                                                         uint16_t* dst, uint64_t n,
                                                                         uint32_t* inexact) {
    convert_bf16_to_f16(src, dst, n, inexact);
}
