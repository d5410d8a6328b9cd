// tfq_gemm.hip — the prefill dequant-fused GEMM: the 64-token MFMA projection tile
// and the few-token weight stream, int4 and 3-bit, fp16 and bf16 activations.
#include "entry_points.hpp"

#define TFQ_GEMM(TAG, BITS, DT, X_BF16)                                                          \
    extern "C" __global__ __launch_bounds__(kProjGemmThreads) void tfq_gemm_##TAG##_##DT(        \
        const uint16_t* X, const uint8_t* W, const uint16_t* S, const uint16_t* B, uint16_t* Y,  \
        uint32_t M, uint32_t N, uint32_t K, uint32_t ldx, uint32_t ldy) {                          \
        gemm_q4_proj<X_BF16, BITS>(X, W, S, B, Y, M, N, K, ldx, ldy);                             \
    }
TFQ_GEMM(q4, 4, f16, false)
TFQ_GEMM(q4, 4, bf16, true)
TFQ_GEMM(q3, 3, f16, false)
TFQ_GEMM(q3, 3, bf16, true)

// Few-token form (gemm_skinny.hpp): RT 16-row MFMA tiles per wave, C = ceil(K/1024)
// 128-code tiles per wave.
#define TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, C)                                                 \
    extern "C" __global__ __launch_bounds__(kSkinnyThreads) void                                  \
        tfq_gemm_skinny_##TAG##_##DT##_r##RT##_c##C(const uint16_t* X, const uint8_t* W,          \
                                                    const uint16_t* S, const uint16_t* B,         \
                                                    uint16_t* Y, uint32_t M, uint32_t N,          \
                                                    uint32_t K, uint32_t ldx, uint32_t ldy) {     \
        gemm_skinny<X_BF16, RT, BITS, C>(X, W, S, B, Y, M, N, K, ldx, ldy);                       \
    }
#define TFQ_SKINNY_C(TAG, BITS, DT, X_BF16, RT)                                                  \
    TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 1) TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 2)              \
    TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 3) TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 4)              \
    TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 5) TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 6)              \
    TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 7) TFQ_SKINNY(TAG, BITS, DT, X_BF16, RT, 8)
TFQ_SKINNY_C(q4, 4, f16, false, 1)
TFQ_SKINNY_C(q4, 4, f16, false, 2)
TFQ_SKINNY_C(q4, 4, bf16, true, 1)
TFQ_SKINNY_C(q4, 4, bf16, true, 2)
TFQ_SKINNY_C(q3, 3, f16, false, 1)
TFQ_SKINNY_C(q3, 3, f16, false, 2)
TFQ_SKINNY_C(q3, 3, bf16, true, 1)
TFQ_SKINNY_C(q3, 3, bf16, true, 2)
