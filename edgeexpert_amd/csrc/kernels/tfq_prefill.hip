// tfq_prefill.hip — grouped MoE prefill: device grouping of the routed pairs and the
// grouped gate/up and down launches (MFMA tile for large grouping tiles, weight
// stream for small ones, one launch each), at 4, 3 and 2 bits.
#include "entry_points.hpp"

extern "C" __global__ __launch_bounds__(kGroupThreads) void tfq_moe_group(
    const uint32_t* idx, const uint16_t* w, uint32_t T, uint32_t k, uint32_t E, Pair* sorted,
    uint32_t* offsets, uint32_t* counts, Tile* tiles, uint32_t* n_tiles, uint32_t* status) {
    moe_group(idx, w, T, k, E, sorted, offsets, counts, tiles, n_tiles, status);
}

// _t: the units' scale/bias tables staged through registers (aligned
// tables that fit, chosen by the host)
#define TFQ_GROUPED(SUFFIX, BITS, TAB)                                                           \
    extern "C" __global__ __launch_bounds__(kProjThreads, 2) void tfq_moe_grouped_gate_up##SUFFIX( \
        ExpertPool pool, const Pair* sorted, const Tile* tiles, uint32_t* n_tiles,               \
        const uint16_t* hidden, uint32_t stride, uint16_t* act, uint32_t D, uint32_t F,          \
        GroupedLaunch gl) {                                                                      \
        moe_grouped_gate_up_launch<BITS, TAB>(pool, sorted, tiles, n_tiles, hidden, stride, act, D, F, gl); \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(kProjThreads, 2) void tfq_moe_grouped_down##SUFFIX(  \
        ExpertPool pool, const Pair* sorted, const Tile* tiles, uint32_t* n_tiles,               \
        const uint16_t* act, uint16_t* partials, uint32_t D, uint32_t F, uint32_t k,             \
        GroupedLaunch gl) {                                                                      \
        moe_grouped_down_launch<BITS, TAB>(pool, sorted, tiles, n_tiles, act, partials, D, F, k, gl); \
    }
TFQ_GROUPED(, 4, false)
TFQ_GROUPED(_b2, 2, false)
TFQ_GROUPED(_b3, 3, false)
TFQ_GROUPED(_t, 4, true)
TFQ_GROUPED(_b2_t, 2, true)
TFQ_GROUPED(_b3_t, 3, true)
