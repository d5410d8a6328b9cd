// module.hpp — the loaded gfx950 code object and the launch/error plumbing
// shared by the operator classes (ops.hpp) and the C ABI (tfq.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../../include/tfq.h"

namespace tfq {

// Per-thread record of the last failure (returned through tfq_last_*()).
struct ErrorState {
    int hip = 0;
    char message[512] = {0};
};
ErrorState& error_state();

inline int fail(int status, const char* fmt, ...) {
    ErrorState& e = error_state();
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(e.message, sizeof(e.message), fmt, ap);
    va_end(ap);
    return status;
}

inline int hip_check(hipError_t err, const char* what) {
    if (err == hipSuccess) return TFQ_OK;
    ErrorState& e = error_state();
    e.hip = (int)err;
    std::snprintf(e.message, sizeof(e.message), "%s: %s", what, hipGetErrorString(err));
    return TFQ_E_HIP;
}

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

inline uint32_t pow2ceil(uint32_t v) {
    uint32_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

// The code objects (one per kernel translation unit, lib/tfq_*.co): every
// kernel resolved by name once, at creation, across all of them.
class Module {
public:
    // dir: the directory holding the code objects.
    int load(const std::string& dir);
    ~Module();
    hipFunction_t get(const std::string& name) const {
        auto it = fns_.find(name);
        return it == fns_.end() ? nullptr : it->second;
    }
    int device() const { return device_; }

    // Blocks of `block` threads and `lds` dynamic LDS bytes that the whole GPU
    // holds resident at once for kernel f (occupancy per CU x CUs); cached
    // per (kernel, lds), at least 1.
    uint32_t resident_blocks(hipFunction_t f, uint32_t block, uint32_t lds) const;

private:
    std::vector<hipModule_t> modules_;
    int device_ = -1;
    uint32_t cus_ = 1;
    std::unordered_map<std::string, hipFunction_t> fns_;
    mutable std::mutex occ_mu_;
    mutable std::map<std::pair<hipFunction_t, uint64_t>, uint32_t> occ_;
};

// Launch with kernel arguments given as an array of pointers to values.
inline int launch(hipFunction_t f, uint32_t grid, uint32_t block, uint32_t lds, void* stream,
                  void** args, const char* name) {
    if (!f) return fail(TFQ_E_NOT_LOADED, "kernel %s is not in the code object", name);
    return hip_check(hipModuleLaunchKernel(f, grid, 1, 1, block, 1, 1, lds, (hipStream_t)stream,
                                           args, nullptr),
                     name);
}

// Instantiation picked for a reduction of `chunks` 16-byte chunks per row:
// SEG lanes per row (power of two <= 64) and P chunks per lane.
struct SegShape {
    uint32_t seg;
    uint32_t p;
};

inline SegShape seg_shape(uint32_t chunks, uint32_t min_seg) {
    if (chunks <= 64) {
        uint32_t s = pow2ceil(chunks);
        return {s < min_seg ? min_seg : s, 1};
    }
    return {64, (chunks + 63) / 64};
}

// int4 families: the (SEG >= 8, P <= 4) pair with the fewest idle chunk
// slots (SEG·P - chunks); ties go to the larger SEG (fewer registers).
inline SegShape seg_shape_fit(uint32_t chunks, uint32_t min_seg) {
    if (chunks <= 8) return seg_shape(chunks, min_seg);
    SegShape best{64, (chunks + 63) / 64};
    uint32_t best_waste = best.seg * best.p - chunks;
    for (uint32_t seg = 32; seg >= 8; seg >>= 1) {
        const uint32_t p = (chunks + seg - 1) / seg;
        if (p > 4) continue;
        const uint32_t waste = seg * p - chunks;
        if (waste < best_waste) {
            best = {seg, p};
            best_waste = waste;
        }
    }
    return best;
}

}  // namespace tfq
