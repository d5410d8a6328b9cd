// abi_types.h — kernel-argument structs shared by the device code and the
// host launcher (plain C layout; passed by value through hipModuleLaunchKernel).
#pragma once
#include <stdint.h>

namespace tfq {

// One int4 matrix and its fp16 output, as seen by a multi-matrix launch.
struct Q4Mat {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
    uint16_t* y;
    uint32_t rows;
    uint32_t pad_;
};

// Up to three matrices sharing x and n (plain GEMV: 1; fused QKV: 3).
struct Q4Multi {
    Q4Mat m[3];
    uint32_t nmat;
    uint32_t total_rows;
};

// Sub-tensor byte offsets inside one routed-expert blob (MoEExpertOffsets).
struct ExpertOffsets {
    uint32_t gate_w, gate_s, gate_b;
    uint32_t up_w, up_s, up_b;
    uint32_t down_w, down_s, down_b;
};

// A layer's routed experts resident in HBM: blob(e) = base + e*stride.
struct ExpertPool {
    const uint8_t* base;
    uint64_t stride;
    uint32_t num_experts;
    uint32_t pad_;
    ExpertOffsets off;
};

// PrefillTokenExpertPair (S/Kernels/Prefill/MoE/PrefillRouter.swift:5-28).
struct Pair {
    uint32_t token;
    uint32_t expert;
    uint32_t rank;
    uint32_t weight_bits;
};

// One 128-row MFMA tile of one expert's run in the sorted pair list.
struct Tile {
    uint32_t expert;
    uint32_t start;
    uint32_t count;
    uint32_t pad_;
};

}  // namespace tfq
