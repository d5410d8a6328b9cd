// noalloc.hpp — the fixed device scratch of the allocation-free decode entry
// point (tfq_moe_decode_token_noalloc): its size, layout and address lookup.
#pragma once

#include <stddef.h>

#include "../../../include/tfq.h"

namespace tfq {

// Routed activations of one token (fp16 [top_k][f]): phase 2 takes f <= 1024
// and top_k <= 8, so 16 KiB holds every shape the decode phases accept.
constexpr size_t kNoAllocActsBytes = 8u * 1024u * 2u;
// Then the router's fp32 logits (the router workspace).
constexpr size_t kNoAllocLogitsOffset = kNoAllocActsBytes;
constexpr size_t kNoAllocScratchBytes = kNoAllocActsBytes + TFQ_ROUTER_WORKSPACE_BYTES;
static_assert(TFQ_NOALLOC_SCRATCH_BYTES == kNoAllocScratchBytes, "tfq.h states the scratch size");

// Device address of the scratch array on the current device (its own copy on
// every GPU); hipGetSymbolAddress's status as a TFQ_* code.
int noalloc_scratch_address(void** out);

}  // namespace tfq
