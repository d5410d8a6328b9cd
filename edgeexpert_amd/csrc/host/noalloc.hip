// noalloc.hip — the device-resident scratch of tfq_moe_decode_token_noalloc.
//
// Compiled by hipcc into libtfq.so (host code plus a fat binary holding only
// this array). The array lives in device memory for as long as the process
// does, one copy per GPU; host code never uses its name as an address (in
// host code it is a stand-in symbol): tfq_create resolves the device address
// once per context with hipGetSymbolAddress, on the context's device, and the
// entry point passes that address to the kernels.
#include <hip/hip_runtime.h>

#include "module.hpp"
#include "noalloc.hpp"

namespace tfq {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

int noalloc_scratch_address(void** out) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_check(err, "hipGetSymbolAddress(scratch)");
    *out = ptr;
    return TFQ_OK;
}

}  // namespace tfq
