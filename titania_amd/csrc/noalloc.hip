// A fixed device array for the entry points that must not allocate
// (th_attention_noalloc): callers under HIP graph capture, serving loops and
// harnesses that forbid hipMalloc.
//
// The array lives in the library's code object, so every GPU the library runs
// on holds its own copy, at its own address, until the process ends. In host
// code `scratch` names a host-side stand-in, not device memory: host code uses
// only the address hipGetSymbolAddress gives for the current device, which
// th_device_create looks up once per device and keeps in the device handle.
#include "common.h"

namespace {
// Covers the partials of one token at any context for up to 126 heads of
// head_dim 128 (63 of head_dim 256): a single-token call takes at most 256
// splits of (head_dim + 2) floats a head.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
}

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace th {

size_t noalloc_scratch_bytes() { return kNoAllocScratchBytes; }

int noalloc_scratch_address(void **ptr) {
    *ptr = nullptr;
    // ::scratch, the array: inside namespace th the bare name would be the
    // growable-scratch function th::scratch.
    hipError_t e = hipGetSymbolAddress(ptr, HIP_SYMBOL(::scratch));
    if (e != hipSuccess || !*ptr)
        return fail(TH_ERR_HIP, "hipGetSymbolAddress of the no-alloc scratch failed: %s", hipGetErrorString(e));
    return TH_OK;
}

}  // namespace th
