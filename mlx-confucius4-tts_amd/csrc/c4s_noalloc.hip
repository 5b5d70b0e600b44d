// Static device scratch of the no-allocation entry point
// (c4s_lmhead_sample_noalloc): when the caller passes no logits buffer, the
// LM head's logits handed to the sampler (the head folds its LayerNorm into
// the GEMM and keeps nothing else in memory).
//
// The array lives in the library's code object: each GPU the library runs on
// holds its own copy until the process ends. Host code never uses the array's
// name as an address: c4s_create asks for the current device's address once
// (noalloc_scratch) and passes that pointer to the kernels.

#include <hip/hip_runtime.h>

#include "c4s_internal.h"

namespace c4s {
namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

}  // namespace

hipError_t noalloc_scratch(void** ptr) {
  *ptr = nullptr;
  return hipGetSymbolAddress(ptr, HIP_SYMBOL(scratch));
}

}  // namespace c4s
