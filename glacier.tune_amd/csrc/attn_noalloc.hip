// attn_noalloc.hip -- the fixed device scratch of glacier_attn_backward_noalloc.
//
// The allocation-free backward keeps every buffer it needs beyond the
// caller's tensors (RoPE tables, tile table, row stats, per-head dK/dV
// partials) in one file-scope device array.  Each GPU that loads the library
// holds its own copy of the array, at its own address, until the process
// ends.  Host code must never pass the array's name to a kernel or a copy:
// in host code it is only a stand-in for the symbol.  The device address is
// taken once per device with hipGetSymbolAddress (glacier_attn_create calls
// noalloc_scratch_init with that device current) and used from then on.
#include <hip/hip_runtime.h>

#include <mutex>

#include "noalloc.hpp"

namespace glacier {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kNoAllocMaxDevices] = {};

}  // namespace

hipError_t noalloc_scratch_init(int device) {
  if (device < 0 || device >= kNoAllocMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_scratch_mutex);
  if (g_scratch_ptr[device] != nullptr) return hipSuccess;
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return e;
  if (current != device) return hipErrorInvalidDevice;
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  g_scratch_ptr[device] = p;
  return hipSuccess;
}

void* noalloc_scratch(int device) {
  if (device < 0 || device >= kNoAllocMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(g_scratch_mutex);
  return g_scratch_ptr[device];
}

}  // namespace glacier
