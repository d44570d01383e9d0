// noalloc.hpp -- the fixed device scratch behind glacier_attn_backward_noalloc.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "../../include/glacier_attn.h"

namespace glacier {

constexpr size_t kNoAllocScratchBytes = GLACIER_ATTN_NOALLOC_SCRATCH_BYTES;
constexpr int kNoAllocMaxDevices = 64;

// Looks up the scratch array's address on `device`, which must be the
// current device; once per device (later calls return at once).
hipError_t noalloc_scratch_init(int device);

// The scratch array's address on `device`, or nullptr before
// noalloc_scratch_init succeeded there.
void* noalloc_scratch(int device);

}  // namespace glacier
