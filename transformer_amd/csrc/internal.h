// Declarations shared between the library's source files (not part of the C ABI).
#ifndef MSD_INTERNAL_H
#define MSD_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "../../include/msdecode.h"

namespace msdc {

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) acts on the current device only, so the
// largest size set so far is remembered per (kernel, device) under a lock; a kernel launched on
// a second device gets its own call.  Thread-safe.  (msdecode.hip)
hipError_t ensure_dynamic_lds(const void* fn, size_t lds);

// The fused decode step has an instance and a plan for cfg on a grid of n_workgroups
// (LDS fit included; residency is checked at launch).  No HIP call.  (msdecode.hip)
bool decode_supported(const msd_config* cfg, int n_workgroups);

// The sampler takes a vocabulary of this size.  (sample.hip)
bool sample_supported(int vocab);

}  // namespace msdc

#endif  // MSD_INTERNAL_H
