// Persistent batched decode step (batched.hip), called by msd_batch_decode_step (prefill.hip).
#ifndef MSD_BATCHED_H
#define MSD_BATCHED_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/msdecode.h"

namespace mbd {

// Bytes at the start of the batched workspace that the persistent step owns (exchange
// vectors, barrier flags, epoch, status, argmax keys); 0 when the shape has no persistent plan.
int64_t region_bytes(const msd_config* cfg);

struct StepArgs {
  const msd_config* cfg;
  const uint16_t* emb;
  const uint16_t* outp;
  const uint16_t* w;
  const uint16_t* lnf;
  const float* rope;
  const int32_t* tokens;
  const int32_t* positions;
  int32_t batch;
  const int32_t* pages;
  int32_t max_pages;
  uint16_t* kv;
  int32_t pool_pages;
  void* region;      // region_bytes(cfg) bytes, zero-filled before the first step
  float* logits;
  int32_t* out;
  hipStream_t stream;
};

// Launches the persistent step when the shape, the batch and the device allow it: returns
// MSD_OK (launched), 1 (not applicable: the caller runs the multi-kernel step) or an error.
int32_t try_step(const StepArgs& s);

}  // namespace mbd

#endif  // MSD_BATCHED_H
