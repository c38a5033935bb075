// Internal declarations shared by the engine's translation units.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include <hip/hip_runtime_api.h>

#include "bsscl_hip.h"

namespace bsscl {

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const std::string &msg);

// Sampler hand-off used by bsscl_boost_round (sampler.cpp).
struct SamplerRound {
  const uint32_t *draws;  // j(n-1-t) at [t], t < n-1 (row bagging), else null
  const uint32_t *draws_dev;  // device copy of draws (device-rows samplers)
  hipEvent_t draws_copied;    // completes when draws_dev is written
  const int32_t *rows;    // sample_idx[n_sub] (host-rows samplers), else null
  const int32_t *feats;   // f_sub ascending feature indices
  int32_t round;          // 0-based round number
};
struct SamplerShape {
  int64_t n, n_sub;
  int32_t f_sub;
  bool do_rows, device_rows;
  int32_t device;
};
// Blocks until the next round is ready.  The buffers stay valid (and may be
// read by copies in flight) until sampler_give_back(token).
int sampler_take(bsscl_sampler *s, SamplerRound *out, void **token);
void sampler_give_back(bsscl_sampler *s, void *token);
SamplerShape sampler_shape(bsscl_sampler *s);
// Rounds not yet taken.
int32_t sampler_remaining(bsscl_sampler *s);

// The process's stream for the bagging draws' host-to-device copies on
// `device`, created once and kept until the process ends (nullptr when it
// cannot be created).  An engine asks for it right after creating its own
// two streams.  (With a new copy stream per sampler, some 10M x 50 fits ran
// their rounds in 3.9 ms against 2.5 ms, presumably when the new stream
// shared a hardware queue with the tree stream; with one stream per
// process no fit did.)
hipStream_t copy_stream(int device);

}  // namespace bsscl
