// Host-side description of one prefill launch.
#pragma once

#include "prefill_kernel.hpp"

namespace sia {

struct PrefillLaunch {
  PrefillArgs a;
  PackArgs pack;   // V -> f16 V^T block images (run first on the same stream)
  int D;
  int dtype;
  int var;         // prefill_fwd configuration: 0, or 1 = 4-wave groups at D = 128 (grids too small for the CUs)
  hipStream_t stream;
};

int launch_prefill(PrefillLaunch& L);

}  // namespace sia
