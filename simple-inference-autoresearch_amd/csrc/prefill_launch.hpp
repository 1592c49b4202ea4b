// Host-side description of one prefill launch.
#pragma once

#include "prefill_kernel.hpp"

namespace sia {

struct PrefillLaunch {
  PrefillArgs a;
  PackArgs pack;   // V -> f16 V^T block images (run first on the same stream)
  int D;
  int dtype;
  hipStream_t stream;
};

int launch_prefill(PrefillLaunch& L);

}  // namespace sia
