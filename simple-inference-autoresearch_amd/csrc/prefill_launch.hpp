// Host-side description of one prefill launch.
#pragma once

#include "prefill_kernel.hpp"

namespace sia {

struct PrefillLaunch {
  PrefillArgs a;
  int D;
  int dtype;
  hipStream_t stream;
};

int launch_prefill(PrefillLaunch& L);

}  // namespace sia
