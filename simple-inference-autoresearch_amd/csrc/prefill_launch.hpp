// Host-side description of one prefill launch.
#pragma once

#include "prefill_kernel.hpp"

namespace sia {

struct PrefillLaunch {
  PrefillArgs a;
  PackArgs pack;   // V -> f16 V^T block images (run first on the same stream)
  int D;
  int dtype;
  int var;         // prefill_fwd configuration: 0, or 1 = 4-wave groups at D = 128 (grids too small for the CUs),
                   // 2 = variant 1 with the V^T images built in LDS (short key ranges; no prefill_pack_v)
  hipStream_t stream;
};

// Longest key range that runs variant 2 (bfloat16: float16 at D = 128 reads
// raw V rows at every length and never repacks).  The in-LDS conversion costs a
// work-group ~0.65 us per 64-key block, the separate repack ~3 us per call
// (its launch and one load/store round trip): one sequence of 128 tokens
// 9.8 -> 8.1 us per call, but 512 tokens 15.7 -> 18.1 and 1024 24.0 -> 31.0.
constexpr int kPackvMaxKeys = 256;

int launch_prefill(PrefillLaunch& L);

}  // namespace sia
