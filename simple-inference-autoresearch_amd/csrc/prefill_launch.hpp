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
// raw V rows at every length and never repacks).  Converting each block in
// LDS costs the work-group ~0.3 us per 64-key block (its 16 KB read,
// converted and written back, one barrier); the separate repack ~3 us per
// call plus a kernel boundary.  One sequence at 32/8 heads, per call back to
// back: 128 / 256 / 384 / 512 tokens 8.15 / 11.24 / 13.89 / 15.84 ->
// 7.45 / 9.97 / 12.48 / 15.16 us, but 768 tokens 19.97 -> 20.24 and 1024
// 24.07 -> 25.32.
constexpr int kPackvMaxKeys = 512;

int launch_prefill(PrefillLaunch& L);

}  // namespace sia
