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
// The same at D = 32 and 64, whose blocks (4 and 8 KB) cost less to convert:
// 768 tokens 13.41 -> 12.78 us (D = 32) and 17.41 -> 16.76 (D = 64), 1024
// tokens 16.15 -> 16.24 and 20.81 -> 20.98.
constexpr int kPackvMaxKeysD64 = 768;

int launch_prefill(PrefillLaunch& L);

}  // namespace sia
