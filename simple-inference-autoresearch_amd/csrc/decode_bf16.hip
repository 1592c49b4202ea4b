// Decode kernel instantiations for bf16 K/V (compiled separately to build in parallel).
#include "decode_launch.hpp"

namespace sia {

int launch_decode_bf16(DecodeLaunch& L) {
  return launch_decode_q<BF16, F32>(L);
}

}  // namespace sia
