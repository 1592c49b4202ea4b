// Decode kernel instantiations for f16 K/V (compiled separately to build in parallel).
#include "decode_launch.hpp"

namespace sia {

int launch_decode_f16(DecodeLaunch& L) {
  return launch_decode_q<F16, F32>(L);
}

}  // namespace sia
