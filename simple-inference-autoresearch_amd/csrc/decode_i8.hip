// Decode kernel instantiations for i8 K/V (compiled separately to build in parallel).
#include "decode_launch.hpp"

namespace sia {

int launch_decode_i8(DecodeLaunch& L) {
  if (L.scale_dtype == SIA_F32) return launch_decode_q<I8, F32>(L);
  if (L.scale_dtype == SIA_F16) return launch_decode_q<I8, F16>(L);
  return fail(SIA_ERR_UNSUPPORTED, "int8 KV scales must be float32 or float16");
}

}  // namespace sia
