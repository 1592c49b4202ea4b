// Decode kernel instantiations for head_dim 256 (all K/V types).  Compiled
// without -amdgpu-mfma-vgpr-form: at this width the accumulators need AGPRs.
#include "decode_launch.hpp"

namespace sia {

template <class KV, class QT, class ST>
int launch_decode_256(DecodeLaunch& L) {
  return launch_decode_typed<256, KV, QT, ST>(L);
}

template int launch_decode_256<F16, F16, F32>(DecodeLaunch&);
template int launch_decode_256<F16, BF16, F32>(DecodeLaunch&);
template int launch_decode_256<BF16, F16, F32>(DecodeLaunch&);
template int launch_decode_256<BF16, BF16, F32>(DecodeLaunch&);
template int launch_decode_256<I8, F16, F32>(DecodeLaunch&);
template int launch_decode_256<I8, BF16, F32>(DecodeLaunch&);
template int launch_decode_256<I8, F16, F16>(DecodeLaunch&);
template int launch_decode_256<I8, BF16, F16>(DecodeLaunch&);

}  // namespace sia
