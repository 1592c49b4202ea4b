// Prefill (flash-attention forward) instantiations and launcher.
#include "host_util.hpp"
#include "prefill_kernel.hpp"
#include "prefill_launch.hpp"

namespace sia {

template <int D, class T, int VAR>
static int launch_fwd(PrefillLaunch& L, int rope);

template <int D, class T>
static int launch_prefill_typed(PrefillLaunch& L) {
  // rotary variant: none, or split-half / interleaved pairs from 16-bit / fp32 tables
  const int rope = L.a.cs == nullptr ? kRopeNone : 1 + (L.a.interleaved ? 1 : 0) + (L.a.tab_dt == SIA_F32 ? 2 : 0);
  if (L.pack.nblocks > 0) {
    // one work-group per 64-key V^T image
    hipLaunchKernelGGL((prefill_pack_v<D, T>), dim3((unsigned)L.pack.nblocks), dim3(256), 0, L.stream, L.pack);
  }
  // (variant 2 converts bf16 V in LDS; float16 V needs no conversion and
  // runs without a repack in any variant)
  if constexpr ((D == 32 || D == 64 || D == 128) && std::is_same<T, BF16>::value)
    if (L.var == 2) return launch_fwd<D, T, 2>(L, rope);
  if constexpr (D == 128)
    if (L.var == 1) return launch_fwd<D, T, 1>(L, rope);
  // (a variant the host picked but this head_dim/dtype has no kernel for
  // would run the images path on V^T images nobody wrote)
  if (L.var != 0) return fail(SIA_ERR_LAUNCH, "prefill variant %d is not built for head_dim %d", L.var, D);
  return launch_fwd<D, T, 0>(L, rope);
}

template <int D, class T, int VAR>
static int launch_fwd(PrefillLaunch& L, int rope) {
  const int nwg = L.a.nqblk * L.a.nunit;
  const dim3 grid(nwg), block(PfCfg<D, VAR>::waves * 64);
  switch (rope) {
    case kRopeNone: hipLaunchKernelGGL((prefill_fwd<D, T, kRopeNone, VAR>), grid, block, 0, L.stream, L.a); break;
    case kRopeSplit16: hipLaunchKernelGGL((prefill_fwd<D, T, kRopeSplit16, VAR>), grid, block, 0, L.stream, L.a); break;
    case kRopeInter16: hipLaunchKernelGGL((prefill_fwd<D, T, kRopeInter16, VAR>), grid, block, 0, L.stream, L.a); break;
    case kRopeSplit32: hipLaunchKernelGGL((prefill_fwd<D, T, kRopeSplit32, VAR>), grid, block, 0, L.stream, L.a); break;
    default: hipLaunchKernelGGL((prefill_fwd<D, T, kRopeInter32, VAR>), grid, block, 0, L.stream, L.a); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIA_ERR_LAUNCH, "prefill launch: %s", hipGetErrorString(e));
  return SIA_OK;
}

int launch_prefill(PrefillLaunch& L) {
  const bool bf = L.dtype == SIA_BF16;
  switch (L.D) {
    case 16: return bf ? launch_prefill_typed<16, BF16>(L) : launch_prefill_typed<16, F16>(L);
    case 32: return bf ? launch_prefill_typed<32, BF16>(L) : launch_prefill_typed<32, F16>(L);
    case 64: return bf ? launch_prefill_typed<64, BF16>(L) : launch_prefill_typed<64, F16>(L);
    case 128: return bf ? launch_prefill_typed<128, BF16>(L) : launch_prefill_typed<128, F16>(L);
    case 256: return bf ? launch_prefill_typed<256, BF16>(L) : launch_prefill_typed<256, F16>(L);
    default: return fail(SIA_ERR_UNSUPPORTED, "prefill head_dim %d not supported (16, 32, 64, 128, 256)", L.D);
  }
}

}  // namespace sia
