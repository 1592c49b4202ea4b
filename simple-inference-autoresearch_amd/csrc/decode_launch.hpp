// Host-side launch of the decode kernels (one instantiation unit per K/V dtype).
#pragma once

#include <type_traits>

#include "decode_kernel.hpp"
#include "host_util.hpp"

namespace sia {

constexpr int kDecodeWaves = 8;   // waves per work-group: one per KV-head unit of a page

// Waves per work-group of decode_main at head_dim D.  Up to D = 128 a group of
// 8 waves runs two per SIMD with 256 registers each.  At D = 256 the
// accumulators, the double-buffered tiles and the query operand need more
// than 256 registers, so the group has 4 waves, one per SIMD, each with the
// whole 512-entry register file (VGPRs plus AGPRs for the MFMA accumulators).
constexpr int decode_waves(int D) { return D >= 256 ? 4 : kDecodeWaves; }

struct DecodeLaunch {
  DecodeArgs a;
  int D;
  int q_dtype;       // SIA_F16 / SIA_BF16 / SIA_F32 (also the output dtype)
  int scale_dtype;   // SIA_F32 / SIA_F16 (int8 only)
  hipStream_t stream;
  hipEvent_t begin_event;   // optional, recorded around the main kernel
  hipEvent_t end_event;
  void* ws;                 // the caller's workspace (the fp32 path lays it out itself)
  size_t ws_bytes;
  int page_size;            // paged pools: tokens per page (0: contiguous cache)
};

inline size_t decode_lds_bytes(int D, int G16, int B, int NW) {
  return (size_t)NW * G16 * D * 4 + (size_t)2 * NW * G16 * 4 + (size_t)(2 * NW + 2) * 4 +
         (size_t)(B + 1) * 4 + (B <= kLensInLds ? (size_t)B * 4 : 0);
}

template <int D, class KV, class QT, class ST>
int launch_decode_typed(DecodeLaunch& L) {
  constexpr int NW = decode_waves(D);
  // int8 K/V: one vector scale load per lane (16 bytes of fp32 or 8 of fp16
  // scales) when the scale rows allow it (decided on the host, compiled as
  // two kernels)
  auto kmain = decode_main<D, KV, QT, ST, NW, false>;
  if constexpr (std::is_same<KV, I8>::value)
    if (L.a.scale_vec) kmain = decode_main<D, KV, QT, ST, NW, true>;
  // The split charges every segment start this many virtual tiles: starting
  // a segment costs about four dependent memory round trips (its length and
  // query, its first page id, its first tile), about two tiles of streaming
  // time for 16-bit K/V and three for int8.  Equal lengths keep their shares
  // aligned to sequence boundaries whatever the charge.
  L.a.seg_pen = std::is_same<KV, I8>::value ? 3 : 2;
  const size_t lds = decode_lds_bytes(D, L.a.G16, L.a.B, NW);
  const int occ = kernel_occupancy((const void*)kmain, NW * 64, lds);
  if (occ <= 0) return fail(SIA_ERR_LAUNCH, "decode kernel does not fit on a CU (LDS %zu B)", lds);
  L.a.slots = device_info().cus * occ;
  // One length for the whole batch and a segment count ((sequence, unit
  // block) pairs) that is a multiple of the persistent grid: the split gives
  // every group whole segments, so decode_main writes every row itself
  // (zeros for a zero length) and decode_reduce is not launched.
  const int64_t nseg = (int64_t)L.a.B * L.a.UB;
  L.a.direct_only = !L.a.kv_per_seq && L.a.tps_force == 0 && nseg >= L.a.slots && nseg % L.a.slots == 0 &&
                    L.a.max_items / 2 >= L.a.slots;
  // 1. main (persistent, stream-K share per group), 2. merge of the split
  // pieces (unless direct_only)
  const int rc = launch_kernel(kmain, dim3(L.a.slots), dim3(NW * 64), lds, L.stream, L.begin_event, L.end_event,
                               "decode", L.a);
  if (rc != SIA_OK || L.a.direct_only) return rc;
  const int rows = L.a.B * L.a.Hq;
  constexpr int kRowsPerGroup = 64 / (D / 4);
  const int ngroups = (rows + kRowsPerGroup - 1) / kRowsPerGroup;
  // rows too few to fill the CUs: 8 waves split each row's pieces
  if (ngroups < device_info().cus)
    hipLaunchKernelGGL((decode_reduce<D, QT, NW, 8>), dim3(ngroups), dim3(8 * 64), 0, L.stream, L.a);
  else
    hipLaunchKernelGGL((decode_reduce<D, QT, NW, 1>), dim3(ngroups), dim3(64), 0, L.stream, L.a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIA_ERR_LAUNCH, "decode reduce launch: %s", hipGetErrorString(e));
  return SIA_OK;
}

// head_dim 256 is compiled in its own unit (decode_d256.hip) with different
// register-allocation flags.
template <class KV, class QT, class ST>
int launch_decode_256(DecodeLaunch& L);

// head_dim 16 and 32 run on a wave-per-row kernel (decode_small.hip).
template <class KV, class QT, class ST>
int launch_decode_small(DecodeLaunch& L);

template <class KV, class QT, class ST>
int launch_decode_d(DecodeLaunch& L) {
  switch (L.D) {
    case 16: case 32: return launch_decode_small<KV, QT, ST>(L);
    case 64: return launch_decode_typed<64, KV, QT, ST>(L);
    case 128: return launch_decode_typed<128, KV, QT, ST>(L);
    case 256: return launch_decode_256<KV, QT, ST>(L);
    default: return fail(SIA_ERR_UNSUPPORTED, "head_dim %d not supported (16, 32, 64, 128, 256)", L.D);
  }
}

template <class KV, class ST>
int launch_decode_q(DecodeLaunch& L) {
  if (L.q_dtype == SIA_F16) return launch_decode_d<KV, F16, ST>(L);
  if (L.q_dtype == SIA_BF16) return launch_decode_d<KV, BF16, ST>(L);
  return fail(SIA_ERR_UNSUPPORTED, "query dtype must be float16 or bfloat16");
}

// Entry points implemented by decode_f16.hip / decode_bf16.hip / decode_i8.hip.
int launch_decode_f16(DecodeLaunch& L);
int launch_decode_bf16(DecodeLaunch& L);
int launch_decode_i8(DecodeLaunch& L);

}  // namespace sia
