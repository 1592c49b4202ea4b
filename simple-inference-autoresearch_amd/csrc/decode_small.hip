// Decode for head_dim 16 and 32 (the small head dims of the reference's
// assert set, kernels/flash_decode_kernel.py:142 and friends).
//
// The MFMA decode kernel (decode_kernel.hpp) tiles 16 tokens x head_dim with
// at least four bytes per lane per token, which head_dim 16/32 cannot fill.
// Here one wave serves one (sequence, query head, piece of the context): lanes
// stride over the piece's tokens, each keeping its own online-softmax state
// (m, l, acc[D]) in fp32, and the 64 states are merged with wave shuffles.
// When there are too few (sequence, head) rows to fill the GPU the context is
// cut into pieces of `tps` tokens, each piece writes an fp32 partial (acc, m,
// l) to the workspace, and attn_f32_merge combines them.  Semantics are
// the same as every other decode entry point: contiguous or paged K/V
// (block-table indirection, kernels/paged_flash_decode_kernel.py:74-84),
// fp16/bf16 or int8 K/V with per-token scales folded as qk * s_k and
// p * s_v (kernels/flash_decode_int8_kernel.py:98,111-112), kv_len shared or
// per sequence, an empty prefix giving zeros.
#include <string.h>

#include <algorithm>

#include "attn_f32.hpp"
#include "decode_launch.hpp"

namespace sia {

template <class T>
__device__ __forceinline__ void load_row(const char* p, float* x, int n);
template <>
__device__ __forceinline__ void load_row<F16>(const char* p, float* x, int n) {
  for (int c = 0; c < n / 8; ++c) {
    const u32x4 w = *(const u32x4*)(p + 16 * c);
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[8 * c + 2 * i] = lo_f32(F16{}, w[i]); x[8 * c + 2 * i + 1] = hi_f32(F16{}, w[i]); }
  }
}
template <>
__device__ __forceinline__ void load_row<BF16>(const char* p, float* x, int n) {
  for (int c = 0; c < n / 8; ++c) {
    const u32x4 w = *(const u32x4*)(p + 16 * c);
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[8 * c + 2 * i] = lo_f32(BF16{}, w[i]); x[8 * c + 2 * i + 1] = hi_f32(BF16{}, w[i]); }
  }
}
template <>
__device__ __forceinline__ void load_row<I8>(const char* p, float* x, int n) {
  for (int c = 0; c < n / 16; ++c) {
    const u32x4 w = *(const u32x4*)(p + 16 * c);
#pragma unroll
    for (int i = 0; i < 16; ++i) x[16 * c + i] = (float)(int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xffu);
  }
}

template <int D, class KV, class QT, class ST>
__global__ __launch_bounds__(256) void decode_small(const DecodeArgs a, const int nsplit, const int tps,
                                                   float* const part) {
  static_assert(D == 16 || D == 32, "small head dims only");
  constexpr bool kInt8 = std::is_same<KV, I8>::value;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);  // (b, hq, piece), pieces fastest
  const int lane = threadIdx.x & 63;
  if (item >= a.B * a.Hq * nsplit) return;                 // whole waves leave together
  const int row = item / nsplit, piece = item - row * nsplit;
  const int b = row / a.Hq, hq = row - b * a.Hq, hkv = hq / a.G;
  float q[D];
  load_row<QT>(a.q + b * a.q_sb + (int64_t)hq * a.q_sh, q, D);
  const int n = seq_tokens(a, b);
  const int t_lo = piece * tps, t_hi = min(n, t_lo + tps);   // this wave's tokens
  const bool paged = a.bt != nullptr;
  const int page = kTile << a.lg_tiles_per_page;
  float m = -INFINITY, l = 0.f, acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) acc[d] = 0.f;
  for (int t = t_lo + lane; t < t_hi; t += 64) {
    int64_t base = 0;
    int pos = t;
    if (paged) {
      const int pg = a.bt[(int64_t)b * a.bt_sb + (int64_t)(t / page) * a.bt_sl];
      if ((unsigned)pg >= (unsigned long long)a.num_pages) continue;   // never read outside the pool
      base = pg;
      pos = t % page;
    } else {
      base = b;
    }
    float k[D], v[D];
    load_row<KV>(a.k + base * a.k_s0 + (int64_t)hkv * a.k_sh + (int64_t)pos * a.k_sn, k, D);
    load_row<KV>(a.v + base * a.v_s0 + (int64_t)hkv * a.v_sh + (int64_t)pos * a.v_sn, v, D);
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < D; ++d) s = __builtin_fmaf(q[d], k[d], s);
    float sv = 1.0f;
    if constexpr (kInt8) {
      s *= load_scale<ST>(a.ks + base * a.ks_s0 + (int64_t)hkv * a.ks_sh + (int64_t)pos * a.ks_sn);
      sv = load_scale<ST>(a.vs + base * a.vs_s0 + (int64_t)hkv * a.vs_sh + (int64_t)pos * a.vs_sn);
    }
    s *= a.qk_scale;                                         // log2 units
    const float m_new = fmaxf(m, s);
    const float alpha = fast_exp2(m - m_new);               // 0 on the first key (m = -inf)
    const float p = fast_exp2(s - m_new);
    l = l * alpha + p;
    const float pv = p * sv;
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = acc[d] * alpha + pv * v[d];
    m = m_new;
  }
  // merge the 64 lane states
  float M = m;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
  const float f = m == -INFINITY ? 0.f : fast_exp2(m - M);
  l *= f;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
  float mine = 0.f;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    float x = acc[d] * f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    if (lane == d) mine = x;
  }
  if (nsplit == 1) {
    if (lane < D) {
      const float inv = 1.0f / (l == 0.f ? 1.f : l);
      store_out(QT{}, a.out + b * a.o_sb + (int64_t)hq * a.o_sh + lane * (int)sizeof(uint16_t), mine * inv);
    }
  } else {
    // partial (acc[D], M, l) of this piece, relative to its max M (-inf: no key)
    float* dst = part + (int64_t)item * (D + 4);
    if (lane < D) dst[lane] = mine;
    if (lane == D) dst[D] = M;
    if (lane == D + 1) dst[D + 1] = l;
  }
}

template <class KV, class QT, class ST>
int launch_decode_small(DecodeLaunch& L) {
  const int64_t rows = (int64_t)L.a.B * L.a.Hq;
  // Pieces per row: enough waves for two per SIMD when the rows alone are
  // fewer, pieces of at least 256 tokens (4 per lane), and partials that fit
  // the caller's workspace (the lengths stay on the device: the cut is made
  // from the cache capacity, so one captured graph serves every length).
  const int64_t cap = L.a.cap_tokens > 0 ? L.a.cap_tokens : 1;
  const int cus = device_info().cus > 0 ? device_info().cus : 256;
  int64_t nsplit = (8LL * cus + rows - 1) / rows;
  nsplit = std::min<int64_t>(nsplit, (cap + 255) / 256);
  const int64_t room = (int64_t)(L.ws_bytes / f32_partial_bytes(rows, 1, L.D));
  nsplit = std::max<int64_t>(1, std::min<int64_t>(nsplit, room));
  int64_t tps = (cap + nsplit - 1) / nsplit;
  tps = (tps + 63) / 64 * 64;
  nsplit = (cap + tps - 1) / tps;
  if (rows * nsplit > 0x7fffffff || tps > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "too many decode rows");
  const int64_t waves = rows * nsplit;
  const dim3 grid((unsigned)((waves + 3) / 4));
  float* part = (float*)L.ws;
  const int rc = L.D == 16 ? launch_kernel(decode_small<16, KV, QT, ST>, grid, dim3(256), 0, L.stream, L.begin_event,
                                           L.end_event, "small decode", L.a, (int)nsplit, (int)tps, part)
                           : launch_kernel(decode_small<32, KV, QT, ST>, grid, dim3(256), 0, L.stream, L.begin_event,
                                           L.end_event, "small decode", L.a, (int)nsplit, (int)tps, part);
  if (rc != SIA_OK) return rc;
  if (nsplit == 1) return SIA_OK;
  F32Args m;
  memset(&m, 0, sizeof(m));
  m.B = L.a.B; m.Hq = L.a.Hq; m.Tq = 1;
  m.nsplit = (int)nsplit;
  m.part = part;
  m.out = L.a.out; m.o_sb = L.a.o_sb; m.o_sh = L.a.o_sh; m.o_sm = 0;
  return launch_attn_merge(m, L.D, L.q_dtype, L.stream);
}

#define SIA_SMALL(KV, QT, ST) template int launch_decode_small<KV, QT, ST>(DecodeLaunch&);
SIA_SMALL(F16, F16, F32)
SIA_SMALL(F16, BF16, F32)
SIA_SMALL(BF16, F16, F32)
SIA_SMALL(BF16, BF16, F32)
SIA_SMALL(I8, F16, F32)
SIA_SMALL(I8, BF16, F32)
SIA_SMALL(I8, F16, F16)
SIA_SMALL(I8, BF16, F16)
#undef SIA_SMALL

}  // namespace sia
