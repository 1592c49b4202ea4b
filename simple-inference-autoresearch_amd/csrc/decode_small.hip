// Decode for head_dim 16 and 32 (the small head dims of the reference's
// assert set, kernels/flash_decode_kernel.py:142 and friends).
//
// The MFMA decode kernel (decode_kernel.hpp) tiles 16 tokens x head_dim with
// at least four bytes per lane per token, which head_dim 16/32 cannot fill.
// Here one wave serves one (sequence, query head): lanes stride over the
// tokens, each keeping its own online-softmax state (m, l, acc[D]) in fp32,
// and the 64 states are merged with wave shuffles at the end.  Semantics are
// the same as every other decode entry point: contiguous or paged K/V
// (block-table indirection, kernels/paged_flash_decode_kernel.py:74-84),
// fp16/bf16 or int8 K/V with per-token scales folded as qk * s_k and
// p * s_v (kernels/flash_decode_int8_kernel.py:98,111-112), kv_len shared or
// per sequence, an empty prefix giving zeros.
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
__global__ __launch_bounds__(256) void decode_small(const DecodeArgs a) {
  static_assert(D == 16 || D == 32, "small head dims only");
  constexpr bool kInt8 = std::is_same<KV, I8>::value;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);   // (b, hq)
  const int lane = threadIdx.x & 63;
  if (row >= a.B * a.Hq) return;                            // whole waves leave together
  const int b = row / a.Hq, hq = row - b * a.Hq, hkv = hq / a.G;
  float q[D];
  load_row<QT>(a.q + b * a.q_sb + (int64_t)hq * a.q_sh, q, D);
  const int n = seq_tokens(a, b);
  const bool paged = a.bt != nullptr;
  const int page = kTile << a.lg_tiles_per_page;
  float m = -INFINITY, l = 0.f, acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) acc[d] = 0.f;
  for (int t = lane; t < n; t += 64) {
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
  if (lane < D) {
    const float inv = 1.0f / (l == 0.f ? 1.f : l);
    store_out(QT{}, a.out + b * a.o_sb + (int64_t)hq * a.o_sh + lane * (int)sizeof(uint16_t), mine * inv);
  }
}

template <class KV, class QT, class ST>
int launch_decode_small(DecodeLaunch& L) {
  const int rows = L.a.B * L.a.Hq;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (L.begin_event && hipEventRecord(L.begin_event, L.stream) != hipSuccess)
    return fail(SIA_ERR_LAUNCH, "cannot record main_begin_event");
  if (L.D == 16) hipLaunchKernelGGL((decode_small<16, KV, QT, ST>), grid, dim3(256), 0, L.stream, L.a);
  else hipLaunchKernelGGL((decode_small<32, KV, QT, ST>), grid, dim3(256), 0, L.stream, L.a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIA_ERR_LAUNCH, "small decode launch: %s", hipGetErrorString(e));
  if (L.end_event && hipEventRecord(L.end_event, L.stream) != hipSuccess)
    return fail(SIA_ERR_LAUNCH, "cannot record main_end_event");
  return SIA_OK;
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
