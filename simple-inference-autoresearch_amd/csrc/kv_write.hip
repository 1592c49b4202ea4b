// KV write path for gfx950: store new K/V tokens into a contiguous cache or a
// paged pool, quantising to int8 with per-token-per-head scales on the way
// when the destination is int8.
//
// Semantics follow the reference engine:
//  * quantize_kv_int8 (model/kv_cache.py:58-67): amax = max |x| over head_dim,
//    computed in the source dtype and clamped from below by 1e-8 rounded to
//    that dtype; scale = amax / 127 in fp32; xi = round-half-even(x / scale)
//    clamped to [-127, 127]; the scale is stored as fp16 (KVCache) or fp32
//    (paged pools).  Both divisions are correctly rounded, as torch's are.
//  * KVCache.update (model/kv_cache.py:133-184) writes tokens [start, start+T)
//    of every (b, kv head); the decode step writes one token at a position
//    held in device memory (ops/attention.py:217-228, index_copy_ at
//    ctx.pos_index).
//  * PagedKVCache.write_prefill (model/paged_kv_cache.py:89-109) scatters
//    token t of sequence b to block_table[b][t / page] at offset t % page; the
//    same rule serves the per-step decode write the reference leaves
//    unimplemented (slot_for, model/paged_kv_cache.py:29-30), with the start
//    position read per sequence on the device.
//
// Layout: a row is one (b, kv head, token) vector of head_dim elements; D/8
// lanes own a row, 8 consecutive elements each (one 16-byte load for 16-bit
// sources), so a wave covers 64 / (D/8) consecutive tokens of one head and
// both the source rows and the destination slots are read and written as
// contiguous runs.  Destinations outside the cache (position past its
// capacity, page id outside the pool) are skipped: the kernel never writes
// outside the buffers it was given.
#include "host_util.hpp"
#include "kv_write.hpp"
#include "sia_common.hpp"

namespace sia {

template <class T>
__device__ __forceinline__ void load8(const char* p, float* x);
template <>
__device__ __forceinline__ void load8<F16>(const char* p, float* x) {
  const u32x4 w = *(const u32x4*)p;
#pragma unroll
  for (int i = 0; i < 4; ++i) { x[2 * i] = lo_f32(F16{}, w[i]); x[2 * i + 1] = hi_f32(F16{}, w[i]); }
}
template <>
__device__ __forceinline__ void load8<BF16>(const char* p, float* x) {
  const u32x4 w = *(const u32x4*)p;
#pragma unroll
  for (int i = 0; i < 4; ++i) { x[2 * i] = lo_f32(BF16{}, w[i]); x[2 * i + 1] = hi_f32(BF16{}, w[i]); }
}
template <>
__device__ __forceinline__ void load8<F32>(const char* p, float* x) {
  const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 16);
#pragma unroll
  for (int i = 0; i < 4; ++i) { x[i] = a[i]; x[4 + i] = b[i]; }
}

template <class T>
__device__ __forceinline__ void store8(char* p, const float* x);
template <>
__device__ __forceinline__ void store8<F16>(char* p, const float* x) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack2(F16{}, x[2 * i], x[2 * i + 1]);
  *(u32x4*)p = w;
}
template <>
__device__ __forceinline__ void store8<BF16>(char* p, const float* x) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack2(BF16{}, x[2 * i], x[2 * i + 1]);
  *(u32x4*)p = w;
}
template <>
__device__ __forceinline__ void store8<F32>(char* p, const float* x) {
  *(f32x4*)p = f32x4{x[0], x[1], x[2], x[3]};
  *(f32x4*)(p + 16) = f32x4{x[4], x[5], x[6], x[7]};
}

// Max over the `width` lanes of a row group (width = D/8 <= 32, power of two).
__device__ __forceinline__ float group_max(float x, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

template <class S, class DT>
__global__ __launch_bounds__(256) void kv_write_kernel(const KvWriteArgs a) {
  const int width = a.D / 8;                                    // lanes per row
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / width;
  const int part = (int)(gid - row * width);
  // rows are (b, h, t) with t fastest; rows past the end idle but still take
  // part in their group's shuffles (all lanes of a group share `row`)
  const bool live_row = row < a.rows;
  int t = 0, h = 0, b = 0;
  if (live_row) {
    t = (int)(row % a.T);
    const int64_t bh = row / a.T;
    h = (int)(bh % a.H);
    b = (int)(bh / a.H);
  }
  const int pos = t + a.start_host + (a.start ? a.start[a.start_per_seq ? b : 0] : 0);
  bool ok = live_row && pos >= 0 && pos < a.cap;
  int64_t dst_row = 0, sc_row = 0;
  if (ok) {
    int64_t slot0 = b, slot1 = pos;                             // (page or batch row, position inside it)
    if (a.bt) {
      const int pg = a.bt[(int64_t)b * a.bt_sb + (int64_t)(pos / a.page) * a.bt_sl];
      ok = pg >= 0 && (int64_t)pg < a.num_pages;
      slot0 = pg;
      slot1 = pos % a.page;
    }
    dst_row = slot0 * a.d_s0 + (int64_t)h * a.d_sh + slot1 * a.d_sn;
    sc_row = slot0 * a.c_s0 + (int64_t)h * a.c_sh + slot1 * a.c_sn;
  }
  const int64_t src_row = (int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)t * a.s_st;
  for (int which = 0; which < a.ntensors; ++which) {
    const char* src = which ? a.src1 : a.src0;
    char* dst = which ? a.dst1 : a.dst0;
    char* sdst = which ? a.sc1 : a.sc0;
    float x[8];
    if (live_row) load8<S>(src + src_row + (int64_t)part * 8 * S::bytes, x);
    else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = 0.f;
    }
    if constexpr (std::is_same<DT, I8>::value) {
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
      m = group_max(m, width);
      const float amax = fmaxf(m, a.amax_floor);
      const float scale = __fdiv_rn(amax, 127.0f);
      uint32_t w0 = 0, w1 = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float q = __builtin_rintf(__fdiv_rn(x[i], scale));
        // 0 / 0 (an all-zero fp16 row: 1e-8 underflows to a zero scale) is NaN,
        // which torch's float -> int8 conversion turns into 0
        q = q != q ? 0.0f : fminf(fmaxf(q, -127.0f), 127.0f);
        const uint32_t byte = (uint32_t)((int)q) & 0xffu;
        if (i < 4) w0 |= byte << (8 * i);
        else w1 |= byte << (8 * (i - 4));
      }
      if (ok) {
        *(u32x2*)(dst + dst_row + (int64_t)part * 8) = u32x2{w0, w1};
        if (part == 0) {
          if (a.scale_f32) *(float*)(sdst + sc_row) = scale;
          else *(_Float16*)(sdst + sc_row) = (_Float16)scale;
        }
      }
    } else {
      if (ok) store8<DT>(dst + dst_row + (int64_t)part * 8 * DT::bytes, x);
    }
  }
}

template <class S>
static int launch_src(const KvWriteArgs& a, int dst_dtype, hipStream_t stream) {
  const int64_t threads = a.rows * (a.D / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  switch (dst_dtype) {
    case SIA_F16: hipLaunchKernelGGL((kv_write_kernel<S, F16>), grid, dim3(256), 0, stream, a); break;
    case SIA_BF16: hipLaunchKernelGGL((kv_write_kernel<S, BF16>), grid, dim3(256), 0, stream, a); break;
    case SIA_F32: hipLaunchKernelGGL((kv_write_kernel<S, F32>), grid, dim3(256), 0, stream, a); break;
    case SIA_I8: hipLaunchKernelGGL((kv_write_kernel<S, I8>), grid, dim3(256), 0, stream, a); break;
    default: return fail(SIA_ERR_UNSUPPORTED, "destination dtype %s not supported", dtype_name(dst_dtype));
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIA_ERR_LAUNCH, "kv write launch: %s", hipGetErrorString(e));
  return SIA_OK;
}

int launch_kv_write(const KvWriteArgs& a, int src_dtype, int dst_dtype, hipStream_t stream) {
  if (a.rows == 0) return SIA_OK;
  switch (src_dtype) {
    case SIA_F16: return launch_src<F16>(a, dst_dtype, stream);
    case SIA_BF16: return launch_src<BF16>(a, dst_dtype, stream);
    case SIA_F32: return launch_src<F32>(a, dst_dtype, stream);
    default: return fail(SIA_ERR_UNSUPPORTED, "source dtype %s not supported", dtype_name(src_dtype));
  }
}

}  // namespace sia
