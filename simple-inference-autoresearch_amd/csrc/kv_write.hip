// KV write path for gfx950: store new K/V tokens into a contiguous cache or a
// paged pool, quantising to int8 with per-token-per-head scales on the way
// when the destination is int8.
//
// Semantics follow the reference engine:
//  * quantize_kv_int8 (model/kv_cache.py:58-67): amax = max |x| over head_dim,
//    computed in the source dtype and clamped from below by 1e-8 rounded to
//    that dtype; scale = amax / 127 in fp32; xi = round-half-even(x / scale)
//    clamped to [-127, 127]; the scale is stored as fp16 (KVCache) or fp32
//    (paged pools).  Both divisions give torch's correctly rounded results
//    (x / scale through a reciprocal and one FMA correction, div_by_scale).
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
// sources).  Rows are walked in the source's memory order: consecutive
// tokens of one head for a head-major source (a wave's destination slots are
// then one contiguous run), consecutive heads of one token for a token-major
// source (the qkv projection's layout; a wave then reads one contiguous run).  Destinations outside the cache (position past its
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

// N (4 or 8) consecutive table values of dtype C from element j0 of `row`
// (a 16-byte aligned chunk: the host requires aligned tables).
template <class C, int N>
__device__ __forceinline__ void tab_n(const char* row, int j0, float* c) {
  if constexpr (std::is_same<C, F32>::value) {
    const f32x4 a = *(const f32x4*)(row + j0 * 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = a[i];
    if constexpr (N == 8) {
      const f32x4 b = *(const f32x4*)(row + j0 * 4 + 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) c[4 + i] = b[i];
    }
  } else {
    uint32_t w[N / 2];
    if constexpr (N == 8) {
      const u32x4 v = *(const u32x4*)(row + j0 * 2);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = v[i];
    } else {
      const u32x2 v = *(const u32x2*)(row + j0 * 2);
      w[0] = v[0]; w[1] = v[1];
    }
#pragma unroll
    for (int i = 0; i < N / 2; ++i) { c[2 * i] = lo_f32(C{}, w[i]); c[2 * i + 1] = hi_f32(C{}, w[i]); }
  }
}

// Round a float to the source dtype (the rotated row is stored in that dtype
// before it is quantised or cast, as a separate RoPE pass would store it).
template <class S> __device__ __forceinline__ float to_src(float x) { return x; }
template <> __device__ __forceinline__ float to_src<F16>(float x) { return (float)(_Float16)x; }
template <> __device__ __forceinline__ float to_src<BF16>(float x) { return (float)(__bf16)x; }

// Rotate this lane's 8 elements of a K row (lane `part` of the row's `width`
// lanes holds elements [8 part, 8 part + 8)) by table row `pos` (already
// clamped into the table).  Split-half: the partner elements sit in lane
// part ^ width/2 of the same row group; all lanes of a group call this (the
// shuffle needs them).  Products and sums are rounded one by one, in the
// order out_a = x_a c - x_b s, out_b = x_b c + x_a s.
template <class C, int ROPE>
__device__ __forceinline__ void rope8(float (&x)[8], int part, int width, const KvWriteArgs& a, int pos) {
  const char* crow = a.cs + (int64_t)pos * a.tab_rs;
  const char* srow = a.sn + (int64_t)pos * a.tab_rs;
  float c[8], s[8];
  if constexpr (ROPE == 1) {
    const int hw = width >> 1;
    const bool first = part < hw;
    const int j0 = (first ? part : part - hw) * 8;
    tab_n<C, 8>(crow, j0, c);
    tab_n<C, 8>(srow, j0, s);
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = __shfl_xor(x[i], hw);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float oa, ob;
      if (first) rope_rotate(x[i], y[i], c[i], s[i], oa, ob);
      else rope_rotate(y[i], x[i], c[i], s[i], ob, oa);
      x[i] = oa;
    }
  } else {
    tab_n<C, 4>(crow, part * 4, c);
    tab_n<C, 4>(srow, part * 4, s);
#pragma unroll
    for (int j = 0; j < 4; ++j) rope_rotate(x[2 * j], x[2 * j + 1], c[j], s[j], x[2 * j], x[2 * j + 1]);
  }
}

// x / s correctly rounded, from inv = RN(1/s): q0 = RN(x inv) is within one
// ulp of x/s, r = x - q0 s is exact under an FMA, and RN(q0 + r inv) is the
// correctly rounded quotient (Markstein's correction step) while the scale
// stays a normal number, which the amax floor guarantees.  Three VALU
// operations per element instead of a full division; checked against the
// correctly rounded division for every bf16 and fp16 (x, amax) pair and for
// sampled fp32 pairs (tests/test_quant_division.py).
__device__ __forceinline__ float div_by_scale(float x, float s, float inv) {
#pragma clang fp contract(off)
  const float q0 = x * inv;
  const float r = __builtin_fmaf(-q0, s, x);
  return __builtin_fmaf(r, inv, q0);
}

// Max over the `width` lanes of a row group (width = D/8 <= 32, power of two).
__device__ __forceinline__ float group_max(float x, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

// The q part of a RoPE write: one work-group per token (b, t); a work item is
// 8 pairs of one query head, read and written with 16-byte accesses (both
// halves of a split-half pair, or 16 consecutive elements of interleaved
// pairs, in the same thread).  A token whose position lies outside the table
// is written as zeros.  Loads are unconditional (a position outside the
// table reads row 0 and the result is then zeroed), so no branch sits
// between a load and its use.
template <class S, class C, int ROPE>
__device__ __forceinline__ void rope_q_token(const KvWriteArgs& a, uint32_t token) {
  constexpr int ES = S::bytes;
  const uint32_t b = token / (uint32_t)a.T, t = token - b * (uint32_t)a.T;
  const int pos = (int)t + a.start_host + (a.start ? a.start[a.start_per_seq ? b : 0] : 0);
  const bool tab_ok = pos >= 0 && pos < a.Tc;
  const int half = a.D >> 1;
  const int per_head = half >> 3;
  const int items = a.Hq * per_head;
  const char* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)t * a.q_st;
  char* orow = a.qo + (int64_t)b * a.qo_sb + (int64_t)t * a.qo_st;
  const char* crow = a.cs + (int64_t)(tab_ok ? pos : 0) * a.tab_rs;
  const char* srow = a.sn + (int64_t)(tab_ok ? pos : 0) * a.tab_rs;
  for (int it = threadIdx.x; it < items; it += 256) {
    const int h = it / per_head;
    const int i0 = (it - h * per_head) * 8;
    const char* src = qrow + (int64_t)h * a.q_sh;
    char* dst = orow + (int64_t)h * a.qo_sh;
    float c[8], s[8], x0[8], x1[8];
    // split-half: x0 = elements [i0, i0+8), x1 = [i0+half, ...); interleaved: 16 consecutive
    const int o0 = ROPE == 1 ? i0 : 2 * i0;
    const int o1 = ROPE == 1 ? i0 + half : 2 * i0 + 8;
    load8<S>(src + o0 * ES, x0);
    load8<S>(src + o1 * ES, x1);
    tab_n<C, 8>(crow, i0, c);
    tab_n<C, 8>(srow, i0, s);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c[i] = tab_ok ? c[i] : 0.f;
      s[i] = tab_ok ? s[i] : 0.f;
    }
    if constexpr (ROPE == 1) {
#pragma unroll
      for (int i = 0; i < 8; ++i) rope_rotate(x0[i], x1[i], c[i], s[i], x0[i], x1[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) rope_rotate(x0[2 * j], x0[2 * j + 1], c[j], s[j], x0[2 * j], x0[2 * j + 1]);
#pragma unroll
      for (int j = 0; j < 4; ++j) rope_rotate(x1[2 * j], x1[2 * j + 1], c[4 + j], s[4 + j], x1[2 * j], x1[2 * j + 1]);
    }
    store8<S>(dst + o0 * ES, x0);
    store8<S>(dst + o1 * ES, x1);
  }
}

// K/V part: rows are (b, kv head, token).  Loads are unconditional: a row past
// the end (the last work-group's tail) reads the last row, a position outside
// the destination or the table reads table row 0 and page-table entry 0, and
// only the stores are skipped, so no branch sits between a load and its use.
template <class S, class DT, class C, int ROPE>
__global__ __launch_bounds__(256) void kv_write_kernel(const KvWriteArgs a) {
  const int width = a.D >> 3;                                   // lanes per row
  if constexpr (ROPE != 0) {
    if (blockIdx.x >= a.kv_blocks) {                            // whole work-group in the q part
      rope_q_token<S, C, ROPE>(a, blockIdx.x - a.kv_blocks);
      return;
    }
  }
  // 32-bit indexing: the host keeps rows * width below 2^31
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t row_raw = gid >> a.log2_width;
  const int part = (int)(gid & (uint32_t)(width - 1));
  const bool live_row = row_raw < (uint32_t)a.rows;
  const uint32_t row = live_row ? row_raw : (uint32_t)a.rows - 1u;
  uint32_t t, h, b;
  if (a.h_fast) {                       // token-major source: rows (b, t, h), heads fastest
    const uint32_t bt = row / (uint32_t)a.H;
    h = row - bt * (uint32_t)a.H;
    b = bt / (uint32_t)a.T;
    t = bt - b * (uint32_t)a.T;
  } else {                              // rows (b, h, t), tokens fastest
    const uint32_t bh = row / (uint32_t)a.T;
    t = row - bh * (uint32_t)a.T;
    b = bh / (uint32_t)a.H;
    h = bh - b * (uint32_t)a.H;
  }
  const int pos = (int)t + a.start_host + (a.start ? a.start[a.start_per_seq ? b : 0] : 0);
  const bool in_range = live_row && pos >= 0 && pos < a.cap && (ROPE == 0 || pos < a.Tc);
  const int pos_c = in_range ? pos : 0;
  // sources: both rows' loads are issued before either is processed
  const int64_t src_row = (int64_t)b * a.s_sb + (int64_t)h * a.s_sh + (int64_t)t * a.s_st + part * 8 * S::bytes;
  float xs[2][8];
  load8<S>(a.src0 + src_row, xs[0]);
  load8<S>(a.src1 + src_row, xs[1]);                            // src1 == src0 when there is no v
  // destination slot (page-table entry 0 of the row's sequence when out of range)
  int64_t slot0 = b, slot1 = pos_c;
  bool ok = in_range;
  if (a.paged) {
    const int pg = a.bt[(int64_t)b * a.bt_sb + (int64_t)(pos_c / a.page) * a.bt_sl];
    ok = ok && pg >= 0 && (int64_t)pg < a.num_pages;
    slot0 = pg;
    slot1 = pos_c % a.page;
  }
  const int64_t dst_row = slot0 * a.d_s0 + (int64_t)h * a.d_sh + slot1 * a.d_sn;
  const int64_t sc_row = slot0 * a.c_s0 + (int64_t)h * a.c_sh + slot1 * a.c_sn;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    char* dst = which ? a.dst1 : a.dst0;
    char* sdst = which ? a.sc1 : a.sc0;
    const bool store = ok && which < a.ntensors;
    float (&x)[8] = xs[which];
    if constexpr (ROPE != 0) {
      if (which == 0) {                                         // K only
        rope8<C, ROPE>(x, part, width, a, pos_c);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = to_src<S>(x[i]);
      }
    }
    if constexpr (std::is_same<DT, I8>::value) {
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
      m = group_max(m, width);
      const float amax = fmaxf(m, a.amax_floor);
      const float scale = __fdiv_rn(amax, 127.0f);
      const float inv = __fdiv_rn(1.0f, scale);
      uint32_t w0 = 0, w1 = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float q = __builtin_rintf(div_by_scale(x[i], scale, inv));
        // 0 / 0 (an all-zero fp16 row: 1e-8 underflows to a zero scale) is NaN,
        // which torch's float -> int8 conversion turns into 0
        q = q != q ? 0.0f : fminf(fmaxf(q, -127.0f), 127.0f);
        const uint32_t byte = (uint32_t)((int)q) & 0xffu;
        if (i < 4) w0 |= byte << (8 * i);
        else w1 |= byte << (8 * (i - 4));
      }
      if (store) {
        *(u32x2*)(dst + dst_row + (int64_t)part * 8) = u32x2{w0, w1};
        if (part == 0) {
          if (a.scale_f32) *(float*)(sdst + sc_row) = scale;
          else *(_Float16*)(sdst + sc_row) = (_Float16)scale;
        }
      }
    } else {
      if (store) store8<DT>(dst + dst_row + (int64_t)part * 8 * DT::bytes, x);
    }
  }
}

template <class S, class C, int ROPE>
static int launch_dst(const KvWriteArgs& a, int dst_dtype, hipStream_t stream) {
  const int64_t q_blocks = ROPE != 0 && a.q && a.Hq > 0 ? (int64_t)a.B * a.T : 0;   // one per token
  const dim3 grid((unsigned)(a.kv_blocks + q_blocks));
  switch (dst_dtype) {
    case SIA_F16: hipLaunchKernelGGL((kv_write_kernel<S, F16, C, ROPE>), grid, dim3(256), 0, stream, a); break;
    case SIA_BF16: hipLaunchKernelGGL((kv_write_kernel<S, BF16, C, ROPE>), grid, dim3(256), 0, stream, a); break;
    case SIA_F32: hipLaunchKernelGGL((kv_write_kernel<S, F32, C, ROPE>), grid, dim3(256), 0, stream, a); break;
    case SIA_I8: hipLaunchKernelGGL((kv_write_kernel<S, I8, C, ROPE>), grid, dim3(256), 0, stream, a); break;
    default: return fail(SIA_ERR_UNSUPPORTED, "destination dtype %s not supported", dtype_name(dst_dtype));
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIA_ERR_LAUNCH, "kv write launch: %s", hipGetErrorString(e));
  return SIA_OK;
}

template <class S, int ROPE>
static int launch_tab(const KvWriteArgs& a, int dst_dtype, hipStream_t stream) {
  switch (a.tab_dt) {
    case SIA_F16: return launch_dst<S, F16, ROPE>(a, dst_dtype, stream);
    case SIA_BF16: return launch_dst<S, BF16, ROPE>(a, dst_dtype, stream);
    default: return launch_dst<S, F32, ROPE>(a, dst_dtype, stream);
  }
}

template <class S>
static int launch_src(const KvWriteArgs& a, int dst_dtype, hipStream_t stream) {
  switch (a.rope) {
    case 1: return launch_tab<S, 1>(a, dst_dtype, stream);
    case 2: return launch_tab<S, 2>(a, dst_dtype, stream);
    default: return launch_dst<S, F32, 0>(a, dst_dtype, stream);
  }
}

int launch_kv_write(const KvWriteArgs& a_in, int src_dtype, int dst_dtype, hipStream_t stream) {
  KvWriteArgs a = a_in;
  const int width = a.D / 8;
  if (a.rows * width + 255 > 0x7fffffff || (int64_t)a.B * a.T > 0x7fffffff)
    return fail(SIA_ERR_UNSUPPORTED, "too many rows for one launch");
  a.log2_width = __builtin_ctz((unsigned)width);
  // walk rows in the source's memory order: heads fastest when a token's heads
  // sit closer together than a head's tokens (the qkv projection's layout)
  a.h_fast = (a.H > 1 && a.T > 1 && (a.s_sh < 0 ? -a.s_sh : a.s_sh) < (a.s_st < 0 ? -a.s_st : a.s_st)) ? 1 : 0;
  a.kv_blocks = (uint32_t)((a.rows * width + 255) / 256);
  // loads are unconditional: a missing v reads k again (never stored), and a
  // contiguous destination (or an empty block table) points the page-table
  // read at the source row base, which is never used either
  if (a.src1 == nullptr) a.src1 = a.src0;
  a.paged = a.bt != nullptr && a.cap > 0 ? 1 : 0;
  if (!a.paged) { a.bt = (const int32_t*)a.src0; a.bt_sb = 0; a.bt_sl = 0; }
  if (a.rows == 0 && (a.rope == 0 || a.q == nullptr || a.q_rows == 0)) return SIA_OK;
  switch (src_dtype) {
    case SIA_F16: return launch_src<F16>(a, dst_dtype, stream);
    case SIA_BF16: return launch_src<BF16>(a, dst_dtype, stream);
    case SIA_F32: return launch_src<F32>(a, dst_dtype, stream);
    default: return fail(SIA_ERR_UNSUPPORTED, "source dtype %s not supported", dtype_name(src_dtype));
  }
}

}  // namespace sia
