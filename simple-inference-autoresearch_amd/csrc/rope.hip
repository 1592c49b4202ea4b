// Rotary position embedding of Q and K in one launch, for gfx950.
//
// Semantics follow the reference kernel kernels/rope_kernel.py:86-165
// (_rope_qk_fwd) and its wrapper _apply_qk / rope_triton (193-285):
//  * q (B, T, Hq, D) and k (B, T, Hkv, D) are read through a flattened row
//    stride (row = b*T + t), so Q/K slices of a fused qkv buffer are rotated
//    without a copy; the outputs are contiguous (B, T, H, D).
//  * the position of row r is r % Tc, Tc = the number of cos/sin rows; only
//    the first D/2 columns of a cos/sin row are read (a duplicated width-D
//    table and a raw width-D/2 table give the same result).
//  * pair (a, b) is (i, i + D/2) (split-half, Llama/NeoX) or (2i, 2i + 1)
//    (interleaved, GPT-J); out_a = x_a cos - x_b sin, out_b = x_b cos + x_a sin
//    in fp32, stored in the input dtype with round-to-nearest-even.  Each
//    product and the sum are rounded separately (no fused multiply-add), so
//    the result is a fixed function of the inputs.
//
// Work decomposition: one work-group per row, sized to the row's work items
// (whole waves, at most 1024 threads); a work item is a chunk of 8 pairs of
// one head (16 contiguous bytes of each half for 16-bit split-half data).
// Head dims whose half is not a multiple of 8, or rows that are not 16-byte
// aligned, take a one-pair-per-item path.  Memory-bound: x and out once;
// cos/sin once per row from HBM, the other heads' reads hit in L2.
#include <string.h>

#include <algorithm>

#include "host_util.hpp"
#include "sia_common.hpp"

namespace sia {

struct RopeArgs {
  const char* q; const char* k;      // inputs
  int64_t q_rs, k_rs;                // input row strides (bytes)
  char* qo; char* ko;                // outputs, contiguous
  const char* cs; const char* sn;    // cos / sin tables
  int64_t c_rs;                      // their row stride (bytes)
  int32_t rows, Tc, Hq, Hkv, D;
  int32_t block;                     // threads per work-group (multiple of 64, <= 1024)
};

template <class T> __device__ __forceinline__ float ld1(const char* p);
template <> __device__ __forceinline__ float ld1<F16>(const char* p) { return (float)*(const _Float16*)p; }
template <> __device__ __forceinline__ float ld1<BF16>(const char* p) { return (float)*(const __bf16*)p; }
template <> __device__ __forceinline__ float ld1<F32>(const char* p) { return *(const float*)p; }

template <class T> __device__ __forceinline__ void st1(char* p, float x);
template <> __device__ __forceinline__ void st1<F16>(char* p, float x) { *(_Float16*)p = (_Float16)x; }
template <> __device__ __forceinline__ void st1<BF16>(char* p, float x) { *(__bf16*)p = (__bf16)x; }
template <> __device__ __forceinline__ void st1<F32>(char* p, float x) { *(float*)p = x; }

template <class T> struct Sz { static constexpr int v = 2; };
template <> struct Sz<F32> { static constexpr int v = 4; };

// 8 consecutive elements at p (16-byte aligned for 16-bit types, 32 for fp32)
template <class T>
__device__ __forceinline__ void ld8(const char* p, float* x) {
  if constexpr (std::is_same<T, F32>::value) {
    const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[i] = a[i]; x[4 + i] = b[i]; }
  } else {
    const u32x4 w = *(const u32x4*)p;
#pragma unroll
    for (int i = 0; i < 4; ++i) { x[2 * i] = lo_f32(T{}, w[i]); x[2 * i + 1] = hi_f32(T{}, w[i]); }
  }
}
template <class T>
__device__ __forceinline__ void st8(char* p, const float* x) {
  if constexpr (std::is_same<T, F32>::value) {
    *(f32x4*)p = f32x4{x[0], x[1], x[2], x[3]};
    *(f32x4*)(p + 16) = f32x4{x[4], x[5], x[6], x[7]};
  } else {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack2(T{}, x[2 * i], x[2 * i + 1]);
    *(u32x4*)p = w;
  }
}

// VEC: 8 pairs per work item (16-byte accesses); otherwise one pair.
template <class T, class C, bool IL, bool VEC>
__global__ __launch_bounds__(1024) void rope_qk_kernel(const RopeArgs a) {
  constexpr int ES = Sz<T>::v, CS = Sz<C>::v;
  constexpr int PP = VEC ? 8 : 1;                 // pairs per item
  const int row = blockIdx.x;
  const int half = a.D / 2;
  const int per_head = half / PP;
  const int items = (a.Hq + a.Hkv) * per_head;
  const char* crow = a.cs + (int64_t)(row % a.Tc) * a.c_rs;
  const char* srow = a.sn + (int64_t)(row % a.Tc) * a.c_rs;
  for (int it = threadIdx.x; it < items; it += blockDim.x) {
    const int h = it / per_head;
    const int i0 = (it - h * per_head) * PP;      // first pair of the item
    const bool isq = h < a.Hq;
    const int hh = isq ? h : h - a.Hq;
    const char* src = (isq ? a.q + (int64_t)row * a.q_rs : a.k + (int64_t)row * a.k_rs) + (int64_t)hh * a.D * ES;
    char* dst = (isq ? a.qo + ((int64_t)row * a.Hq + hh) * a.D * ES : a.ko + ((int64_t)row * a.Hkv + hh) * a.D * ES);
    float c[PP], s[PP];
    if constexpr (VEC) {
      ld8<C>(crow + i0 * CS, c);
      ld8<C>(srow + i0 * CS, s);
    } else {
      c[0] = ld1<C>(crow + i0 * CS);
      s[0] = ld1<C>(srow + i0 * CS);
    }
    if constexpr (IL) {
      // pairs (2i, 2i+1): 2*PP consecutive elements
      float x[2 * PP], o[2 * PP];
      if constexpr (VEC) {
        ld8<T>(src + 2 * i0 * ES, x);
        ld8<T>(src + (2 * i0 + 8) * ES, x + 8);
      } else {
        x[0] = ld1<T>(src + 2 * i0 * ES);
        x[1] = ld1<T>(src + (2 * i0 + 1) * ES);
      }
#pragma unroll
      for (int p = 0; p < PP; ++p) rope_rotate(x[2 * p], x[2 * p + 1], c[p], s[p], o[2 * p], o[2 * p + 1]);
      if constexpr (VEC) {
        st8<T>(dst + 2 * i0 * ES, o);
        st8<T>(dst + (2 * i0 + 8) * ES, o + 8);
      } else {
        st1<T>(dst + 2 * i0 * ES, o[0]);
        st1<T>(dst + (2 * i0 + 1) * ES, o[1]);
      }
    } else {
      // pairs (i, i + D/2)
      float xa[PP], xb[PP], oa[PP], ob[PP];
      if constexpr (VEC) {
        ld8<T>(src + i0 * ES, xa);
        ld8<T>(src + (i0 + half) * ES, xb);
      } else {
        xa[0] = ld1<T>(src + i0 * ES);
        xb[0] = ld1<T>(src + (i0 + half) * ES);
      }
#pragma unroll
      for (int p = 0; p < PP; ++p) rope_rotate(xa[p], xb[p], c[p], s[p], oa[p], ob[p]);
      if constexpr (VEC) {
        st8<T>(dst + i0 * ES, oa);
        st8<T>(dst + (i0 + half) * ES, ob);
      } else {
        st1<T>(dst + i0 * ES, oa[0]);
        st1<T>(dst + (i0 + half) * ES, ob[0]);
      }
    }
  }
}

namespace {

template <class T, class C>
int launch_rope_tc(const RopeArgs& a, bool il, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)a.rows), block((unsigned)a.block);
  if (il) {
    if (vec) hipLaunchKernelGGL((rope_qk_kernel<T, C, true, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((rope_qk_kernel<T, C, true, false>), grid, block, 0, st, a);
  } else {
    if (vec) hipLaunchKernelGGL((rope_qk_kernel<T, C, false, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((rope_qk_kernel<T, C, false, false>), grid, block, 0, st, a);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SIA_OK : fail(SIA_ERR_LAUNCH, "rope launch: %s", hipGetErrorString(e));
}

template <class T>
int launch_rope_t(const RopeArgs& a, int cdt, bool il, bool vec, hipStream_t st) {
  if (cdt == SIA_F32) return launch_rope_tc<T, F32>(a, il, vec, st);
  if (cdt == SIA_F16) return launch_rope_tc<T, F16>(a, il, vec, st);
  return launch_rope_tc<T, BF16>(a, il, vec, st);
}

bool float_dtype(int d) { return d == SIA_F16 || d == SIA_BF16 || d == SIA_F32; }

// Row stride (elements) of a (B, T, H, D) view read as B*T rows of H*D
// elements: head_dim unit-stride, heads D apart, and either T == 1, B == 1
// or a uniform flattened-row stride.  The stride of a size-1 dim is never
// used.  -1 when the view has no such stride.
int64_t row_stride(const sia_tensor* x, int64_t T, int64_t D) {
  if (x->stride[3] != 1 || (x->shape[2] > 1 && x->stride[2] != D)) return -1;
  if (T == 1) return x->stride[0];
  if (x->shape[0] == 1 || x->stride[0] == T * x->stride[1]) return x->stride[1];
  return -1;
}

// (B, T, H, D) laid out densely in that order (size-1 dims' strides ignored;
// an empty tensor qualifies)
bool dense(const sia_tensor* x) {
  for (int d = 0; d < 4; ++d)
    if (x->shape[d] == 0) return true;  // no element is addressed
  int64_t want = 1;
  for (int d = 3; d >= 0; --d) {
    if (x->shape[d] > 1 && x->stride[d] != want) return false;
    want *= x->shape[d];
  }
  return true;
}

}  // namespace
}  // namespace sia

using namespace sia;

extern "C" int sia_rope_qk(const sia_tensor* q, const sia_tensor* k, const sia_tensor* cos, const sia_tensor* sin,
                           int32_t interleaved, const sia_tensor* q_out, const sia_tensor* k_out, void* stream) {
  if (q == nullptr || k == nullptr || cos == nullptr || sin == nullptr || q_out == nullptr || k_out == nullptr)
    return fail(SIA_ERR_INVALID_ARGUMENT, "q, k, cos, sin, q_out and k_out are required");
  const sia_tensor* all[6] = {q, k, cos, sin, q_out, k_out};
  if (q->ndim != 4 || k->ndim != 4 || q_out->ndim != 4 || k_out->ndim != 4)
    return fail(SIA_ERR_INVALID_ARGUMENT, "q, k, q_out, k_out must be (B, T, H, D)");
  if (cos->ndim != 2 || sin->ndim != 2) return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must be (rows, width)");
  const int64_t B = q->shape[0], T = q->shape[1], Hq = q->shape[2], D = q->shape[3], Hkv = k->shape[2];
  if (D <= 0 || D % 2) return fail(SIA_ERR_INVALID_ARGUMENT, "head_dim must be even for RoPE");
  if (k->shape[0] != B || k->shape[1] != T || k->shape[3] != D)
    return fail(SIA_ERR_INVALID_ARGUMENT, "k must be (B, T, Hkv, D) with q's B, T and D");
  if (k->dtype != q->dtype) return fail(SIA_ERR_INVALID_ARGUMENT, "q and k dtypes differ");
  if (!float_dtype(q->dtype)) return fail(SIA_ERR_UNSUPPORTED, "q/k dtype %s not supported", dtype_name(q->dtype));
  const int64_t half = D / 2;
  if (cos->shape[1] != D && cos->shape[1] != half)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin last dim must be head_dim (%lld) or head_dim/2 (%lld)",
                (long long)D, (long long)half);
  if (cos->shape[0] != sin->shape[0] || cos->shape[1] != sin->shape[1])
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must have identical shape");
  if (cos->dtype != sin->dtype || !float_dtype(cos->dtype))
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must share a float dtype");
  if (cos->stride[1] != 1 || sin->stride[1] != 1)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin must be unit-stride along the last dim");
  if (cos->stride[0] != sin->stride[0]) return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must share the same row stride");
  if (cos->shape[0] <= 0) return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin have no rows");
  const int64_t q_rs = row_stride(q, T, D), k_rs = row_stride(k, T, D);
  if (q_rs < 0 || k_rs < 0)
    return fail(SIA_ERR_INVALID_ARGUMENT, "q/k rows must be flattenable: head_dim unit-stride, heads head_dim apart, "
                                          "and stride(0) == T*stride(1) (copy the view first)");
  for (const sia_tensor* o : {q_out, k_out}) {
    const sia_tensor* src = o == q_out ? q : k;
    if (o->dtype != q->dtype) return fail(SIA_ERR_INVALID_ARGUMENT, "outputs must have the inputs' dtype");
    for (int d = 0; d < 4; ++d)
      if (o->shape[d] != src->shape[d]) return fail(SIA_ERR_INVALID_ARGUMENT, "output shape differs from its input");
    if (!dense(o)) return fail(SIA_ERR_INVALID_ARGUMENT, "q_out/k_out must be contiguous");
  }
  if (B * T > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "too many rows");
  if (B * T == 0 || Hq + Hkv == 0) return SIA_OK;
  // empty tensors may carry a null pointer; every tensor read or written must not
  if (cos->data == nullptr || sin->data == nullptr || (Hq > 0 && (q->data == nullptr || q_out->data == nullptr)) ||
      (Hkv > 0 && (k->data == nullptr || k_out->data == nullptr)))
    return fail(SIA_ERR_INVALID_ARGUMENT, "a non-empty tensor has no data pointer");
  const int es = elem_size(q->dtype), cs = elem_size(cos->dtype);
  RopeArgs a;
  memset(&a, 0, sizeof(a));
  a.q = (const char*)q->data; a.k = (const char*)k->data;
  a.q_rs = q_rs * es; a.k_rs = k_rs * es;
  a.qo = (char*)q_out->data; a.ko = (char*)k_out->data;
  a.cs = (const char*)cos->data; a.sn = (const char*)sin->data;
  a.c_rs = cos->stride[0] * cs;
  a.rows = (int32_t)(B * T); a.Tc = (int32_t)cos->shape[0];
  a.Hq = (int32_t)Hq; a.Hkv = (int32_t)Hkv; a.D = (int32_t)D;
  // 8-pair items need 16-byte aligned halves/chunks everywhere
  const int64_t chunk = 8 * es * (interleaved ? 2 : 1);
  bool vec = half % 8 == 0 && (half * es) % 16 == 0 && (8 * cs) % 16 == 0;
  for (const sia_tensor* t : all) vec = vec && (t->data == nullptr || aligned16(t->data));
  vec = vec && a.q_rs % 16 == 0 && a.k_rs % 16 == 0 && a.c_rs % 16 == 0 && (D * es) % 16 == 0 && chunk % 16 == 0;
  // one work-group per row, sized to the row's work items (whole waves, at most 1024 threads)
  const int64_t items = (Hq + Hkv) * (half / (vec ? 8 : 1));
  if (items > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "too many heads");
  a.block = (int32_t)std::min<int64_t>(1024, (items + 63) / 64 * 64);
  int rc;
  if ((rc = device_ok())) return rc;
  const hipStream_t st = (hipStream_t)stream;
  switch (q->dtype) {
    case SIA_F16: return launch_rope_t<F16>(a, cos->dtype, interleaved != 0, vec, st);
    case SIA_BF16: return launch_rope_t<BF16>(a, cos->dtype, interleaved != 0, vec, st);
    default: return launch_rope_t<F32>(a, cos->dtype, interleaved != 0, vec, st);
  }
}
