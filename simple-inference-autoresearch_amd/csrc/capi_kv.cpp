// extern "C" KV write-path entry points: validation and dispatch of kv_write.hip.
#include <math.h>
#include <string.h>

#include "host_util.hpp"
#include "kv_write.hpp"

using namespace sia;

namespace {

// 1e-8 rounded to `dtype` the way torch's clamp_min(1e-8) rounds it (the
// clamp runs in fp32, its result is stored in the tensor's dtype).
float amax_floor(int dtype) {
  const float f = 1e-8f;
  if (dtype == SIA_BF16) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;   // round to nearest even
    float r;
    memcpy(&r, &u, 4);
    return r;
  }
  if (dtype == SIA_F16) return (float)(_Float16)f;
  return f;
}

bool src_dtype_ok(int d) { return d == SIA_F16 || d == SIA_BF16 || d == SIA_F32; }

int check_rows(const sia_tensor* t, const char* name, int align) {
  if (t == nullptr || t->data == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "%s is missing", name);
  if (t->ndim != 4) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must have 4 dims", name);
  if (t->stride[3] != 1) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must be contiguous along head_dim", name);
  if ((uintptr_t)t->data % align) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must be %d-byte aligned", name, align);
  for (int d = 0; d < 3; ++d)
    if (t->shape[d] > 1 && bstride(t, d) % align)
      return fail(SIA_ERR_INVALID_ARGUMENT, "%s strides must be multiples of %d bytes", name, align);
  return SIA_OK;
}

int check_scale(const sia_tensor* s, const sia_tensor* like, const char* name) {
  if (s == nullptr || s->data == nullptr)
    return fail(SIA_ERR_INVALID_ARGUMENT, "%s is required for an int8 destination", name);
  if (s->ndim != 3) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must have 3 dims", name);
  if (s->dtype != SIA_F32 && s->dtype != SIA_F16)
    return fail(SIA_ERR_UNSUPPORTED, "%s must be float32 or float16", name);
  for (int d = 0; d < 3; ++d)
    if (s->shape[d] != like->shape[d])
      return fail(SIA_ERR_INVALID_ARGUMENT, "%s shape must be the destination shape without head_dim", name);
  if ((uintptr_t)s->data % elem_size(s->dtype)) return fail(SIA_ERR_INVALID_ARGUMENT, "%s misaligned", name);
  return SIA_OK;
}

// Validates a KV write of k/v (B, H, T, D) and fills `a` (everything but the
// RoPE fields); *dst_dtype receives the destination dtype.
int setup_kv_write(const sia_tensor* k, const sia_tensor* v, const sia_tensor* k_dst, const sia_tensor* v_dst,
                   const sia_tensor* k_scale_dst, const sia_tensor* v_scale_dst, const sia_tensor* block_table,
                   const sia_tensor* start_pos, int32_t start_pos_host, int32_t page_size, KvWriteArgs& a,
                   int* dst_dtype) {
  int rc;
  if ((rc = check_rows(k, "k", 16))) return rc;
  if (!src_dtype_ok(k->dtype)) return fail(SIA_ERR_UNSUPPORTED, "k dtype %s: expected float16, bfloat16 or float32",
                                           dtype_name(k->dtype));
  const bool two = v != nullptr;
  if (two) {
    if ((rc = check_rows(v, "v", 16))) return rc;
    if (v->dtype != k->dtype) return fail(SIA_ERR_INVALID_ARGUMENT, "k and v dtypes differ");
    for (int d = 0; d < 4; ++d)
      if (v->shape[d] != k->shape[d]) return fail(SIA_ERR_INVALID_ARGUMENT, "k and v shapes differ");
    if (bstride(v, 0) != bstride(k, 0) || bstride(v, 1) != bstride(k, 1) || bstride(v, 2) != bstride(k, 2))
      return fail(SIA_ERR_INVALID_ARGUMENT, "k and v must have the same strides");
  }
  const int64_t B = k->shape[0], H = k->shape[1], T = k->shape[2], D = k->shape[3];
  if (D != 64 && D != 128 && D != 256 && D != 16 && D != 32)
    return fail(SIA_ERR_UNSUPPORTED, "head_dim %lld not supported (16, 32, 64, 128, 256)", (long long)D);
  if (k_dst == nullptr || k_dst->data == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "k_dst is missing");
  const int dd = k_dst->dtype;
  const bool int8 = dd == SIA_I8;
  const int align = int8 ? 8 : 16;
  if ((rc = check_rows(k_dst, "k_dst", align))) return rc;
  if (two) {
    if ((rc = check_rows(v_dst, "v_dst", align))) return rc;
    if (v_dst->dtype != dd) return fail(SIA_ERR_INVALID_ARGUMENT, "k_dst and v_dst dtypes differ");
    for (int d = 0; d < 4; ++d)
      if (v_dst->shape[d] != k_dst->shape[d]) return fail(SIA_ERR_INVALID_ARGUMENT, "k_dst and v_dst shapes differ");
    if (bstride(v_dst, 0) != bstride(k_dst, 0) || bstride(v_dst, 1) != bstride(k_dst, 1) ||
        bstride(v_dst, 2) != bstride(k_dst, 2))
      return fail(SIA_ERR_INVALID_ARGUMENT, "k_dst and v_dst must have the same strides");
  }
  if (k_dst->shape[1] != H || k_dst->shape[3] != D)
    return fail(SIA_ERR_INVALID_ARGUMENT, "destination must be (*, %lld, *, %lld)", (long long)H, (long long)D);
  if (int8) {
    if ((rc = check_scale(k_scale_dst, k_dst, "k_scale_dst"))) return rc;
    if (two) {
      if ((rc = check_scale(v_scale_dst, k_dst, "v_scale_dst"))) return rc;
      if (v_scale_dst->dtype != k_scale_dst->dtype || v_scale_dst->stride[0] != k_scale_dst->stride[0] ||
          v_scale_dst->stride[1] != k_scale_dst->stride[1] || v_scale_dst->stride[2] != k_scale_dst->stride[2])
        return fail(SIA_ERR_INVALID_ARGUMENT, "k_scale_dst and v_scale_dst must share dtype and strides");
    }
  } else if (dd != SIA_F16 && dd != SIA_BF16 && dd != SIA_F32) {
    return fail(SIA_ERR_UNSUPPORTED, "destination dtype %s not supported", dtype_name(dd));
  }

  memset(&a, 0, sizeof(a));
  if (block_table != nullptr) {
    if (block_table->data == nullptr || block_table->ndim != 2 || block_table->dtype != SIA_I32)
      return fail(SIA_ERR_INVALID_ARGUMENT, "block_table must be a (B, max_blocks) int32 tensor");
    if (block_table->shape[0] < B) return fail(SIA_ERR_INVALID_ARGUMENT, "block_table has fewer rows than the batch");
    if (page_size <= 0 || k_dst->shape[2] != page_size)
      return fail(SIA_ERR_INVALID_ARGUMENT, "pool page dim %lld != page_size %d", (long long)k_dst->shape[2], page_size);
    const int64_t cap = block_table->shape[1] * (int64_t)page_size;
    if (cap > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "block table capacity too large");
    a.bt = (const int32_t*)block_table->data;
    a.bt_sb = block_table->stride[0];
    a.bt_sl = block_table->stride[1];
    a.num_pages = k_dst->shape[0];
    a.page = page_size;
    a.cap = (int32_t)cap;
  } else {
    if (k_dst->shape[0] < B) return fail(SIA_ERR_INVALID_ARGUMENT, "cache batch dim smaller than the batch");
    if (k_dst->shape[2] > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "cache length too large");
    a.cap = (int32_t)k_dst->shape[2];
    a.page = 1;
  }
  if (start_pos != nullptr) {
    if (start_pos->data == nullptr || start_pos->dtype != SIA_I32 || start_pos->ndim > 1)
      return fail(SIA_ERR_INVALID_ARGUMENT, "start_pos must be an int32 scalar, (1,) or (B,) tensor");
    const int64_t n = start_pos->ndim == 0 ? 1 : start_pos->shape[0];
    if (n != 1 && n != B) return fail(SIA_ERR_INVALID_ARGUMENT, "start_pos must have 1 or B elements");
    if (n == B && B > 1 && start_pos->stride[0] != 1)
      return fail(SIA_ERR_INVALID_ARGUMENT, "start_pos must be contiguous");
    a.start = (const int32_t*)start_pos->data;
    a.start_per_seq = (n == B && B > 1) ? 1 : 0;
    a.start_host = start_pos_host;   // added to the device value
  } else {
    a.start_host = start_pos_host;
    if (block_table == nullptr && (start_pos_host < 0 || (int64_t)start_pos_host + T > a.cap))
      return fail(SIA_ERR_INVALID_ARGUMENT, "positions [%d, %lld) exceed the cache length %d", start_pos_host,
                  (long long)start_pos_host + T, a.cap);
  }
  if (B * H * T > ((int64_t)1 << 40)) return fail(SIA_ERR_UNSUPPORTED, "too many rows");
  if (B > 0x7fffffff || H > 0x7fffffff || T > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "sizes too large");
  if ((rc = device_ok())) return rc;

  a.src0 = (const char*)k->data;
  a.src1 = two ? (const char*)v->data : nullptr;
  a.s_sb = bstride(k, 0); a.s_sh = bstride(k, 1); a.s_st = bstride(k, 2);
  a.dst0 = (char*)k_dst->data;
  a.dst1 = two ? (char*)v_dst->data : nullptr;
  a.d_s0 = bstride(k_dst, 0); a.d_sh = bstride(k_dst, 1); a.d_sn = bstride(k_dst, 2);
  if (int8) {
    a.sc0 = (char*)k_scale_dst->data;
    a.sc1 = two ? (char*)v_scale_dst->data : nullptr;
    a.c_s0 = bstride(k_scale_dst, 0); a.c_sh = bstride(k_scale_dst, 1); a.c_sn = bstride(k_scale_dst, 2);
    a.scale_f32 = k_scale_dst->dtype == SIA_F32;
  }
  a.B = (int32_t)B; a.H = (int32_t)H; a.T = (int32_t)T; a.D = (int32_t)D;
  a.rows = B * H * T;
  a.ntensors = two ? 2 : 1;
  a.amax_floor = amax_floor(k->dtype);
  *dst_dtype = dd;
  return SIA_OK;
}

// (B, T, H, D) viewed as (B, H, T, D): dims 1 and 2 swapped, same memory.
sia_tensor token_major_as_head_major(const sia_tensor* x) {
  sia_tensor y = *x;
  y.shape[1] = x->shape[2]; y.stride[1] = x->stride[2];
  y.shape[2] = x->shape[1]; y.stride[2] = x->stride[1];
  return y;
}

}  // namespace

extern "C" {

int sia_kv_write(const sia_tensor* k, const sia_tensor* v, const sia_tensor* k_dst, const sia_tensor* v_dst,
                 const sia_tensor* k_scale_dst, const sia_tensor* v_scale_dst, const sia_tensor* block_table,
                 const sia_tensor* start_pos, int32_t start_pos_host, int32_t page_size, void* stream) {
  KvWriteArgs a;
  int dd = 0, rc;
  if ((rc = setup_kv_write(k, v, k_dst, v_dst, k_scale_dst, v_scale_dst, block_table, start_pos, start_pos_host,
                           page_size, a, &dd)))
    return rc;
  return launch_kv_write(a, k->dtype, dd, (hipStream_t)stream);
}

int sia_rope_kv_write(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, const sia_tensor* cos,
                      const sia_tensor* sin, int32_t interleaved, const sia_tensor* q_out, const sia_tensor* k_dst,
                      const sia_tensor* v_dst, const sia_tensor* k_scale_dst, const sia_tensor* v_scale_dst,
                      const sia_tensor* block_table, const sia_tensor* start_pos, int32_t start_pos_host,
                      int32_t page_size, void* stream) {
  if (k == nullptr || cos == nullptr || sin == nullptr)
    return fail(SIA_ERR_INVALID_ARGUMENT, "k, cos and sin are required");
  if (k->ndim != 4 || (v != nullptr && v->ndim != 4))
    return fail(SIA_ERR_INVALID_ARGUMENT, "k and v must be (B, T, Hkv, D)");
  const sia_tensor kh = token_major_as_head_major(k);
  sia_tensor vh;
  if (v != nullptr) vh = token_major_as_head_major(v);
  KvWriteArgs a;
  int dd = 0, rc;
  if ((rc = setup_kv_write(&kh, v ? &vh : nullptr, k_dst, v_dst, k_scale_dst, v_scale_dst, block_table, start_pos,
                           start_pos_host, page_size, a, &dd)))
    return rc;
  const int64_t B = k->shape[0], T = k->shape[1], D = k->shape[3];
  // tables
  if (cos->data == nullptr || sin->data == nullptr || cos->ndim != 2 || sin->ndim != 2)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must be (rows, width) tables");
  if (cos->shape[0] != sin->shape[0] || cos->shape[1] != sin->shape[1])
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must have identical shape");
  if (cos->shape[1] != D && cos->shape[1] != D / 2)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin last dim must be head_dim (%lld) or head_dim/2 (%lld)",
                (long long)D, (long long)(D / 2));
  if (cos->dtype != sin->dtype || (cos->dtype != SIA_F16 && cos->dtype != SIA_BF16 && cos->dtype != SIA_F32))
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must share a float dtype");
  if (cos->stride[1] != 1 || sin->stride[1] != 1 || cos->stride[0] != sin->stride[0])
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin must be unit-stride rows with one row stride");
  if (cos->shape[0] <= 0 || cos->shape[0] > 0x7fffffff) return fail(SIA_ERR_INVALID_ARGUMENT, "bad table row count");
  // positions known on the host must have a table row (device positions are
  // checked on the device: rows outside the table are skipped / zeroed)
  if (start_pos == nullptr && (start_pos_host < 0 || (int64_t)start_pos_host + T > cos->shape[0]))
    return fail(SIA_ERR_INVALID_ARGUMENT, "positions [%d, %lld) need cos/sin rows the %lld-row tables do not have",
                start_pos_host, (long long)start_pos_host + T, (long long)cos->shape[0]);
  a.rope = interleaved ? 2 : 1;
  a.cs = (const char*)cos->data;
  a.sn = (const char*)sin->data;
  a.tab_rs = cos->stride[0] * elem_size(cos->dtype);
  a.Tc = (int32_t)cos->shape[0];
  a.tab_dt = cos->dtype;
  if (!aligned16(cos->data) || !aligned16(sin->data) || a.tab_rs % 16 != 0)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin must be 16-byte aligned with 16-byte multiple row strides");
  // q
  if ((q == nullptr) != (q_out == nullptr)) return fail(SIA_ERR_INVALID_ARGUMENT, "q and q_out go together");
  if (q != nullptr) {
    if ((rc = check_rows(q, "q", 16)) || (rc = check_rows(q_out, "q_out", 16))) return rc;
    if (q->dtype != k->dtype || q_out->dtype != k->dtype)
      return fail(SIA_ERR_INVALID_ARGUMENT, "q, q_out and k must share a dtype");
    if (q->shape[0] != B || q->shape[1] != T || q->shape[3] != D)
      return fail(SIA_ERR_INVALID_ARGUMENT, "q must be (B, T, Hq, D) with k's B, T and D");
    for (int d = 0; d < 4; ++d)
      if (q_out->shape[d] != q->shape[d]) return fail(SIA_ERR_INVALID_ARGUMENT, "q_out shape differs from q");
    if (q->shape[2] > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "too many query heads");
    a.q = (const char*)q->data;
    a.qo = (char*)q_out->data;
    a.q_sb = bstride(q, 0); a.q_st = bstride(q, 1); a.q_sh = bstride(q, 2);
    a.qo_sb = bstride(q_out, 0); a.qo_st = bstride(q_out, 1); a.qo_sh = bstride(q_out, 2);
    a.Hq = (int32_t)q->shape[2];
    a.q_rows = B * q->shape[2] * T;
  }
  return launch_kv_write(a, k->dtype, dd, (hipStream_t)stream);
}

int sia_quantize_kv_int8(const sia_tensor* x, const sia_tensor* out_int8, const sia_tensor* out_scale, void* stream) {
  if (x == nullptr || out_int8 == nullptr || out_scale == nullptr)
    return fail(SIA_ERR_INVALID_ARGUMENT, "x, out_int8 and out_scale are required");
  if (x->ndim < 1 || x->ndim > 4) return fail(SIA_ERR_UNSUPPORTED, "x must have 1 to 4 dims");
  if (out_int8->ndim != x->ndim || out_scale->ndim != x->ndim - 1)
    return fail(SIA_ERR_INVALID_ARGUMENT, "out_int8 must match x and out_scale must drop head_dim");
  if (out_int8->dtype != SIA_I8) return fail(SIA_ERR_INVALID_ARGUMENT, "out_int8 must be int8");
  for (int d = 0; d < x->ndim; ++d)
    if (out_int8->shape[d] != x->shape[d]) return fail(SIA_ERR_INVALID_ARGUMENT, "out_int8 shape differs from x");
  for (int d = 0; d + 1 < x->ndim; ++d)
    if (out_scale->shape[d] != x->shape[d]) return fail(SIA_ERR_INVALID_ARGUMENT, "out_scale shape differs from x[:-1]");
  // view all three as 4-dim (leading dims of size 1)
  sia_tensor xv, ov, sv;
  memset(&xv, 0, sizeof(xv));
  memset(&ov, 0, sizeof(ov));
  memset(&sv, 0, sizeof(sv));
  const int pad = 4 - x->ndim;
  xv.data = x->data; xv.dtype = x->dtype; xv.ndim = 4;
  ov.data = out_int8->data; ov.dtype = SIA_I8; ov.ndim = 4;
  sv.data = out_scale->data; sv.dtype = out_scale->dtype; sv.ndim = 3;
  for (int d = 0; d < 4; ++d) {
    const int s = d - pad;
    xv.shape[d] = s >= 0 ? x->shape[s] : 1;
    xv.stride[d] = s >= 0 ? x->stride[s] : 0;
    ov.shape[d] = s >= 0 ? out_int8->shape[s] : 1;
    ov.stride[d] = s >= 0 ? out_int8->stride[s] : 0;
    if (d < 3) {
      sv.shape[d] = s >= 0 ? out_scale->shape[s] : 1;
      sv.stride[d] = s >= 0 ? out_scale->stride[s] : 0;
    }
  }
  return sia_kv_write(&xv, nullptr, &ov, nullptr, &sv, nullptr, nullptr, nullptr, 0, 0, stream);
}

}  // extern "C"
