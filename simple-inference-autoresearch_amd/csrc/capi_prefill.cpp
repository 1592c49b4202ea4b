// extern "C" prefill entry points: validation, workspace size and dispatch.
#include <math.h>
#include <string.h>

#include "attn_f32.hpp"
#include "host_util.hpp"
#include "prefill_launch.hpp"

using namespace sia;

namespace {

int check4(const sia_tensor* t, const char* name) {
  if (t == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "%s is missing", name);
  if (t->ndim != 4) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must have 4 dims", name);
  // an empty tensor (no queries, or no keys) may have no data pointer: it is
  // never read or written
  const bool empty = t->shape[0] == 0 || t->shape[1] == 0 || t->shape[2] == 0 || t->shape[3] == 0;
  if (t->data == nullptr && !empty) return fail(SIA_ERR_INVALID_ARGUMENT, "%s is missing", name);
  if (t->stride[3] != 1) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must be contiguous along head_dim", name);
  if (!aligned16(t->data)) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must be 16-byte aligned", name);
  for (int d = 0; d < 3; ++d)
    if (bstride(t, d) % 16) return fail(SIA_ERR_INVALID_ARGUMENT, "%s strides must be multiples of 16 bytes", name);
  return SIA_OK;
}

bool head_dim_ok(int64_t D) { return D == 16 || D == 32 || D == 64 || D == 128 || D == 256; }

// V^T block images: one f16 (64 x max(head_dim, 32)) image per 64-key block of every (b, kv head).
int64_t image_bytes(int64_t B, int64_t Hkv, int64_t Tk, int64_t D) {
  const int64_t nkb = (Tk + kPfBN - 1) / kPfBN;
  const int64_t DV = D < 32 ? 32 : D;
  return B * Hkv * nkb * kPfBN * DV * 2;
}

// Float32 q/k/v: the vector-ALU path (attn_f32.hpp), one work item per
// (sequence, KV head, chunk of query rows x heads), no workspace.
int prefill_f32(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, int32_t causal, float sm_scale,
                const sia_tensor* out, void* stream) {
  const int64_t B = q->shape[0], Hq = q->shape[1], Tq = q->shape[2], D = q->shape[3];
  const int64_t Hkv = k->shape[1], Tk = k->shape[2];
  const int64_t G = Hq / Hkv;
  if (Tq * G > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "too many query rows");
  const DeviceInfo& dev = device_info();
  if (dev.id < 0) return fail(SIA_ERR_DEVICE, "no HIP device is current");
  if (!dev.gfx950) return fail(SIA_ERR_DEVICE, "this library is built for gfx950 (MI355X) only");
  if (Tq == 0) return SIA_OK;
  F32Launch L;
  memset(&L, 0, sizeof(L));
  F32Args& a = L.a;
  a.q = (const char*)q->data; a.q_sb = bstride(q, 0); a.q_sh = bstride(q, 1); a.q_sm = bstride(q, 2);
  a.out = (char*)out->data; a.o_sb = bstride(out, 0); a.o_sh = bstride(out, 1); a.o_sm = bstride(out, 2);
  a.k = (const char*)k->data; a.k_s0 = bstride(k, 0); a.k_sh = bstride(k, 1); a.k_sn = bstride(k, 2);
  a.v = (const char*)v->data; a.v_s0 = bstride(v, 0); a.v_sh = bstride(v, 1); a.v_sn = bstride(v, 2);
  a.cap = (int)Tk;
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)G; a.Tq = (int)Tq; a.Tk = (int)Tk;
  a.causal = causal != 0;
  a.ncol = (int)(Tq * G);
  a.nchunk = (int)((Tq * G + kF32Cols - 1) / kF32Cols);
  a.nsplit = 1;
  a.tps = Tk > 0 ? (int)Tk : 1;
  a.qk_scale = sm_scale * 1.4426950408889634f;
  L.D = (int)D;
  L.q_dtype = SIA_F32;
  L.kv_dtype = SIA_F32;
  L.stream = (hipStream_t)stream;
  return launch_attn_f32(L);
}

// Rotary tables of the fused entry point (NULL cos: no rotation).
struct RopeIn {
  const sia_tensor* cos;
  const sia_tensor* sin;
  const sia_tensor* start_pos;
  int32_t start_host;
  int32_t interleaved;
};

// Checks the tables and positions against q (B, Hq, Tq, D) and fills the
// rotation fields of the kernel arguments.
int setup_rope(const RopeIn& r, int64_t B, int64_t Tq, int64_t D, int q_dtype, PrefillArgs& a) {
  const sia_tensor* cos = r.cos;
  const sia_tensor* sin = r.sin;
  if (cos == nullptr || sin == nullptr || cos->data == nullptr || sin->data == nullptr || cos->ndim != 2 ||
      sin->ndim != 2)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must be (rows, width) tables");
  if (cos->shape[0] != sin->shape[0] || cos->shape[1] != sin->shape[1])
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must have identical shape");
  if (cos->shape[1] != D && cos->shape[1] != D / 2)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin last dim must be head_dim (%lld) or head_dim/2 (%lld)",
                (long long)D, (long long)(D / 2));
  if (cos->dtype != sin->dtype || (cos->dtype != SIA_F16 && cos->dtype != SIA_BF16 && cos->dtype != SIA_F32))
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos and sin must share a float dtype");
  if (cos->dtype != q_dtype && cos->dtype != SIA_F32)
    return fail(SIA_ERR_UNSUPPORTED, "cos/sin dtype %s: the fused prologue reads tables in q's dtype or float32",
                dtype_name(cos->dtype));
  if (cos->stride[1] != 1 || sin->stride[1] != 1 || cos->stride[0] != sin->stride[0])
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin must be unit-stride rows with one row stride");
  if (cos->shape[0] <= 0 || cos->shape[0] > 0x7fffffff) return fail(SIA_ERR_INVALID_ARGUMENT, "bad table row count");
  a.tab_rs = cos->stride[0] * elem_size(cos->dtype);
  if (!aligned16(cos->data) || !aligned16(sin->data) || a.tab_rs % 16 != 0)
    return fail(SIA_ERR_INVALID_ARGUMENT, "cos/sin must be 16-byte aligned with 16-byte multiple row strides");
  if (r.start_pos != nullptr) {
    const sia_tensor* sp = r.start_pos;
    if (sp->data == nullptr || sp->dtype != SIA_I32 || sp->ndim > 1)
      return fail(SIA_ERR_INVALID_ARGUMENT, "start_pos must be an int32 scalar, (1,) or (B,) tensor");
    const int64_t n = sp->ndim == 0 ? 1 : sp->shape[0];
    if (n != 1 && n != B) return fail(SIA_ERR_INVALID_ARGUMENT, "start_pos must have 1 or B elements");
    if (n == B && B > 1 && sp->stride[0] != 1) return fail(SIA_ERR_INVALID_ARGUMENT, "start_pos must be contiguous");
    a.start_pos = (const int32_t*)sp->data;
    a.pos_per_seq = n == B && B > 1;
  } else if (r.start_host < 0 || (int64_t)r.start_host + Tq > cos->shape[0]) {
    // positions known on the host must have a table row; device positions
    // outside the table rotate q to zeros
    return fail(SIA_ERR_INVALID_ARGUMENT, "positions [%d, %lld) need cos/sin rows the %lld-row tables do not have",
                r.start_host, (long long)r.start_host + Tq, (long long)cos->shape[0]);
  }
  a.start_host = r.start_host;
  a.cs = (const char*)cos->data;
  a.sn = (const char*)sin->data;
  a.Tc = (int32_t)cos->shape[0];
  a.tab_dt = cos->dtype;
  a.interleaved = r.interleaved != 0;
  return SIA_OK;
}

int flash_fwd(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, int32_t causal, float sm_scale,
              const sia_tensor* out, void* workspace, size_t workspace_bytes, void* stream, const RopeIn* rope) {
  int rc;
  if ((rc = check4(q, "q")) || (rc = check4(k, "k")) || (rc = check4(v, "v")) || (rc = check4(out, "out"))) return rc;
  if (q->dtype != SIA_F16 && q->dtype != SIA_BF16 && q->dtype != SIA_F32)
    return fail(SIA_ERR_UNSUPPORTED, "q dtype %s: expected float16, bfloat16 or float32", dtype_name(q->dtype));
  if (k->dtype != q->dtype || v->dtype != q->dtype || out->dtype != q->dtype)
    return fail(SIA_ERR_INVALID_ARGUMENT, "q, k, v and out must share one dtype");
  const int64_t B = q->shape[0], Hq = q->shape[1], Tq = q->shape[2], D = q->shape[3];
  const int64_t Hkv = k->shape[1], Tk = k->shape[2];
  if (k->shape[0] != B || v->shape[0] != B || k->shape[3] != D || v->shape[3] != D || v->shape[1] != Hkv ||
      v->shape[2] != Tk)
    return fail(SIA_ERR_INVALID_ARGUMENT, "k and v must be (B, Hkv, Tk, D) matching q");
  if (out->shape[0] != B || out->shape[1] != Hq || out->shape[2] != Tq || out->shape[3] != D)
    return fail(SIA_ERR_INVALID_ARGUMENT, "out must be a (B, Hq, Tq, D) view");
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Tq < 0 || Tk < 0) return fail(SIA_ERR_INVALID_ARGUMENT, "bad sizes");
  if (Hq % Hkv) return fail(SIA_ERR_INVALID_ARGUMENT, "Hq must be a multiple of Hkv");
  if (!head_dim_ok(D))
    return fail(SIA_ERR_UNSUPPORTED, "prefill head_dim %lld not supported (16, 32, 64, 128, 256)", (long long)D);
  if (Tq > (1 << 30) || Tk > (1 << 30)) return fail(SIA_ERR_UNSUPPORTED, "sequence too long");
  // K rows are fetched by 32-bit buffer offsets of up to 64 rows from a block start
  const int64_t k_sn = bstride(k, 2);
  if (Tk > 1 && (k_sn < 2 * D || k_sn * kPfBN >= ((int64_t)1 << 31)))
    return fail(SIA_ERR_UNSUPPORTED, "k token stride %lld bytes: expected [%lld, 2^31/64)", (long long)k_sn,
                (long long)(2 * D));
  // float16 V at head_dim 32-128 is read in place like K (no V^T images)
  const bool v_in_place = q->dtype == SIA_F16 && D >= 32 && D <= 128;
  const int64_t v_sn = bstride(v, 2);
  const bool v_rows_ok = Tk <= 1 || (v_sn >= 2 * D && v_sn * kPfBN < ((int64_t)1 << 31));
  if (v_in_place && !v_rows_ok)
    return fail(SIA_ERR_UNSUPPORTED, "v token stride %lld bytes: expected [%lld, 2^31/64)", (long long)v_sn,
                (long long)(2 * D));
  if (!(sm_scale > 0.f) || !isfinite(sm_scale)) return fail(SIA_ERR_INVALID_ARGUMENT, "sm_scale must be positive");
  if (q->dtype == SIA_F32) {
    if (rope != nullptr)
      return fail(SIA_ERR_UNSUPPORTED, "the rotary prologue runs on the float16/bfloat16 MFMA path only");
    return prefill_f32(q, k, v, causal, sm_scale, out, stream);
  }
  const int64_t need = v_in_place ? 0 : image_bytes(B, Hkv, Tk, D);   // (V^T images)
  if (need > 0 && (workspace == nullptr || (uintptr_t)workspace % 256 || workspace_bytes < (size_t)need))
    return fail(SIA_ERR_WORKSPACE, "prefill workspace missing, misaligned or smaller than %lld bytes",
                (long long)need);
  const DeviceInfo& dev = device_info();
  if (dev.id < 0) return fail(SIA_ERR_DEVICE, "no HIP device is current");
  if (!dev.gfx950) return fail(SIA_ERR_DEVICE, "this library is built for gfx950 (MI355X) only");

  PrefillLaunch L;
  memset(&L, 0, sizeof(L));
  PrefillArgs& a = L.a;
  a.q = (const char*)q->data; a.q_sb = bstride(q, 0); a.q_sh = bstride(q, 1); a.q_sm = bstride(q, 2);
  a.k = (const char*)k->data; a.k_sb = bstride(k, 0); a.k_sh = bstride(k, 1); a.k_sn = k_sn;
  a.vimg = (const char*)workspace;
  a.out = (char*)out->data; a.o_sb = bstride(out, 0); a.o_sh = bstride(out, 1); a.o_sm = bstride(out, 2);
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv); a.Tq = (int)Tq; a.Tk = (int)Tk;
  a.causal = causal != 0;
  a.qk_scale = sm_scale * 1.4426950408889634f;
  // a work-group: hpw query heads of one KV head x 32 * waves / hpw rows each.
  // At D = 128, a grid of at most one 8-wave group per CU runs as 4-wave
  // groups instead (prefill_fwd variant 1): twice the groups, each with half
  // the rows.  (Up to two 8-wave groups per CU this was measured slower.)
  auto groups = [&](int var) {
    const int h = pf_heads_per_group((int)D, a.G, var);
    const int64_t r = 32 * pf_waves((int)D, var) / h;
    return ((Tq + r - 1) / r) * (B * Hkv * (a.G / h));
  };
  L.var = D == 128 && groups(0) <= dev.cus ? 1 : 0;
  const int hpw = pf_heads_per_group((int)D, a.G, L.var);
  int lg = 0;
  while ((1 << lg) < hpw) ++lg;
  a.hpw_lg = lg;
  const int rows = 32 * pf_waves((int)D, L.var) / hpw;
  a.nqblk = (int)((Tq + rows - 1) / rows);
  a.nkb = (int)((Tk + kPfBN - 1) / kPfBN);
  const int64_t nunit = B * Hkv * (a.G / hpw);
  if ((int64_t)a.nqblk * nunit > 0x7fffffff || B * Hkv > 0x7fffffff)
    return fail(SIA_ERR_UNSUPPORTED, "grid too large");
  a.nunit = (int)nunit;
  a.remap = nunit % 8 == 0;
  a.dU = make_fastdiv((uint32_t)nunit);
  a.dU8 = make_fastdiv((uint32_t)(a.remap ? nunit / 8 : 1));
  a.dBH = make_fastdiv((uint32_t)(B * Hkv));
  a.dHkv = make_fastdiv((uint32_t)Hkv);
  if (rope != nullptr && (rc = setup_rope(*rope, B, Tq, D, q->dtype, a))) return rc;

  // Variant 1 runs two work-groups per CU: a grid of one to two per CU is
  // resident at once and is folded so that each CU holds a heavy and a light
  // one (B1 x 2048 tokens: the first CU otherwise holds the two heaviest
  // causal query blocks' work against half of that on the last).
  const int64_t nall = (int64_t)a.nqblk * nunit;
  a.fold = L.var == 1 && dev.cus % 8 == 0 && nall > dev.cus && nall <= 2 * (int64_t)dev.cus ? dev.cus : 0;

  PackArgs& p = L.pack;
  p.v = (const char*)v->data; p.v_sb = bstride(v, 0); p.v_sh = bstride(v, 1); p.v_sn = bstride(v, 2);
  p.vimg = (char*)workspace;
  p.Hkv = (int)Hkv; p.Tk = (int)Tk; p.nkb = a.nkb;
  p.nblocks = B * Hkv * a.nkb;
  // Short key ranges on a 4-wave grid of at most two work-groups per CU:
  // every work-group converts the bf16 V blocks it walks to f16 in LDS
  // (variant 2) instead of prefill_pack_v repacking V, one launch less.
  // The raw V rows take the K rows' path (32-bit offsets within a block).
  if (v_in_place) {
    // float16 V needs no conversion: every variant takes raw V rows and reads
    // them transposed from LDS (no V^T images, no repack)
    a.v = p.v; a.v_sb = p.v_sb; a.v_sh = p.v_sh; a.v_sn = v_sn;
    p.nblocks = 0;
  } else if (q->dtype == SIA_BF16 && (L.var == 1 || ((D == 32 || D == 64) && L.var == 0)) &&
             Tk <= (D <= 64 ? kPackvMaxKeysD64 : kPackvMaxKeys) &&
             (int64_t)a.nqblk * nunit <= 2 * (int64_t)dev.cus &&
             v_rows_ok) {
    L.var = 2;
    a.v = p.v; a.v_sb = p.v_sb; a.v_sh = p.v_sh; a.v_sn = v_sn;
    p.nblocks = 0;   // no separate repack
  }
  // one work-group per image (grid x dimension), 32-bit indexed in the kernel
  if (p.nblocks > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "K/V too large");
  if (Tq == 0) return SIA_OK;
  L.D = (int)D;
  L.dtype = q->dtype;
  L.stream = (hipStream_t)stream;
  return launch_prefill(L);
}

}  // namespace

extern "C" int sia_prefill_workspace_size(int64_t batch, int64_t kv_heads, int64_t kv_len, int64_t head_dim,
                                          size_t* bytes) {
  if (bytes == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "bytes is NULL");
  if (batch <= 0 || kv_heads <= 0 || kv_len < 0) return fail(SIA_ERR_INVALID_ARGUMENT, "bad sizes");
  if (!head_dim_ok(head_dim))
    return fail(SIA_ERR_UNSUPPORTED, "prefill head_dim %lld not supported (16, 32, 64, 128, 256)",
                (long long)head_dim);
  *bytes = (size_t)image_bytes(batch, kv_heads, kv_len, head_dim);
  return SIA_OK;
}

extern "C" int sia_attention_flash_fwd(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, int32_t causal,
                                       float sm_scale, const sia_tensor* out, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  return flash_fwd(q, k, v, causal, sm_scale, out, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int sia_attention_flash_fwd_rope(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v,
                                            const sia_tensor* cos, const sia_tensor* sin, int32_t interleaved,
                                            const sia_tensor* start_pos, int32_t start_pos_host, int32_t causal,
                                            float sm_scale, const sia_tensor* out, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  const RopeIn r{cos, sin, start_pos, start_pos_host, interleaved};
  return flash_fwd(q, k, v, causal, sm_scale, out, workspace, workspace_bytes, stream, &r);
}
