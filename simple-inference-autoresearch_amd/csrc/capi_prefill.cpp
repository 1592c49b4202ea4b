// extern "C" prefill entry points: validation, workspace size and dispatch.
#include <math.h>
#include <string.h>

#include "attn_f32.hpp"
#include "host_util.hpp"
#include "prefill_launch.hpp"

using namespace sia;

namespace {

int check4(const sia_tensor* t, const char* name) {
  if (t == nullptr || t->data == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "%s is missing", name);
  if (t->ndim != 4) return fail(SIA_ERR_INVALID_ARGUMENT, "%s must have 4 dims", name);
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
  if (!(sm_scale > 0.f) || !isfinite(sm_scale)) return fail(SIA_ERR_INVALID_ARGUMENT, "sm_scale must be positive");
  if (q->dtype == SIA_F32) return prefill_f32(q, k, v, causal, sm_scale, out, stream);
  const int64_t need = image_bytes(B, Hkv, Tk, D);
  if (need > 0 && (workspace == nullptr || (uintptr_t)workspace % 256 || workspace_bytes < (size_t)need))
    return fail(SIA_ERR_WORKSPACE, "prefill workspace missing, misaligned or smaller than %lld bytes",
                (long long)need);
  const DeviceInfo& dev = device_info();
  if (dev.id < 0) return fail(SIA_ERR_DEVICE, "no HIP device is current");
  if (!dev.gfx950) return fail(SIA_ERR_DEVICE, "this library is built for gfx950 (MI355X) only");
  if (Tq == 0) return SIA_OK;

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
  const int bm = pf_rows_per_group((int)D);
  a.nqblk = (int)((Tq + bm - 1) / bm);
  a.nkb = (int)((Tk + kPfBN - 1) / kPfBN);
  const int64_t groups = (int64_t)a.nqblk * B * Hkv;   // work-groups come in runs of G sharing a KV head
  if (groups * a.G > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "grid too large");
  a.remap = groups % 8 == 0;

  PackArgs& p = L.pack;
  p.v = (const char*)v->data; p.v_sb = bstride(v, 0); p.v_sh = bstride(v, 1); p.v_sn = bstride(v, 2);
  p.vimg = (char*)workspace;
  p.Hkv = (int)Hkv; p.Tk = (int)Tk; p.nkb = a.nkb;
  p.nblocks = B * Hkv * a.nkb;
  // one work-group per image (grid x dimension), 32-bit indexed in the kernel
  if (p.nblocks > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "K/V too large");
  L.D = (int)D;
  L.dtype = q->dtype;
  L.stream = (hipStream_t)stream;
  return launch_prefill(L);
}
