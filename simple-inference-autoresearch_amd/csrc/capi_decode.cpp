// extern "C" decode entry points: validation, workspace layout, dispatch.
#include <math.h>
#include <string.h>

#include <mutex>

#include "attn_f32.hpp"
#include "decode_launch.hpp"
#include "host_util.hpp"

namespace sia {
const char* last_message();
}

using namespace sia;

namespace {


inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

struct Geometry {
  int B, Hq, Hkv, D, G, HG, U, UB, IU, G16;
};

size_t plan_bytes(int B) { return (size_t)round_up((int64_t)(kPlanHeader + B + 1) * 4, 256); }
// One item holds a partial for each of its decode_waves(D) unit slots.
size_t item_bytes(const Geometry& g) { return (size_t)decode_waves(g.D) * g.G16 * (g.D + 2) * 4; }

// Partial slots the workspace must hold: two per persistent work-group (its
// first and last segment may each be a piece of a split sequence), for up to
// four groups per CU, plus slack.
int64_t wanted_items(const Geometry& g) {
  const int cus = device_info().cus > 0 ? device_info().cus : 256;
  return 2LL * cus * 4 + 64;
}

int geometry(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, Geometry& g) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0)
    return fail(SIA_ERR_INVALID_ARGUMENT, "batch, heads and head_dim must be positive");
  if (Hq % Hkv != 0)
    return fail(SIA_ERR_INVALID_ARGUMENT, "num_q_heads (%lld) must be a multiple of num_kv_heads (%lld)",
                (long long)Hq, (long long)Hkv);
  if (B > 16384) return fail(SIA_ERR_UNSUPPORTED, "batch %lld exceeds 16384", (long long)B);
  g.B = (int)B; g.Hq = (int)Hq; g.Hkv = (int)Hkv; g.D = (int)D;
  g.G = (int)(Hq / Hkv);
  g.HG = (g.G + 15) / 16;
  g.U = g.Hkv * g.HG;
  const int nw = decode_waves(g.D);
  g.IU = g.U < nw ? g.U : nw;   // units per item (see item_units)
  g.UB = (g.U + g.IU - 1) / g.IU;
  g.G16 = g.G < 16 ? g.G : 16;
  return SIA_OK;
}

// Units per item (the work-group's unit of work: IU units, NW / IU waves
// each).  IU starts at min(U, NW) and halves while the batch has fewer items
// than CUs: smaller items give the split more, shorter pieces to share out,
// and once there is an item per work-group every output row is written
// directly, with nothing for the split-K merge.  A contiguous cache takes the
// halved IU.  A paged pool takes it when it reaches an item per CU (B64 x 8
// KV heads: 2 units of 4 waves, config 3 182.5 -> 180.6 us per call) or holds
// at most 4 sequences (each otherwise split into up to hundreds of pieces:
// B1 x 8192 tokens 20.2 -> 16.7 us with inputs rotated past the MALL).
// Otherwise it keeps wide items: a page holds every KV head's 16 tokens side
// by side and the waves of a wide item read them together; narrower items
// that still leave a split ran config 2's main kernel 2-2.5 us (7%) slower.
void item_units(Geometry& g, bool paged) {
  const int nw = decode_waves(g.D);
  const int cus = device_info().cus > 0 ? device_info().cus : 256;
  auto items = [&](int iu) { return (int64_t)g.B * ((g.U + iu - 1) / iu); };
  g.IU = g.U < nw ? g.U : nw;
  int iu = g.IU;
  while (iu % 2 == 0 && items(iu) < cus) iu /= 2;
  if (!paged || items(iu) >= cus || g.B <= 4) g.IU = iu;
  g.UB = (g.U + g.IU - 1) / g.IU;
}

int check_tensor(const sia_tensor* t, const char* name, int ndim) {
  if (t == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "%s is NULL", name);
  if (t->data == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "%s has no data pointer", name);
  if (t->ndim != ndim)
    return fail(SIA_ERR_INVALID_ARGUMENT, "%s must have %d dims, got %d", name, ndim, t->ndim);
  return SIA_OK;
}

// Common checks of q/out/kv_len and fill of the q/out/len fields.
int prepare_common(const sia_tensor* q, const sia_tensor* kv_len, const sia_tensor* out, int Hkv,
                   float sm_scale, Geometry& g, DecodeLaunch& L) {
  int rc;
  if ((rc = check_tensor(q, "q", 4))) return rc;
  if ((rc = check_tensor(out, "out", 4))) return rc;
  if (kv_len == nullptr || kv_len->data == nullptr)
    return fail(SIA_ERR_INVALID_ARGUMENT, "kv_len is missing");
  if (q->dtype != SIA_F16 && q->dtype != SIA_BF16 && q->dtype != SIA_F32)
    return fail(SIA_ERR_UNSUPPORTED, "q dtype %s: expected float16, bfloat16 or float32", dtype_name(q->dtype));
  if (q->shape[2] != 1) return fail(SIA_ERR_INVALID_ARGUMENT, "decode kernel expects a single query position");
  if ((rc = geometry(q->shape[0], q->shape[1], Hkv, q->shape[3], g))) return rc;
  if (g.D != 16 && g.D != 32 && g.D != 64 && g.D != 128 && g.D != 256)
    return fail(SIA_ERR_UNSUPPORTED, "unsupported head_dim %d (16, 32, 64, 128, 256)", g.D);
  if (q->stride[3] != 1) return fail(SIA_ERR_INVALID_ARGUMENT, "q must be contiguous along head_dim");
  if (!aligned16(q->data) || bstride(q, 0) % 16 || bstride(q, 1) % 16)
    return fail(SIA_ERR_INVALID_ARGUMENT, "q rows must be 16-byte aligned");
  if (out->dtype != q->dtype) return fail(SIA_ERR_INVALID_ARGUMENT, "out dtype must equal q dtype");
  if (out->shape[0] != g.B || out->shape[1] != 1 || out->shape[2] != g.Hq || out->shape[3] != g.D)
    return fail(SIA_ERR_INVALID_ARGUMENT, "out must be (B, 1, Hq, D)");
  if (out->stride[3] != 1) return fail(SIA_ERR_INVALID_ARGUMENT, "out must be contiguous along head_dim");
  if (kv_len->dtype != SIA_I32) return fail(SIA_ERR_INVALID_ARGUMENT, "kv_len must be int32");
  int64_t n = 1;
  for (int i = 0; i < kv_len->ndim; ++i) n *= kv_len->shape[i];
  if (kv_len->ndim > 1 || (n != 1 && n != g.B))
    return fail(SIA_ERR_INVALID_ARGUMENT, "kv_len must be a scalar, (1,) or (B,) tensor");
  if (n == g.B && g.B > 1 && kv_len->ndim == 1 && kv_len->stride[0] != 1)
    return fail(SIA_ERR_INVALID_ARGUMENT, "kv_len must be contiguous");
  if (!(sm_scale > 0.0f) || !isfinite(sm_scale))
    return fail(SIA_ERR_INVALID_ARGUMENT, "sm_scale must be a positive finite number");
  const DeviceInfo& dev = device_info();
  if (dev.id < 0) return fail(SIA_ERR_DEVICE, "no HIP device is current");
  if (!dev.gfx950) return fail(SIA_ERR_DEVICE, "this library is built for gfx950 (MI355X) only");

  DecodeArgs& a = L.a;
  memset(&a, 0, sizeof(a));
  a.q = (const char*)q->data; a.q_sb = bstride(q, 0); a.q_sh = bstride(q, 1);
  a.out = (char*)out->data; a.o_sb = bstride(out, 0); a.o_sh = bstride(out, 2);
  a.kv_len = (const int32_t*)kv_len->data;
  a.kv_per_seq = (n == g.B && g.B > 1) ? 1 : 0;
  a.B = g.B; a.Hq = g.Hq; a.Hkv = g.Hkv; a.G = g.G; a.HG = g.HG; a.U = g.U; a.UB = g.UB; a.IU = g.IU; a.G16 = g.G16;
  a.qk_scale = sm_scale * 1.4426950408889634f;
  L.D = g.D;
  L.q_dtype = q->dtype;
  return SIA_OK;
}

// K/V (and scale) layout checks.  Contiguous: (B', Hkv, S, D) with B' >= B.
// Paged: (num_pages, Hkv, page_size, D).
int prepare_kv(const sia_tensor* k, const sia_tensor* v, const Geometry& g, bool paged, int page_size,
               DecodeLaunch& L) {
  int rc;
  if ((rc = check_tensor(k, "k", 4))) return rc;
  if ((rc = check_tensor(v, "v", 4))) return rc;
  if (k->dtype != v->dtype) return fail(SIA_ERR_INVALID_ARGUMENT, "k and v dtypes differ");
  for (int d = 0; d < 4; ++d)
    if (k->shape[d] != v->shape[d]) return fail(SIA_ERR_INVALID_ARGUMENT, "k and v shapes differ");
  if (k->shape[1] != g.Hkv || k->shape[3] != g.D)
    return fail(SIA_ERR_INVALID_ARGUMENT, "k/v must be (*, Hkv=%d, *, D=%d)", g.Hkv, g.D);
  if (k->stride[3] != 1 || v->stride[3] != 1)
    return fail(SIA_ERR_INVALID_ARGUMENT, "k/v must be contiguous along head_dim");
  if (!aligned16(k->data) || !aligned16(v->data))
    return fail(SIA_ERR_INVALID_ARGUMENT, "k/v base pointers must be 16-byte aligned");
  for (int d = 0; d < 3; ++d)
    if (bstride(k, d) % 16 || bstride(v, d) % 16)
      return fail(SIA_ERR_INVALID_ARGUMENT, "k/v strides must be multiples of 16 bytes");
  DecodeArgs& a = L.a;
  a.k = (const char*)k->data; a.k_s0 = bstride(k, 0); a.k_sh = bstride(k, 1); a.k_sn = bstride(k, 2);
  a.v = (const char*)v->data; a.v_s0 = bstride(v, 0); a.v_sh = bstride(v, 1); a.v_sn = bstride(v, 2);
  if (a.k_sn > 0x7fffffff || a.v_sn > 0x7fffffff || (paged && (a.k_s0 > 0xffffffffLL || a.v_s0 > 0xffffffffLL)))
    return fail(SIA_ERR_UNSUPPORTED, "k/v token or page stride too large");
  a.k_tok = (uint32_t)a.k_sn; a.v_tok = (uint32_t)a.v_sn;
  a.k_pg = paged ? (uint32_t)a.k_s0 : 0u; a.v_pg = paged ? (uint32_t)a.v_s0 : 0u;
  if (paged) {
    if (k->shape[2] != page_size)
      return fail(SIA_ERR_INVALID_ARGUMENT, "k_pool page dim %lld != page_size %d", (long long)k->shape[2], page_size);
    if (page_size < 1) return fail(SIA_ERR_INVALID_ARGUMENT, "page_size %d must be positive", page_size);
    // 16 * 2^k: whole 16-token tiles per page (the MFMA kernels); any other
    // page size runs on the vector-ALU path, which looks up every token's page
    int lg = 0;
    while ((16 << lg) < page_size) ++lg;
    a.lg_tiles_per_page = (16 << lg) == page_size ? lg : 0;
    a.num_pages = k->shape[0];
    L.page_size = page_size;
  } else {
    if (k->shape[0] < g.B) return fail(SIA_ERR_INVALID_ARGUMENT, "k/v batch dim smaller than q's");
    if (k->shape[2] > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "cache length too large");
    a.cap_tokens = (int)k->shape[2];
  }
  return SIA_OK;
}

int prepare_scales(const sia_tensor* ks, const sia_tensor* vs, const sia_tensor* k, bool paged, DecodeLaunch& L) {
  int rc;
  if ((rc = check_tensor(ks, "k_scale", 3))) return rc;
  if ((rc = check_tensor(vs, "v_scale", 3))) return rc;
  if (ks->dtype != vs->dtype || (ks->dtype != SIA_F32 && ks->dtype != SIA_F16))
    return fail(SIA_ERR_UNSUPPORTED, "k_scale/v_scale must both be float32 or float16");
  for (int d = 0; d < 3; ++d)
    if (ks->shape[d] != k->shape[d] || vs->shape[d] != k->shape[d])
      return fail(SIA_ERR_INVALID_ARGUMENT, "scale shape must be the K/V shape without head_dim");
  DecodeArgs& a = L.a;
  a.ks = (const char*)ks->data; a.ks_s0 = bstride(ks, 0); a.ks_sh = bstride(ks, 1); a.ks_sn = bstride(ks, 2);
  a.vs = (const char*)vs->data; a.vs_s0 = bstride(vs, 0); a.vs_sh = bstride(vs, 1); a.vs_sn = bstride(vs, 2);
  if (a.ks_sn > 0x7fffffff || a.vs_sn > 0x7fffffff)
    return fail(SIA_ERR_UNSUPPORTED, "k_scale/v_scale token stride too large");
  a.ks_tok = (uint32_t)a.ks_sn; a.vs_tok = (uint32_t)a.vs_sn;
  if (paged) {
    if (a.ks_s0 > 0xffffffffLL || a.vs_s0 > 0xffffffffLL)
      return fail(SIA_ERR_UNSUPPORTED, "k_scale/v_scale page stride too large");
    a.ks_pg = (uint32_t)a.ks_s0; a.vs_pg = (uint32_t)a.vs_s0;
  }
  L.scale_dtype = ks->dtype;
  // the 4 scales a lane reads per tile form one aligned vector (16 bytes of
  // fp32, 8 of fp16) when the rows are contiguous and every row start is
  // aligned to that size
  const int64_t al = ks->dtype == SIA_F32 ? 16 : 8;
  a.scale_vec = ks->stride[2] == 1 && vs->stride[2] == 1 && (uintptr_t)ks->data % al == 0 &&
                (uintptr_t)vs->data % al == 0 && bstride(ks, 0) % al == 0 && bstride(ks, 1) % al == 0 &&
                bstride(vs, 0) % al == 0 && bstride(vs, 1) % al == 0;
  return SIA_OK;
}

int prepare_table(const sia_tensor* bt, const Geometry& g, int page_size, DecodeLaunch& L) {
  int rc;
  if ((rc = check_tensor(bt, "block_table", 2))) return rc;
  if (bt->dtype != SIA_I32) return fail(SIA_ERR_INVALID_ARGUMENT, "block_table must be int32");
  if (bt->shape[0] < g.B) return fail(SIA_ERR_INVALID_ARGUMENT, "block_table has fewer rows than the batch");
  const int64_t cap = bt->shape[1] * (int64_t)page_size;
  if (cap > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "block table capacity too large");
  DecodeArgs& a = L.a;
  a.bt = (const int32_t*)bt->data; a.bt_sb = bt->stride[0]; a.bt_sl = bt->stride[1];
  a.cap_tokens = (int)cap;
  return SIA_OK;
}

int prepare_workspace(void* ws, size_t bytes, const Geometry& g, const sia_decode_options* opts, DecodeLaunch& L) {
  if (opts != nullptr) {
    bool dirty = opts->reserved0 != 0;
    for (int i = 0; i < 4; ++i) dirty |= opts->reserved[i] != 0;
    if (dirty) return fail(SIA_ERR_INVALID_ARGUMENT, "sia_decode_options reserved fields must be zero");
    if (opts->tiles_per_split < 0) return fail(SIA_ERR_INVALID_ARGUMENT, "tiles_per_split must be >= 0");
    L.begin_event = (hipEvent_t)opts->main_begin_event;
    L.end_event = (hipEvent_t)opts->main_end_event;
  }
  // the work line (B x (tiles + the split's segment charge, at most 4) x unit
  // blocks) is indexed with 32-bit integers
  if ((int64_t)g.B * ((L.a.cap_tokens + kTile - 1) / kTile + 4) * g.UB > 0x7fffffffLL)
    return fail(SIA_ERR_UNSUPPORTED, "batch x cache capacity too large (more than 2^31 tiles of work)");
  const size_t pb = plan_bytes(g.B);
  const size_t ib = item_bytes(g);
  if (ws == nullptr || bytes < pb + ib * 2 || !aligned16(ws))
    return fail(SIA_ERR_WORKSPACE, "decode workspace missing, misaligned or smaller than %zu bytes", pb + ib * 2);
  int64_t items = (int64_t)((bytes - pb) / ib);
  if (items > 0x7fffffff) items = 0x7fffffff;
  DecodeArgs& a = L.a;
  a.ws_plan = (int32_t*)ws;
  a.max_items = (int32_t)items;
  a.ws_ml = (float*)((char*)ws + pb);
  a.ws_acc = a.ws_ml + (size_t)items * decode_waves(g.D) * g.G16 * 2;
  a.tps_force = opts ? opts->tiles_per_split : 0;
  return SIA_OK;
}

// Float32 q or K/V, or pages of a size other than 16 * 2^k: the vector-ALU
// path (attn_f32.hpp), which finds each token's page on its own.  Same
// checked arguments as the MFMA path; the key range is split on the host
// from the cache capacity so that the partials fit the caller's workspace.
int dispatch_f32(const DecodeLaunch& D, const Geometry& g, int kv_dtype, const sia_tensor* out) {
  const DecodeArgs& d = D.a;
  if (!aligned16(out->data) || bstride(out, 0) % 16 || bstride(out, 2) % 16)
    return fail(SIA_ERR_INVALID_ARGUMENT, "out rows must be 16-byte aligned");
  F32Launch L;
  memset(&L, 0, sizeof(L));
  F32Args& a = L.a;
  a.q = d.q; a.q_sb = d.q_sb; a.q_sh = d.q_sh; a.q_sm = 0;
  a.out = d.out; a.o_sb = d.o_sb; a.o_sh = d.o_sh; a.o_sm = 0;
  a.k = d.k; a.k_s0 = d.k_s0; a.k_sh = d.k_sh; a.k_sn = d.k_sn;
  a.v = d.v; a.v_s0 = d.v_s0; a.v_sh = d.v_sh; a.v_sn = d.v_sn;
  a.ks = d.ks; a.ks_s0 = d.ks_s0; a.ks_sh = d.ks_sh; a.ks_sn = d.ks_sn;
  a.vs = d.vs; a.vs_s0 = d.vs_s0; a.vs_sh = d.vs_sh; a.vs_sn = d.vs_sn;
  a.bt = d.bt; a.bt_sb = d.bt_sb; a.bt_sl = d.bt_sl;
  a.num_pages = d.num_pages;
  a.page_size = D.page_size > 0 ? D.page_size : 1;
  a.kv_len = d.kv_len; a.kv_per_seq = d.kv_per_seq;
  a.cap = d.cap_tokens;
  a.B = g.B; a.Hq = g.Hq; a.Hkv = g.Hkv; a.G = g.G; a.Tq = 1; a.Tk = d.cap_tokens; a.causal = 0;
  a.ncol = g.G;
  a.nchunk = (g.G + kF32Cols - 1) / kF32Cols;
  a.qk_scale = d.qk_scale;
  // split: enough items for four per CU, pieces of >= 128 keys (two steps of a
  // work-group: shorter pieces measured slower, longer ones leave small calls
  // to a few work-groups), within the workspace
  const int64_t rows = (int64_t)g.B * g.Hq;
  const int64_t base = (int64_t)g.B * g.Hkv * a.nchunk;
  const int64_t cap = a.cap > 0 ? a.cap : 1;
  int64_t tps;
  if (d.tps_force > 0) {
    tps = (int64_t)d.tps_force * kTile;
  } else {
    const int cus = device_info().cus > 0 ? device_info().cus : 256;
    int64_t want = (4LL * cus + base - 1) / base;
    want = want < 1 ? 1 : want;
    const int64_t most = (cap + 127) / 128;
    if (want > most) want = most;
    tps = (cap + want - 1) / want;
  }
  tps = (tps + kTile - 1) / kTile * kTile;
  int64_t nsplit = (cap + tps - 1) / tps;
  if (nsplit > 1) {
    const size_t room = D.ws_bytes;
    const int64_t fit = (int64_t)(room / f32_partial_bytes(rows, 1, g.D));
    if (fit < 2) {
      nsplit = 1;
    } else if (nsplit > fit) {
      tps = ((cap + fit - 1) / fit + kTile - 1) / kTile * kTile;
      nsplit = (cap + tps - 1) / tps;
    }
  }
  if (nsplit == 1) tps = cap;
  if (tps > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "cache length too large");
  a.nsplit = (int)nsplit;
  a.tps = (int)tps;
  a.part = (float*)D.ws;
  L.D = g.D;
  L.q_dtype = D.q_dtype;
  L.kv_dtype = kv_dtype;
  L.scale_dtype = D.scale_dtype;
  L.stream = D.stream;
  L.begin_event = D.begin_event;
  L.end_event = D.end_event;
  return launch_attn_f32(L);
}

int dispatch(DecodeLaunch& L, int kv_dtype) {
  switch (kv_dtype) {
    case SIA_F16: return launch_decode_f16(L);
    case SIA_BF16: return launch_decode_bf16(L);
    case SIA_I8: return launch_decode_i8(L);
    default: return fail(SIA_ERR_UNSUPPORTED, "k/v dtype %s not supported", dtype_name(kv_dtype));
  }
}

int decode_any(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v, const sia_tensor* ks,
               const sia_tensor* vs, const sia_tensor* bt, const sia_tensor* kv_len, int page_size,
               float sm_scale, const sia_tensor* out, void* ws, size_t ws_bytes,
               const sia_decode_options* opts, void* stream, bool want_int8) {
  DecodeLaunch L;
  memset(&L, 0, sizeof(L));
  Geometry g;
  int rc;
  if (k == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "k is NULL");
  if ((rc = prepare_common(q, kv_len, out, (int)k->shape[1], sm_scale, g, L))) return rc;
  item_units(g, bt != nullptr);
  L.a.IU = g.IU;
  L.a.UB = g.UB;
  if ((rc = prepare_kv(k, v, g, bt != nullptr, page_size, L))) return rc;
  if (want_int8) {
    if (k->dtype != SIA_I8) return fail(SIA_ERR_INVALID_ARGUMENT, "k/v must be int8 for the int8 entry points");
    if ((rc = prepare_scales(ks, vs, k, bt != nullptr, L))) return rc;
  } else if (k->dtype != SIA_F16 && k->dtype != SIA_BF16 && k->dtype != SIA_F32) {
    return fail(SIA_ERR_INVALID_ARGUMENT,
                "k/v must be float16, bfloat16 or float32 (use the int8 entry points for int8)");
  }
  if (bt != nullptr && (rc = prepare_table(bt, g, page_size, L))) return rc;
  if ((rc = prepare_workspace(ws, ws_bytes, g, opts, L))) return rc;
  L.stream = (hipStream_t)stream;
  L.ws = ws;
  L.ws_bytes = ws_bytes;
  // pages that do not hold whole 16-token tiles (page sizes 1-8, or any size
  // other than 16 * 2^k) go to the vector-ALU path with its per-token lookup
  const bool tiled_pages = bt == nullptr || (kTile << L.a.lg_tiles_per_page) == page_size;
  if (q->dtype == SIA_F32 || k->dtype == SIA_F32 || !tiled_pages) return dispatch_f32(L, g, k->dtype, out);
  return dispatch(L, k->dtype);
}

// Split-K workspace of sia_paged_gqa_int8_flash_decode_noalloc: a static
// device array, one copy per GPU, held until the process ends.  Host code
// never passes `scratch` itself (its name is a host-side stand-in, not a
// device address): the device address of each GPU's copy comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t kScratchBytes = (size_t)SIA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64];

// Device address of this GPU's scratch (looked up on its first use).
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(SIA_ERR_DEVICE, "no HIP device is current");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(SIA_ERR_DEVICE, "cannot resolve the static decode scratch on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SIA_OK;
}

}  // namespace

extern "C" {

int sia_abi_version(void) { return SIA_ABI_VERSION; }

const char* sia_status_string(int status) {
  switch (status) {
    case SIA_OK: return "ok";
    case SIA_ERR_INVALID_ARGUMENT: return "invalid argument";
    case SIA_ERR_UNSUPPORTED: return "unsupported";
    case SIA_ERR_WORKSPACE: return "workspace too small";
    case SIA_ERR_LAUNCH: return "launch failed";
    case SIA_ERR_DEVICE: return "device error";
    default: return "unknown status";
  }
}

const char* sia_last_error_message(void) { return sia::last_message(); }

int sia_decode_workspace_size(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                              size_t* bytes) {
  if (bytes == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "bytes is NULL");
  Geometry g;
  int rc = geometry(batch, num_q_heads, num_kv_heads, head_dim, g);
  if (rc) return rc;
  *bytes = plan_bytes(g.B) + item_bytes(g) * (size_t)wanted_items(g);
  return SIA_OK;
}

int sia_attention_flash_decode(const sia_tensor* q, const sia_tensor* k, const sia_tensor* v,
                               const sia_tensor* kv_len, float sm_scale, const sia_tensor* out,
                               void* workspace, size_t workspace_bytes, const sia_decode_options* opts,
                               void* stream) {
  return decode_any(q, k, v, nullptr, nullptr, nullptr, kv_len, 0, sm_scale, out, workspace,
                    workspace_bytes, opts, stream, false);
}

int sia_attention_flash_decode_int8(const sia_tensor* q, const sia_tensor* k_int8, const sia_tensor* v_int8,
                                    const sia_tensor* k_scale, const sia_tensor* v_scale,
                                    const sia_tensor* kv_len, float sm_scale, const sia_tensor* out,
                                    void* workspace, size_t workspace_bytes, const sia_decode_options* opts,
                                    void* stream) {
  return decode_any(q, k_int8, v_int8, k_scale, v_scale, nullptr, kv_len, 0, sm_scale, out, workspace,
                    workspace_bytes, opts, stream, true);
}

int sia_gqa_int8_flash_decode(const sia_tensor* q, const sia_tensor* k_int8, const sia_tensor* v_int8,
                              const sia_tensor* k_scale, const sia_tensor* v_scale, const sia_tensor* kv_len,
                              float sm_scale, const sia_tensor* out, void* workspace, size_t workspace_bytes,
                              const sia_decode_options* opts, void* stream) {
  return decode_any(q, k_int8, v_int8, k_scale, v_scale, nullptr, kv_len, 0, sm_scale, out, workspace,
                    workspace_bytes, opts, stream, true);
}

int sia_paged_attention_flash_decode(const sia_tensor* q, const sia_tensor* k_pool, const sia_tensor* v_pool,
                                     const sia_tensor* block_table, const sia_tensor* kv_len, int32_t page_size,
                                     float sm_scale, const sia_tensor* out, void* workspace,
                                     size_t workspace_bytes, const sia_decode_options* opts, void* stream) {
  if (block_table == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "block_table is NULL");
  return decode_any(q, k_pool, v_pool, nullptr, nullptr, block_table, kv_len, page_size, sm_scale, out,
                    workspace, workspace_bytes, opts, stream, false);
}

int sia_paged_gqa_int8_flash_decode_noalloc(const sia_tensor* q, const sia_tensor* k_pool, const sia_tensor* v_pool,
                                            const sia_tensor* k_scale_pool, const sia_tensor* v_scale_pool,
                                            const sia_tensor* block_table, const sia_tensor* kv_len,
                                            int32_t page_size, float sm_scale, const sia_tensor* out,
                                            const sia_decode_options* opts, void* stream) {
  if (block_table == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "block_table is NULL");
  if (k_pool == nullptr || q == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "q or k_pool is NULL");
  if (q->ndim != 4 || k_pool->ndim != 4) return fail(SIA_ERR_INVALID_ARGUMENT, "q and k_pool must have 4 dims");
  // the split-K partials of at least one work-group per CU must fit the static scratch
  Geometry g;
  int rc = geometry(q->shape[0], q->shape[1], k_pool->shape[1], q->shape[3], g);
  if (rc) return rc;
  const int cus = device_info().cus > 0 ? device_info().cus : 256;
  const size_t need = plan_bytes(g.B) + item_bytes(g) * 2 * (size_t)cus;
  if (need > kScratchBytes)
    return fail(SIA_ERR_WORKSPACE,
                "this geometry needs %zu bytes of split-K scratch; the static scratch of the no-allocation entry "
                "point holds %zu (use sia_paged_gqa_int8_flash_decode with a workspace)",
                need, kScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_for_current_device(&ws))) return rc;
  // nothing in the scratch needs to start at zero: every call writes the plan
  // and each partial slot before reading it
  return decode_any(q, k_pool, v_pool, k_scale_pool, v_scale_pool, block_table, kv_len, page_size, sm_scale, out,
                    ws, kScratchBytes, opts, stream, true);
}

int sia_paged_gqa_int8_flash_decode(const sia_tensor* q, const sia_tensor* k_pool, const sia_tensor* v_pool,
                                    const sia_tensor* k_scale_pool, const sia_tensor* v_scale_pool,
                                    const sia_tensor* block_table, const sia_tensor* kv_len, int32_t page_size,
                                    float sm_scale, const sia_tensor* out, void* workspace,
                                    size_t workspace_bytes, const sia_decode_options* opts, void* stream) {
  if (block_table == nullptr) return fail(SIA_ERR_INVALID_ARGUMENT, "block_table is NULL");
  return decode_any(q, k_pool, v_pool, k_scale_pool, v_scale_pool, block_table, kv_len, page_size, sm_scale,
                    out, workspace, workspace_bytes, opts, stream, true);
}

}  // extern "C"
