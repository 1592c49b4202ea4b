// Paged / contiguous flash-decode for gfx950 (single query per sequence, GQA).
//
// One kernel template serves every decode entry point of the library
// (fp16/bf16 KV, int8 KV with per-token-per-head scales, contiguous or paged,
// one or many split-K items per sequence).  Semantics follow the reference
// kernels: kernels/flash_decode_kernel.py:53-116 (online softmax, l==0 guard),
// kernels/flash_decode_int8_kernel.py:51-118 (scale folding),
// kernels/paged_flash_decode_kernel.py:40-104 (block-table indirection) and
// kernels/paged_flash_decode_int8_gqa_kernel.py:31-97 (one program per KV head
// serving its whole query-head group).
//
// Work decomposition (MI355X-first, not the reference's):
//  * A unit is one KV head and a group of up to 16 of its query heads; the
//    KV of a unit is read once for all of its query heads.  The work of a
//    call is a line of 16-token tiles (sequence-major, then block of units,
//    then tile) whose length W comes from kv_len on the device.  The
//    persistent grid (CUs x occupancy work-groups) splits it stream-K style:
//    each group takes an equal contiguous share, cut into segments at
//    (sequence, unit block) boundaries, so ragged batches stay balanced with
//    no work queue.
//  * Within a segment the group's NW wave64s cover the IU units of an item
//    (IU chosen on the host, smaller for small batches), NW / IU waves per
//    unit splitting its 16-token tiles (double-buffered in registers); each
//    wave runs its own online softmax and the waves' (m, l, acc) states are
//    merged through LDS.  A segment that covers its whole (sequence, unit block) is
//    normalised and written straight to `out`; otherwise it writes an fp32
//    partial and decode_reduce() merges the pieces.
//  * Per tile a wave computes S^T = K Q^T with v_mfma_f32_16x16x32 (tokens as
//    rows, query heads as columns) and O^T += V^T P^T with v_mfma_f32_16x16x16
//    (head_dim as rows), whose B operand layout is exactly the S^T output
//    layout, so P never leaves registers.  int8 K/V are converted to f16
//    exactly in registers; 16-bit K/V feed the MFMA as loaded.  The softmax
//    runs in base 2 on the MFMA output layout: lane (col c, group g) owns head
//    c, tokens 4g..4g+3 of the tile, and head c's output elements
//    [g*D/4, (g+1)*D/4).  The running max is updated lazily: the cross-lane
//    reduction and the rescale of (l, acc) run only when a wave sees a score
//    above its head's current max.
#pragma once

#include "sia_common.hpp"

namespace sia {

constexpr int kTile = 16;          // tokens per MFMA tile
// Plan header in the workspace (ints), written by work-group 0 of decode_main
// for decode_reduce: total work W (tiles x unit blocks), the number G of
// work-groups that share it, the unit blocks per sequence; the work prefix
// per sequence (B+1 ints) follows.
constexpr int kPlanW = 0, kPlanG = 1, kPlanUB = 2, kPlanPen = 3, kPlanHeader = 4;
constexpr int kMinWaveTiles = 2;   // least work per work-group: this many tiles per wave of a unit
// The running max is only raised when a score exceeds it by more than this
// (log2 units), so p = 2^(s - m) <= 2^8: well inside f16/bf16 range, and the
// rescale of (l, acc) almost never runs after the first tile.
constexpr float kLazyMax = 8.0f;

struct DecodeArgs {
  const char* q; int64_t q_sb, q_sh;                 // byte strides
  char* out; int64_t o_sb, o_sh;
  const char* k; int64_t k_s0, k_sh, k_sn;           // s0: batch (contiguous) or page (paged)
  const char* v; int64_t v_s0, v_sh, v_sn;
  const char* ks; int64_t ks_s0, ks_sh, ks_sn;       // int8 scales (nullptr otherwise)
  const char* vs; int64_t vs_s0, vs_sh, vs_sn;
  const int32_t* bt; int64_t bt_sb, bt_sl;           // block table (element strides), nullptr = contiguous
  int64_t num_pages;
  int32_t lg_tiles_per_page;                         // page_size = 16 << lg
  const int32_t* kv_len; int32_t kv_per_seq;
  int32_t cap_tokens;                                // S (contiguous) or max_blocks*page_size
  int32_t B, Hq, Hkv, G, HG, U, UB;                  // U = Hkv*HG units per sequence, UB unit blocks per item row
  int32_t IU;                                        // units per item (NW / IU waves per unit)
  float qk_scale;                                    // sm_scale * log2(e)
  float* ws_acc; float* ws_ml; int32_t* ws_plan; int32_t max_items; int32_t G16;
  int32_t tps_force;
  int32_t seg_pen;                                   // virtual tiles charged to each segment start (the split)
  int32_t slots;                                     // persistent work-groups of decode_main
  int32_t scale_vec;                                 // scale rows allow one vector load per lane
  int32_t direct_only;                               // no decode_reduce follows: empty calls write zeros here
  // 32-bit copies of the per-tile strides (bytes): page strides (0 when
  // contiguous) and token strides, so the tile address needs only 32x32->64
  // products
  uint32_t k_pg, v_pg, ks_pg, vs_pg;
  uint32_t k_tok, v_tok, ks_tok, vs_tok;
};

// --------------------------------------------------------------------- plan

// Batches up to this size keep their per-sequence token counts in LDS after
// the plan (4 bytes each), so a segment's length needs no second global read.
constexpr int kLensInLds = 4096;

__device__ __forceinline__ int seq_tiles(const DecodeArgs& a, int b) {
  int n = a.kv_len[a.kv_per_seq ? b : 0];
  n = n < 0 ? 0 : (n > a.cap_tokens ? a.cap_tokens : n);
  return (n + kTile - 1) / kTile;
}
__device__ __forceinline__ int seq_tokens(const DecodeArgs& a, int b) {
  int n = a.kv_len[a.kv_per_seq ? b : 0];
  return n < 0 ? 0 : (n > a.cap_tokens ? a.cap_tokens : n);
}

// Exclusive scan over the sequences of their work (tiles + pen per nonempty
// sequence, times UB unit blocks) into pre[0..B] (pre[B] = total), in LDS;
// pre[b] holds sequence b's tile count on entry.
template <int NW>
__device__ __forceinline__ void block_scan(const DecodeArgs& a, int* pre, int* red, int UB, int pen) {
  const int T = NW * 64, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (a.B + T - 1) / T;
  const int b0 = tid * per;
  auto work = [&](int nt) { return (nt + (nt > 0 ? pen : 0)) * UB; };
  int local = 0;
  for (int i = 0; i < per; ++i) {
    int b = b0 + i;
    if (b < a.B) local += work(pre[b]);
  }
  int incl = local;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  __syncthreads();
  if (lane == 63) red[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += red[w];
  int run = base + incl - local;
  for (int i = 0; i < per; ++i) {
    int b = b0 + i;
    if (b < a.B) {
      const int cnt = pre[b];
      pre[b] = run;
      run += work(cnt);
    }
  }
  if (tid == T - 1) pre[a.B] = run;
  __syncthreads();
}

// The work line of one call: sequence-major, then unit block, then 16-token
// tile; pre[b] = position of sequence b's first tile (pre[B] = W).  Every
// segment (sequence, unit block) is charged `pen` virtual tiles ahead of its
// tiles (the cost of starting it), so that the equal shares of the split also
// even out the work-groups whose share holds more segment starts.  With equal
// lengths the shares stay aligned to sequence boundaries without the charge,
// and a charge would only move work between the groups of a sequence: there
// pen is 0.  One length for the whole batch has a closed form; per-sequence
// lengths take a block-wide min/max and scan.
template <int NW>
__device__ int plan_work(const DecodeArgs& a, int* pre, int* red, int tok0, int& pen) {
  const int T = NW * 64;
  if (!a.kv_per_seq) {
    pen = 0;
    const int per = ((tok0 + kTile - 1) / kTile) * a.UB;
    for (int b = threadIdx.x; b <= a.B; b += T) pre[b] = b * per;
    __syncthreads();
    return a.B * per;
  }
  int* lens = pre + a.B + 1;                 // token counts, kept for the segments (small batches)
  int nmin = 0x7fffffff, nmax = -1;
  for (int b = threadIdx.x; b < a.B; b += T) {
    const int n = seq_tokens(a, b);
    const int nt = (n + kTile - 1) / kTile;
    pre[b] = nt;
    nmin = min(nmin, nt);
    nmax = max(nmax, nt);
    if (a.B <= kLensInLds) lens[b] = n;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    nmin = min(nmin, __shfl_xor(nmin, o));
    nmax = max(nmax, __shfl_xor(nmax, o));
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { red[wave] = nmin; red[NW + wave] = nmax; }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NW; ++w) { nmin = min(nmin, red[w]); nmax = max(nmax, red[NW + w]); }
  // (read from LDS, so the compiler cannot tell it is the same in every
  // lane: without readfirstlane the tile descriptors derived from it would be
  // taken as divergent and every tile load wrapped in a waterfall loop)
  pen = uniform(nmin == nmax ? 0 : a.seg_pen);
  block_scan<NW>(a, pre, red, a.UB, pen);
  return pre[a.B];
}

// Stream-K split of W tiles over G work-groups: group g takes
// [lo(g), lo(g+1)) with lo(g) = floor(g W / G); the group holding position x
// is ceil((x+1) G / W) - 1.
__device__ __forceinline__ int sk_lo(int g, int W, int G) { return (int)((int64_t)g * W / G); }
__device__ __forceinline__ int sk_group(int x, int W, int G) {
  return (int)(((int64_t)(x + 1) * G + W - 1) / W) - 1;
}

// -------------------------------------------------------------- tile data

// One 16-token tile's operands as held by one lane.
template <int D, class KV, class ST>
struct Tile {
  // K bytes per lane, token lane16: 16 bytes per MFMA k-step j, at bytes
  // [64 j + 16 grp, +16) of the row (elements [32 j + 8 grp, +8) for 16-bit
  // K, [64 j + 16 grp, +16) for int8), the operand's own order, so the 4
  // lanes of a row read 64 contiguous bytes per load instruction.  (A lane
  // owning a contiguous quarter of the row instead made every 16-bit load
  // instruction touch 64 cache lines at 16 bytes each.)
  static constexpr int KB = (D / 4) * KV::bytes;
  static constexpr int KSTRIDE = 64;                                      // bytes between a lane's K pieces
  static constexpr int VB = (D / 16) * KV::bytes;    // V bytes per lane per token (see kVSplit)
  static constexpr bool kInt8 = std::is_same<KV, I8>::value;
  // V of one token: elements [lane16*D/16, +D/16), or, when a lane's share is
  // more than 16 bytes (16-bit V at D = 256), 16-byte pieces 256 bytes apart,
  // elements [128 p + 8 lane16, +8) for piece p, so that one load instruction
  // reads whole 128-byte lines of the row.
  static constexpr bool kVSplit = !kInt8 && VB > 16;
  Raw<KB> k;
  Raw<VB> v[4];                                      // tokens 4*grp + i
  float ks[4], vs[4];                                // int8 scales of tokens 4*grp + i
};

// This lane's byte offsets inside one tile (constant): K of token lane16
// (its first piece; see Tile); V of token 4*grp+i, elements [lane16*D/16,
// +D/16); the scales of tokens 4*grp .. 4*grp+3.
struct LaneOff {
  uint32_t k;
  uint32_t v[4];
  uint32_t ks, vs;
};

// Uniform base addresses of one tile.  Tiles are read with buffer loads: a
// scalar descriptor per tile plus the constant per-lane offsets, so no
// per-tile vector address arithmetic (and no 64-bit address registers).
struct TilePtr {
  const char* k; const char* v; const char* ks; const char* vs;
};

constexpr int kRawBufferFlags = 0x00020000;   // gfx9 raw buffer descriptor word 3 (32-bit data, no swizzle)
constexpr int kLoadNT = 2;                     // buffer-load cache policy: non-temporal (read once)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const char* p) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, -1, kRawBufferFlags);
}

// BYTES at rsrc + off (BYTES a multiple of 16, or 8 or 4); 16-byte pieces
// STRIDE bytes apart.
template <int BYTES, int STRIDE = 16>
__device__ __forceinline__ void load_raw_buf(Raw<BYTES>& r, __amdgpu_buffer_rsrc_t rs, uint32_t off) {
  if constexpr (BYTES % 16 == 0) {
#pragma unroll
    for (int i = 0; i < BYTES / 16; ++i) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, off + STRIDE * i, 0, kLoadNT);
      r.w[4 * i + 0] = x[0]; r.w[4 * i + 1] = x[1]; r.w[4 * i + 2] = x[2]; r.w[4 * i + 3] = x[3];
    }
  } else if constexpr (BYTES == 8) {
    const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kLoadNT);
    r.w[0] = x[0]; r.w[1] = x[1];
  } else {
    static_assert(BYTES == 4, "tile operand size");
    r.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kLoadNT);
  }
}

template <class ST>
__device__ __forceinline__ float load_scale(const char* p) {
  if constexpr (std::is_same<ST, F32>::value) return *(const float*)p;
  else return (float)*(const _Float16*)p;
}
template <class ST>
__device__ __forceinline__ float load_scale(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  if constexpr (std::is_same<ST, F32>::value) return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kLoadNT));
  else return (float)__builtin_bit_cast(_Float16, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, kLoadNT));
}

// Load this lane's operands of one tile.  FULL: all 16 tokens exist, so no
// per-lane predicate; otherwise tokens >= `valid` read as zero.  SV: the
// int8 scales of a head are contiguous rows (one 16-byte load per lane for
// fp32 scales, one 8-byte load for fp16);
// a compile-time choice, so that the tile loop holds no branch around loads
// (a branch there makes the compiler wait for the next tile's loads as well).
template <int D, class KV, class ST, bool FULL, bool SV>
__device__ __forceinline__ void load_tile(const DecodeArgs& a, const TilePtr& t, const LaneOff& o, int valid,
                                          Tile<D, KV, ST>& c, int lane16, int grp) {
  using C = Tile<D, KV, ST>;
  const __amdgpu_buffer_rsrc_t rk = tile_rsrc(t.k), rv = tile_rsrc(t.v);
  if (FULL || lane16 < valid) load_raw_buf<C::KB, C::KSTRIDE>(c.k, rk, o.k);
  else zero_raw<C::KB>(c.k);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (FULL || 4 * grp + i < valid) load_raw_buf<C::VB, C::kVSplit ? 256 : 16>(c.v[i], rv, o.v[i]);
    else zero_raw<C::VB>(c.v[i]);
  }
  if constexpr (C::kInt8) {
    const __amdgpu_buffer_rsrc_t rks = tile_rsrc(t.ks), rvs = tile_rsrc(t.vs);
    if constexpr (FULL && SV && std::is_same<ST, F32>::value) {
      const u32x4 k4 = __builtin_amdgcn_raw_buffer_load_b128(rks, o.ks, 0, kLoadNT);
      const u32x4 v4 = __builtin_amdgcn_raw_buffer_load_b128(rvs, o.vs, 0, kLoadNT);
#pragma unroll
      for (int i = 0; i < 4; ++i) { c.ks[i] = __uint_as_float(k4[i]); c.vs[i] = __uint_as_float(v4[i]); }
    } else if constexpr (FULL && SV) {   // fp16 scale rows: the 4 scales in one 8-byte load
      const u32x2 k2 = __builtin_amdgcn_raw_buffer_load_b64(rks, o.ks, 0, kLoadNT);
      const u32x2 v2 = __builtin_amdgcn_raw_buffer_load_b64(rvs, o.vs, 0, kLoadNT);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c.ks[i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(k2[i >> 1] >> (16 * (i & 1))));
        c.vs[i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(v2[i >> 1] >> (16 * (i & 1))));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = FULL || 4 * grp + i < valid;
        c.ks[i] = ok ? load_scale<ST>(rks, o.ks + i * a.ks_tok) : 0.0f;
        c.vs[i] = ok ? load_scale<ST>(rvs, o.vs + i * a.vs_tok) : 0.0f;
      }
    }
  }
}

// K operand (A of S^T = K Q^T) for k-step j: 8 elements as 4 words.
template <int D, class KV, class ST>
__device__ __forceinline__ u32x4 k_operand(const Tile<D, KV, ST>& c, int j) {
  u32x4 r;
  if constexpr (std::is_same<KV, I8>::value) {
    const uint32_t w0 = c.k.w[2 * j] ^ 0x80808080u;
    const uint32_t w1 = c.k.w[2 * j + 1] ^ 0x80808080u;
    r[0] = i8pair_to_f16x2(w0, 0x04010400u);
    r[1] = i8pair_to_f16x2(w0, 0x04030402u);
    r[2] = i8pair_to_f16x2(w1, 0x04010400u);
    r[3] = i8pair_to_f16x2(w1, 0x04030402u);
  } else {
    r[0] = c.k.w[4 * j + 0];
    r[1] = c.k.w[4 * j + 1];
    r[2] = c.k.w[4 * j + 2];
    r[3] = c.k.w[4 * j + 3];
  }
  return r;
}

// V^T operand (A of O^T += V^T P^T, 16x16x16) for d-tile e: element e of the
// lane's D/16-wide slice for tokens (4g, 4g+1) and (4g+2, 4g+3).
template <int D, class KV, class ST>
__device__ __forceinline__ u32x2 v_operand(const Tile<D, KV, ST>& c, int e) {
  u32x2 r;
  if constexpr (std::is_same<KV, I8>::value) {
    r[0] = i8gather_to_f16x2(c.v[0].w[e >> 2], c.v[1].w[e >> 2], e & 3);
    r[1] = i8gather_to_f16x2(c.v[2].w[e >> 2], c.v[3].w[e >> 2], e & 3);
  } else {
    r[0] = gather16(c.v[0].w[e >> 1], c.v[1].w[e >> 1], e & 1);
    r[1] = gather16(c.v[2].w[e >> 1], c.v[3].w[e >> 1], e & 1);
  }
  return r;
}

// MFMA element type used for the products: f16 for f16 and int8 K/V.
template <class KV> struct MmaOf { using T = F16; };
template <> struct MmaOf<BF16> { using T = BF16; };

// The query needs a hi/lo split only when its precision exceeds the MFMA type's.
template <class KV, class QT>
struct QSplit {
  static constexpr bool value = std::is_same<typename MmaOf<KV>::T, BF16>::value && !std::is_same<QT, BF16>::value;
};

// ------------------------------------------------------------------ kernel

// Per-wave online-softmax state.  Lane (c, g) holds head c; m is replicated
// over g, l is the lane's partial sum, acc[e][i] is O[c][(4g+i)*D/16 + e].
template <int D>
struct WaveState {
  float m;
  float l;
  int sexp;          // int8 only: acc holds O * 2^-sexp (value-scale headroom)
  f32x4 acc[D / 16];
};

template <int D, class KV, class QT, class ST, bool FULL>
__device__ __forceinline__ void compute_tile(const Tile<D, KV, ST>& c, const u32x4* qop, const u32x4* qop_lo,
                                             float qmul, int tile, int ntok, int grp, WaveState<D>& st) {
  using MT = typename MmaOf<KV>::T;
  constexpr int KSTEPS = D / 32;
  constexpr int E = D / 16;
  constexpr bool kInt8 = std::is_same<KV, I8>::value;
  // P enters the PV product in the MFMA type.  bf16 keeps 8 significant bits,
  // so P is split into a bf16 pair (hi + lo, two MFMAs); f16's 11 bits keep
  // the output within the fp16 bar with one (a rounding of 2^-12 relative per
  // weight); int8 V takes P' in f16 (one MFMA).
  constexpr bool kPSplit = !kInt8 && std::is_same<MT, BF16>::value;

  float s[4];
  if constexpr (kInt8) {
    // int8 K against the three int8 query terms (q = step * (hi + mid/254 +
    // lo/254^2), hi and mid in qop, lo in qop_lo): exact integer dot
    // products, no conversion of K
    i32x4 shi = {0, 0, 0, 0}, smid = {0, 0, 0, 0}, slo = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
      const u32x4 ka = {c.k.w[4 * j], c.k.w[4 * j + 1], c.k.w[4 * j + 2], c.k.w[4 * j + 3]};
      shi = mfma16x16x64_i8(ka, qop[j], shi);
      smid = mfma16x16x64_i8(ka, qop[D / 64 + j], smid);
      slo = mfma16x16x64_i8(ka, qop_lo[j], slo);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = __mul24(shi[i], 254) + smid[i];          // |t| < 2^30: exact
      s[i] = __builtin_fmaf((float)t, 254.0f, (float)slo[i]) * (qmul * c.ks[i]);
    }
  } else {
    f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      const u32x4 ka = k_operand<D, KV, ST>(c, j);
      sacc = mfma16x16x32(MT{}, ka, qop[j], sacc);
      if constexpr (QSplit<KV, QT>::value) sacc = mfma16x16x32(MT{}, ka, qop_lo[j], sacc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = sacc[i] * qmul;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (!FULL && tile * kTile + 4 * grp + i >= ntok) s[i] = -INFINITY;
  // Lazy max: the cross-lane reduction and the rescale of (l, acc) run only
  // when some score of this wave exceeds its head's running max.
  const float lmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  float alpha = 1.0f;        // rescales l and acc when the running max grows
  float acc_alpha = 1.0f;    // extra factor for acc alone (int8 value-scale headroom)
  bool rescale = false;
  if (__any(lmax > st.m + kLazyMax)) {
    const float m_new = fmaxf(st.m, wave_max_xor16_32(lmax));
    alpha = fast_exp2(st.m - m_new);
    st.m = m_new;
    rescale = true;
  }
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = fast_exp2(s[i] - st.m);

  u32x2 pop, pop_lo;
  if constexpr (kInt8) {
    // P' = p * s_v * 2^(4-sexp) stays < 2^12: p <= 2^kLazyMax and 2^sexp bounds every s_v seen.
    const float lv = fmaxf(fmaxf(c.vs[0], c.vs[1]), fmaxf(c.vs[2], c.vs[3]));
    if (__any(lv > ldexpf(1.0f, st.sexp))) {
      const float vmax = wave_max_xor16_32(lv);
      const int e_new = max(st.sexp, __builtin_amdgcn_frexp_expf(vmax));
      acc_alpha = ldexpf(1.0f, st.sexp - e_new);
      st.sexp = e_new;
      rescale = true;
    }
    const float rho = ldexpf(16.0f, -st.sexp);
    pop[0] = pack2(F16{}, p[0] * (c.vs[0] * rho), p[1] * (c.vs[1] * rho));
    pop[1] = pack2(F16{}, p[2] * (c.vs[2] * rho), p[3] * (c.vs[3] * rho));
  } else {
    pop[0] = pack2(MT{}, p[0], p[1]);
    pop[1] = pack2(MT{}, p[2], p[3]);
    if constexpr (kPSplit) {
      pop_lo[0] = pack2(MT{}, p[0] - lo_f32(MT{}, pop[0]), p[1] - hi_f32(MT{}, pop[0]));
      pop_lo[1] = pack2(MT{}, p[2] - lo_f32(MT{}, pop[1]), p[3] - hi_f32(MT{}, pop[1]));
    }
  }
  if (rescale) {
    st.l *= alpha;
    const float f = alpha * acc_alpha;
#pragma unroll
    for (int e = 0; e < E; ++e) st.acc[e] *= f;
  }
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const u32x2 va = v_operand<D, KV, ST>(c, e);
    st.acc[e] = mfma16x16x16(MT{}, va, pop, st.acc[e]);
    if constexpr (kPSplit) st.acc[e] = mfma16x16x16(MT{}, va, pop_lo, st.acc[e]);
  }
}

// The query row of a unit as loaded: head col c (lane16), elements
// [grp*D/4, +D/4) as raw 16-bit words (zero for dead columns).
template <int D>
struct QRaw {
  u32x4 w[D / 32];
};
// The query elements in the order of this lane's K elements (see Tile):
// word w holds elements [32 w + 8 grp, +8) for 16-bit K, and for int8 K
// words 2j and 2j+1 hold elements [64 j + 16 grp, +16) (k-step j).
template <int D, class KV>
__device__ __forceinline__ QRaw<D> load_q_raw(const DecodeArgs& a, int b, int hq, bool live, int grp) {
  constexpr bool kInt8 = std::is_same<KV, I8>::value;
  QRaw<D> r;
  const char* qp = a.q + b * a.q_sb + (int64_t)hq * a.q_sh + (kInt8 ? grp * 32 : grp * 16);
#pragma unroll
  for (int w = 0; w < D / 32; ++w) {
    // int8: k-step w/2 covers elements [64 (w/2) + 16 grp, +16) in two words
    const int off = kInt8 ? 128 * (w >> 1) + 16 * (w & 1) : 64 * w;
    r.w[w] = live ? *(const u32x4*)(qp + off) : u32x4{0u, 0u, 0u, 0u};
  }
  return r;
}

// Q operand for a unit from its raw row.  Returns the per-lane score
// multiplier (sm_scale*log2e, times the query's scale step).
template <int D, class KV, class QT>
__device__ __forceinline__ float prep_q(const DecodeArgs& a, const QRaw<D>& raw, u32x4* qop, u32x4* qop_lo) {
  using MT = typename MmaOf<KV>::T;
  constexpr int KSTEPS = D / 32;
  constexpr int PER = D / 4;
  float qf[PER];
#pragma unroll
  for (int w = 0; w < PER / 8; ++w) {
    const u32x4 x = raw.w[w];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qf[8 * w + 2 * i] = lo_f32(QT{}, x[i]);
      qf[8 * w + 2 * i + 1] = hi_f32(QT{}, x[i]);
    }
  }
  float mul = a.qk_scale;
  if constexpr (std::is_same<KV, I8>::value) {
    // int8 K: the query becomes three int8 vectors, q = step * (hi + mid/254
    // + lo/254^2) with step = max|q| / 127 and |hi|, |mid|, |lo| <= 127
    // (error <= step/129032 per element, finer than an f16 query for every
    // element within 2^9 of the max: a few outlier channels cost nothing).
    // Byte order follows the lane's elements, as K's bytes do.  hi and mid
    // go to qop[0, D/64) and qop[D/64, D/32), lo to qop_lo[0, D/64).
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) amax = fmaxf(amax, fabsf(qf[i]));
    amax = wave_max_xor16_32(amax);
    const float inv = amax > 0.f ? 127.0f / amax : 0.f;
    uint32_t hw[PER / 4], mw[PER / 4], lw[PER / 4];
#pragma unroll
    for (int w = 0; w < PER / 4; ++w) {
      uint32_t h4 = 0, m4 = 0, l4 = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y = qf[4 * w + i] * inv;
        const float h = rintf(y);
        const float r = (y - h) * 254.0f;
        const float m = rintf(r);
        const int lo = (int)rintf((r - m) * 254.0f);
        h4 |= ((uint32_t)(int)h & 0xffu) << (8 * i);
        m4 |= ((uint32_t)(int)m & 0xffu) << (8 * i);
        l4 |= ((uint32_t)lo & 0xffu) << (8 * i);
      }
      hw[w] = h4; mw[w] = m4; lw[w] = l4;
    }
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
      qop[j] = u32x4{hw[4 * j], hw[4 * j + 1], hw[4 * j + 2], hw[4 * j + 3]};
      qop[D / 64 + j] = u32x4{mw[4 * j], mw[4 * j + 1], mw[4 * j + 2], mw[4 * j + 3]};
      qop_lo[j] = u32x4{lw[4 * j], lw[4 * j + 1], lw[4 * j + 2], lw[4 * j + 3]};
    }
    return amax > 0.f ? mul * (amax / (127.0f * 254.0f * 254.0f)) : 0.f;
  }
  if constexpr (std::is_same<MT, F16>::value) {
    // Scale the query by a power of two so that max|q| lies in [2^13, 2^14):
    // no f16 overflow, and only elements below 2^-28 of the max lose bits.
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) amax = fmaxf(amax, fabsf(qf[i]));
    amax = wave_max_xor16_32(amax);
    int sh = 0;
    if (amax > 0.f) sh = 14 - __builtin_amdgcn_frexp_expf(amax);
#pragma unroll
    for (int i = 0; i < PER; ++i) qf[i] = ldexpf(qf[i], sh);
    mul = ldexpf(mul, -sh);
  }
#pragma unroll
  for (int j = 0; j < KSTEPS; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x0 = qf[8 * j + 2 * i], x1 = qf[8 * j + 2 * i + 1];
      const uint32_t hi = pack2(MT{}, x0, x1);
      qop[j][i] = hi;
      if constexpr (QSplit<KV, QT>::value)
        qop_lo[j][i] = pack2(MT{}, x0 - lo_f32(MT{}, hi), x1 - hi_f32(MT{}, hi));
    }
  }
  return mul;
}

// Head-dim index of accumulator element (e, i) of a lane in row group g: the
// PV product's d-tile e holds, in output row 4 g + i, the element that lane
// 4 g + i loaded as element e of its V share (see Tile).
template <int D, class KV>
__device__ __forceinline__ int out_d(int g, int i, int e) {
  if constexpr (Tile<D, KV, F32>::kVSplit) return 128 * (e >> 3) + 32 * g + 8 * i + (e & 7);
  else return g * (D / 4) + i * (D / 16) + e;
}

// Waves per SIMD each instantiation is compiled for (its VGPR budget).  A
// work-group is NW = 8 waves, so below 4 waves per SIMD a CU holds one group.
// int8 at D = 64 gets 256 registers too: its int8 query split, scales and
// conversions do not fit 128 without scratch spills.
template <int D, class KV>
struct DecodeWaves {
  static constexpr int value = D <= 64 && !std::is_same<KV, I8>::value ? 4 : (D <= 128 ? 2 : 1);
};

// Geometry of one item inside a work-group of NW waves (all uniform): it
// covers IU units (chosen on the host), and P = NW / IU waves share each unit
// and split its tiles by phase (merged through LDS afterwards; P = 1 writes
// from registers).
struct ItemShape {
  int units;   // units covered by one item (<= NW)
  int P;       // waves per unit
};
template <int NW>
__device__ __forceinline__ ItemShape item_shape(const DecodeArgs& a) {
  ItemShape sh;
  sh.units = a.IU;
  sh.P = NW / a.IU;
  return sh;
}

template <int D, class KV, class QT, class ST, int NW, bool SV>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(DecodeWaves<D, KV>::value)))
void decode_main(const DecodeArgs a) {
  constexpr int E = D / 16;
  constexpr int KSTEPS = D / 32;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // LDS: [acc: NW*G16*D f32][m: NW*G16][l: NW*G16][red: 2*NW+2 ints][pre: B+1 ints][lens: B ints, B <= kLensInLds]
  float* l_acc = (float*)smem;
  float* l_m = l_acc + NW * a.G16 * D;
  float* l_l = l_m + NW * a.G16;
  int* red = (int*)(l_l + NW * a.G16);
  int* pre = red + 2 * NW + 2;

  const ItemShape shape = item_shape<NW>(a);
  // The work line (every work-group computes the same prefix) and its
  // stream-K split: group g takes an equal contiguous share, so groups finish
  // together whatever the lengths, with no queue or atomics.  Group 0 records
  // the split for decode_reduce.
  const int tok0 = a.kv_per_seq ? 0 : uniform(seq_tokens(a, 0));
  int pen = 0;
  const int W = plan_work<NW>(a, pre, red, tok0, pen);
  int G = (int)gridDim.x;
  if (a.tps_force > 0) G = min(G, max(1, (W + a.tps_force - 1) / a.tps_force));   // forced share (tests)
  // least work per group, but never fewer groups than (sequence, unit block)
  // segments: those are independent, and a group walking several short ones
  // pays each one's chain of dependent loads in turn (B1 x 16 tokens: 8
  // segments on one group took ~50 us)
  G = min(G, max(a.B * a.UB, (W + kMinWaveTiles * shape.P - 1) / (kMinWaveTiles * shape.P)));
  G = min(G, max(1, a.max_items / 2));                      // two partial slots per group
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i <= a.B; i += NW * 64) a.ws_plan[kPlanHeader + i] = pre[i];
    if (threadIdx.x == 0) {
      a.ws_plan[kPlanW] = W;
      a.ws_plan[kPlanG] = G;
      a.ws_plan[kPlanUB] = a.UB;
      a.ws_plan[kPlanPen] = pen;
    }
  }
  if (a.direct_only && W == 0) {
    // one shared length of zero, and no merge kernel follows: every output
    // row is zero (the l == 0 guard), written here as 4-byte words
    const int64_t words = (int64_t)a.B * a.Hq * (D / 2);
    for (int64_t i = (int64_t)blockIdx.x * (NW * 64) + threadIdx.x; i < words; i += (int64_t)gridDim.x * (NW * 64)) {
      const int64_t row = i / (D / 2);
      const int wd = (int)(i - row * (D / 2));
      const int bb = (int)(row / a.Hq), hh = (int)(row - (int64_t)bb * a.Hq);
      *(uint32_t*)(a.out + bb * a.o_sb + (int64_t)hh * a.o_sh + 4 * wd) = 0u;
    }
    return;
  }
  const int g = blockIdx.x;
  const int x_hi = g < G ? sk_lo(g + 1, W, G) : 0;
  int x = g < G ? sk_lo(g, W, G) : 0;
  int* prog = red + 2;   // tiles done per wave (NW ints; read and written without barriers)

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane16 = lane & 15, grp = lane >> 4;
  using TileT = Tile<D, KV, ST>;
  LaneOff lo;
  lo.k = lane16 * a.k_tok + (uint32_t)(grp * 16);
#pragma unroll
  for (int i = 0; i < 4; ++i) lo.v[i] = (4 * grp + i) * a.v_tok + (uint32_t)(lane16 * (TileT::kVSplit ? 16 : TileT::VB));
  lo.ks = 4 * grp * a.ks_tok;
  lo.vs = 4 * grp * a.vs_tok;
  const int uin = wave / shape.P;        // unit slot of this wave inside an item
  const int phase = wave - uin * shape.P;

  // Segments: the maximal pieces of [x, x_hi) inside one (sequence, unit
  // block).  A segment that covers its whole (b, ublk) is written straight to
  // `out`; a piece writes a partial to slot 2g (the group's first segment) or
  // 2g+1 (its last), which decode_reduce finds from the same split.
  //
  // The segment starting at xs: b is the largest index with pre[b] <= xs.
  // (A batch-wide length was read once already; per-sequence ones were kept
  // in LDS by the plan for batches up to kLensInLds, else are read again.)
  // The line holds each segment as pen virtual tiles (the cost of starting
  // it: a few dependent memory round trips) followed by its ntile tiles; a
  // piece of the virtual span maps to real tiles [t_lo, t_hi).
  struct SegAt {
    int b, ntok, ntile, ublk, t_lo, t_hi, seg_end;
  };
  auto seg_at = [&](int xs) {
    SegAt s;
    int blo = 0, bhi = a.B;
    while (bhi - blo > 1) { const int mid = (blo + bhi) >> 1; if (pre[mid] <= xs) blo = mid; else bhi = mid; }
    s.b = uniform(blo);
    s.ntok = a.kv_per_seq ? uniform(a.B <= kLensInLds ? pre[a.B + 1 + s.b] : seq_tokens(a, s.b)) : tok0;
    s.ntile = (s.ntok + kTile - 1) / kTile;
    const int nvt = s.ntile + pen;
    const int rem = uniform(xs - pre[s.b]);
    s.ublk = rem / nvt;
    const int r_lo = rem - s.ublk * nvt;
    s.seg_end = min(x_hi, pre[s.b] + (s.ublk + 1) * nvt);
    const int r_hi = r_lo + (s.seg_end - xs);
    s.t_lo = max(0, r_lo - pen);
    s.t_hi = max(0, r_hi - pen);
    return s;
  };
  // The next segment's query row and first page id are loaded while the
  // current one streams (seg_next: the start of the segment they belong
  // to), so that a segment change waits for its first tile only.
  QRaw<D> q_next;
  int pg_next = 0, seg_next = -1;
  bool first_seg = true;
  while (x < x_hi) {
    const SegAt sg = seg_at(x);
    const int b = sg.b, ntok = sg.ntok, ntile = sg.ntile, ublk = sg.ublk, t_lo = sg.t_lo, t_hi = sg.t_hi;
    const int seg_end = sg.seg_end;
    if (t_hi == t_lo) {        // only the start cost of a segment, at the end of the share
      x = seg_end;
      continue;
    }
    const bool direct = t_lo == 0 && t_hi == ntile;
    const int pslot_id = first_seg ? 2 * g : 2 * g + 1;
    const int unit = ublk * shape.units + uin;
    const bool wave_live = uin < shape.units && unit < a.U;
    const int hkv = unit / a.HG, hg = unit - hkv * a.HG;
    const int nh = wave_live ? min(16, a.G - 16 * hg) : 0;    // live head columns of this wave's unit
    const bool live = lane16 < nh;
    const int hq = live ? hkv * a.G + 16 * hg + lane16 : 0;

    WaveState<D> st;
    st.m = -INFINITY; st.l = 0.f; st.sexp = -100;
#pragma unroll
    for (int e = 0; e < E; ++e) st.acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (wave_live) {
      // This wave takes tiles t_lo + phase, + P, ...: `nfull` full tiles
      // (double-buffered) and possibly the sequence's partial last tile.
      const int P = shape.P;
      const bool paged = a.bt != nullptr;
      const int t_first = t_lo + phase;
      // Page ids come from the block-table row of sequence b; a contiguous
      // cache reads kv_len[0] instead (value ignored, page stride 0).
      const int32_t* btrow = paged ? a.bt + (int64_t)b * a.bt_sb : a.kv_len;
      const int64_t bt_step = paged ? a.bt_sl : 0;
      const int cap_tiles = a.cap_tokens / kTile;
      auto page_id = [&](int k) {
        const int t = min(t_first + k * P, cap_tiles - 1);
        return uniform(btrow[(int64_t)(t >> a.lg_tiles_per_page) * bt_step]);
      };
      // The loads that need only the item go out together: the query row
      // and the first tile's page id (the length is already in flight),
      // unless the previous segment loaded them already.
      QRaw<D> qraw;
      int pg0;
      if (x == seg_next) {
        qraw = q_next;
        pg0 = pg_next;
      } else {
        qraw = load_q_raw<D, KV>(a, b, hq, live, grp);
        pg0 = page_id(0);
      }
      // the next segment of the share, if this wave has a unit there: its
      // query row and first page id (issued behind this segment's first tile)
      auto prefetch_next = [&]() {
        if (seg_end >= x_hi) return;
        const SegAt nx = seg_at(seg_end);
        const int unit_n = nx.ublk * shape.units + uin;
        if (nx.t_hi == nx.t_lo || unit_n >= a.U) return;
        const int hkv_n = unit_n / a.HG, hg_n = unit_n - hkv_n * a.HG;
        const bool live_n = lane16 < min(16, a.G - 16 * hg_n);
        const int hq_n = live_n ? hkv_n * a.G + 16 * hg_n + lane16 : 0;
        q_next = load_q_raw<D, KV>(a, nx.b, hq_n, live_n, grp);
        const int32_t* btrow_n = paged ? a.bt + (int64_t)nx.b * a.bt_sb : a.kv_len;
        const int tn = min(nx.t_lo + phase, cap_tiles - 1);
        pg_next = uniform(btrow_n[(int64_t)(tn >> a.lg_tiles_per_page) * bt_step]);
        seg_next = seg_end;
      };
      const int t_full = min(t_hi, ntok / kTile);
      const int nfull = t_first < t_full ? (t_full - t_first + P - 1) / P : 0;
      const int nt = t_first < t_hi ? (t_hi - t_first + P - 1) / P : 0;
      const int64_t rowk = paged ? 0 : (int64_t)b * a.k_s0, rowv = paged ? 0 : (int64_t)b * a.v_s0;
      const int64_t rowks = paged ? 0 : (int64_t)b * a.ks_s0, rowvs = paged ? 0 : (int64_t)b * a.vs_s0;
      const char* kb = a.k + (rowk + (int64_t)hkv * a.k_sh);
      const char* vb = a.v + (rowv + (int64_t)hkv * a.v_sh);
      const char* ksb = a.ks + (rowks + (int64_t)hkv * a.ks_sh);
      const char* vsb = a.vs + (rowvs + (int64_t)hkv * a.vs_sh);
      // Tile t lives at page `phys`, token (t & mask) * 16 of it.  A
      // contiguous cache is one page of unbounded length (page stride 0), so
      // both layouts share one branch-free formula.
      const int tpp_mask = paged ? (1 << a.lg_tiles_per_page) - 1 : 0x7fffffff;
      const uint32_t npages = paged ? (uint32_t)min(a.num_pages, (int64_t)0x7fffffff) : 1u;
      auto tile_ptr = [&](int t, int phys) {
        TilePtr tp;
        const uint32_t pg = (uint32_t)phys < npages ? (uint32_t)phys : 0u;   // never read outside the pool
        const uint32_t off = (uint32_t)((t & tpp_mask) * kTile);
        tp.k = kb + uniform64((uint64_t)pg * a.k_pg + (uint64_t)off * a.k_tok);
        tp.v = vb + uniform64((uint64_t)pg * a.v_pg + (uint64_t)off * a.v_tok);
        if constexpr (TileT::kInt8) {
          tp.ks = ksb + uniform64((uint64_t)pg * a.ks_pg + (uint64_t)off * a.ks_tok);
          tp.vs = vsb + uniform64((uint64_t)pg * a.vs_pg + (uint64_t)off * a.vs_tok);
        } else {
          tp.ks = tp.vs = nullptr;
        }
        return tp;
      };
      u32x4 qop[KSTEPS], qop_lo[KSTEPS];
      float qmul = 0.f;
      // Full tiles, double-buffered.  The steady-state loop always issues the
      // next tiles' loads, and fetches the page ids of the tiles two ahead
      // with one vector load (lanes 0 and 1; indices clamped to the wave's
      // last tile, the partial one included), so every load retires in order
      // and computing tile k waits only for tile k.
      int pg_last = pg0;   // page of the wave's partial last tile (tile nfull)
      if (nfull > 0) {
        const int klast = nt > nfull ? nfull : nfull - 1;
        auto page_pair = [&](int k0) {
          const int k = min(k0 + (lane & 1), klast);
          const int t = t_first + k * P;
          return btrow[(int64_t)(t >> a.lg_tiles_per_page) * bt_step];
        };
        TileT bufA, bufB;
        // same load order as the loop below (page ids, then a tile), so the
        // wait counts where the two paths meet stay exact
        int pgv = page_pair(1);   // tiles k + 1, k + 2
        load_tile<D, KV, ST, true, SV>(a, tile_ptr(t_first, pg0), lo, 16, bufA, lane16, grp);
        prefetch_next();
        // the query's conversion overlaps the first tile's flight
        qmul = prep_q<D, KV, QT>(a, qraw, qop, qop_lo);
        int k = 0;
        for (; k + 2 < nfull; k += 2) {
          // With 8 waves, waves w and w^4 share a SIMD, where the older one
          // wins issue ties and would finish well ahead: the one that is
          // behind (by tile count, published in LDS) takes the higher
          // priority.  (A 4-wave group has one wave per SIMD.)
          if constexpr (NW == 8) {
            __hip_atomic_store(&prog[wave], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);   // every lane, same value
            if (k > uniform(__hip_atomic_load(&prog[wave ^ 4], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)))
              __builtin_amdgcn_s_setprio(0);
            else
              __builtin_amdgcn_s_setprio(1);
          }
          const int pg1 = __builtin_amdgcn_readlane(pgv, 0), pg2 = __builtin_amdgcn_readlane(pgv, 1);
          load_tile<D, KV, ST, true, SV>(a, tile_ptr(t_first + (k + 1) * P, pg1), lo, 16, bufB, lane16, grp);
          pgv = page_pair(k + 3);
          compute_tile<D, KV, QT, ST, true>(bufA, qop, qop_lo, qmul, 0, ntok, grp, st);
          load_tile<D, KV, ST, true, SV>(a, tile_ptr(t_first + (k + 2) * P, pg2), lo, 16, bufA, lane16, grp);
          compute_tile<D, KV, QT, ST, true>(bufB, qop, qop_lo, qmul, 0, ntok, grp, st);
        }
        if constexpr (NW == 8) {
          __builtin_amdgcn_s_setprio(0);
          __hip_atomic_store(&prog[wave], 1 << 30, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        // pgv holds the pages of tiles k + 1 and k + 2 (clamped); the partial
        // tile, if any, is tile nfull = k + 1 or k + 2
        pg_last = __builtin_amdgcn_readlane(pgv, nfull - k - 1);
        if (k + 1 < nfull) {
          load_tile<D, KV, ST, true, SV>(a, tile_ptr(t_first + (k + 1) * P, __builtin_amdgcn_readlane(pgv, 0)), lo,
                                         16, bufB, lane16, grp);
          compute_tile<D, KV, QT, ST, true>(bufA, qop, qop_lo, qmul, 0, ntok, grp, st);
          compute_tile<D, KV, QT, ST, true>(bufB, qop, qop_lo, qmul, 0, ntok, grp, st);
        } else {
          compute_tile<D, KV, QT, ST, true>(bufA, qop, qop_lo, qmul, 0, ntok, grp, st);
        }
      } else {
        prefetch_next();
        qmul = prep_q<D, KV, QT>(a, qraw, qop, qop_lo);
      }
      if (nt > nfull) {  // the sequence's partial last tile belongs to this wave
        const int t = t_first + nfull * P;
        TileT last;
        load_tile<D, KV, ST, false, false>(a, tile_ptr(t, pg_last), lo, ntok - t * kTile, last, lane16, grp);
        compute_tile<D, KV, QT, ST, false>(last, qop, qop_lo, qmul, t, ntok, grp, st);
      }
    }

    const float lsum = wave_sum_xor16_32(st.l);
    const float unscale = std::is_same<KV, I8>::value ? ldexpf(1.0f, st.sexp - 4) : 1.0f;
    // partial slot of (segment, unit slot, head col)
    const int64_t pslot = ((int64_t)pslot_id * NW + uin) * a.G16;
    if (shape.P == 1) {
      // one wave owns each unit: write straight from registers
      if (live) {
        if (direct) {
          const float inv = unscale / (lsum == 0.f ? 1.f : lsum);
          char* op = a.out + b * a.o_sb + (int64_t)hq * a.o_sh;
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < E; e += 2) {
              const uint32_t w = pack2(QT{}, st.acc[e][i] * inv, st.acc[e + 1][i] * inv);
              *(uint32_t*)(op + out_d<D, KV>(grp, i, e) * 2) = w;
            }
        } else {
          float* dst = a.ws_acc + (pslot + lane16) * D;
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < E; e += 4)
              *(f32x4*)(dst + out_d<D, KV>(grp, i, e)) = f32x4{st.acc[e][i] * unscale, st.acc[e + 1][i] * unscale,
                                                 st.acc[e + 2][i] * unscale, st.acc[e + 3][i] * unscale};
          if (grp == 0) {
            a.ws_ml[(pslot + lane16) * 2 + 0] = st.m;
            a.ws_ml[(pslot + lane16) * 2 + 1] = lsum;
          }
        }
      }
    } else {
      // P waves per unit: merge their (m, l, acc) through LDS
      if (live) {
        float* dst = l_acc + (wave * a.G16 + lane16) * D;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < E; ++e) dst[out_d<D, KV>(grp, i, e)] = st.acc[e][i] * unscale;
      }
      if (lane16 < a.G16 && grp == 0) {
        l_m[wave * a.G16 + lane16] = live ? st.m : -INFINITY;
        l_l[wave * a.G16 + lane16] = live ? lsum : 0.f;
      }
      __syncthreads();
      const int nh_all = min(16, a.G);                 // head columns per unit (same for every unit here)
      for (int idx = threadIdx.x; idx < shape.units * nh_all * D; idx += NW * 64) {
        const int us = idx / (nh_all * D);
        const int r2 = idx - us * nh_all * D;
        const int cc = r2 / D, d = r2 - cc * D;
        const int u2 = ublk * shape.units + us;
        // the last unit block of a geometry whose IU does not divide U has
        // slots past the last unit: they own no output row
        if (u2 >= a.U) continue;
        const int hkv2 = u2 / a.HG, hg2 = u2 - hkv2 * a.HG;
        if (16 * hg2 + cc >= a.G) continue;
        float M = -INFINITY;
        for (int p2 = 0; p2 < shape.P; ++p2) M = fmaxf(M, l_m[(us * shape.P + p2) * a.G16 + cc]);
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
          for (int p2 = 0; p2 < shape.P; ++p2) {
            const int w2 = us * shape.P + p2;
            const float mw = l_m[w2 * a.G16 + cc];
            const float wt = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
            L += wt * l_l[w2 * a.G16 + cc];
            A += wt * l_acc[(w2 * a.G16 + cc) * D + d];
          }
        }
        const int hqo = hkv2 * a.G + 16 * hg2 + cc;
        if (direct) {
          char* op = a.out + b * a.o_sb + (int64_t)hqo * a.o_sh + d * (int)sizeof(uint16_t);
          store_out(QT{}, op, A / (L == 0.f ? 1.f : L));
        } else {
          const int64_t ps = ((int64_t)pslot_id * NW + us) * a.G16 + cc;
          a.ws_acc[ps * D + d] = A;
          if (d == 0) { a.ws_ml[ps * 2 + 0] = M; a.ws_ml[ps * 2 + 1] = L; }
        }
      }
    }
    if (shape.P > 1) __syncthreads();   // merge LDS free for reuse
    x = seg_end;
    first_seg = false;
  }
}

// Merge split-K partials: each (sequence, query head) row is handled by D/4
// lanes holding 4 outputs each (16-byte partial loads), so a wave merges
// 64/(D/4) rows.  A row's pieces are merged online, up to kRedBatch at a
// time (the batch is sized to the wave's remaining piece count): every lane
// loads the batch's (m, l) pairs and its slices of their partials together
// (one memory round trip per batch; the merge is latency-bound, a few MB
// spread over few rows), rescales its running (M, L, acc) to the batch's max
// and adds the pieces with weights 2^(m_s - M).  Loop bounds
// are uniform over the wave (the largest piece count of its rows).  Rows of
// sequences the main kernel wrote directly are skipped; empty sequences are
// written as zeros.
//
// PW waves share a work-group's rows: wave w merges the w-th of PW
// contiguous runs of the pieces, and wave 0 merges the PW states through
// LDS.  PW = 1 when the rows fill the GPU by themselves; a small batch (few
// rows, each split over up to a few hundred work-groups) uses PW = 8, which
// cuts a row's chain of dependent round trips by 8.
constexpr int kRedBatch = 16;

template <int D, class OT, int NW, int PW>
__global__ __launch_bounds__(PW * 64) void decode_reduce(const DecodeArgs a) {
  constexpr int LPR = D / 4;          // lanes per row
  constexpr int RPW = 64 / LPR;       // rows per work-group
  const int lane = threadIdx.x & 63;
  const int wave = PW > 1 ? uniform(threadIdx.x >> 6) : 0;
  const int li = lane % LPR;
  const int row = blockIdx.x * RPW + lane / LPR;
  const bool inr = row < a.B * a.Hq;
  // the plan's header and this row's prefix entries in one round trip
  // (loaded before any test of them, for rows past the end as well)
  const int b = (inr ? row : 0) / a.Hq;
  const int hq = (inr ? row : 0) - b * a.Hq;
  const int pb = a.ws_plan[kPlanHeader + b], pe = a.ws_plan[kPlanHeader + b + 1];
  const int W = a.ws_plan[kPlanW], G = a.ws_plan[kPlanG], pen = a.ws_plan[kPlanPen];
  // pieces of this row's (sequence, unit block): one per work-group in
  // [gf, gf + nsplit); the first group's piece is its first segment (slot
  // 2g) only if the range starts exactly at the group's start
  int nsplit = 1, gf = 0, s_first = 0, uin = 0, cc = 0;
  if (inr) {
    const int nvt = (pe - pb) / a.UB;                // virtual tiles per unit block (0: empty sequence)
    const int hkv = hq / a.G, gi = hq - hkv * a.G;
    cc = gi & 15;
    const int unit = hkv * a.HG + (gi >> 4);
    const ItemShape shape = item_shape<NW>(a);
    const int ublk = unit / shape.units;
    uin = unit - ublk * shape.units;
    if (nvt == 0) {
      nsplit = 0;                                   // empty sequence: zeros
    } else {
      // the segment spans virtual [v0, v0 + nvt); its tiles are the part
      // after the first pen positions, held by groups gf .. (pieces); the
      // piece of gf is that group's first segment unless gf started before v0
      const int v0 = pb + ublk * nvt;
      gf = sk_group(v0 + pen, W, G);
      nsplit = sk_group(v0 + nvt - 1, W, G) - gf + 1;
      s_first = sk_lo(gf, W, G) < v0 ? 1 : 0;
    }
  }
  const bool work = inr && nsplit != 1;
  int nmax = work ? nsplit : 0;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) nmax = max(nmax, __shfl_xor(nmax, o));
  // (the same rows in every wave: the whole work-group leaves together)
  if (!__any(work)) return;   // (wave-uniform) nothing to merge or zero here
  auto slot = [&](int s) {
    const int id = 2 * (gf + s) + (s == 0 ? s_first : 0);
    return ((int64_t)id * NW + uin) * a.G16 + cc;
  };
  // this wave's run of pieces [sb, se) (uniform); a lane merges those below
  // its own count
  const int chunk = (nmax + PW - 1) / PW;
  const int sb = min(nmax, wave * chunk), se = min(nmax, sb + chunk);
  const int lim = min(nsplit, se);
  float M = -INFINITY, L = 0.f;
  f32x4 A = {0.f, 0.f, 0.f, 0.f};
  // Merge pieces [s0, s0 + K) below lim.  Every load is issued: a piece at
  // or past lim reads the row's first piece and a lane with no merge to do
  // reads slot 0 (one address per instruction), and both are masked once
  // loaded.
  auto batch = [&](int s0, auto kk) {
    constexpr int K = decltype(kk)::value;
    float m[K], l[K];
    f32x4 x[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int64_t sl = work ? slot(s0 + k < lim ? s0 + k : 0) : 0;
      const float2 ml = *(const float2*)(a.ws_ml + sl * 2);
      m[k] = ml.x;
      l[k] = ml.y;
      x[k] = *(const f32x4*)(a.ws_acc + sl * D + 4 * li);
    }
    __builtin_amdgcn_sched_barrier(0);   // all of the batch's loads before the first use
    float mb = M;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (!(work && s0 + k < lim)) m[k] = -INFINITY;
      mb = fmaxf(mb, m[k]);
    }
    // branch-free, so that no load is moved behind a test of the maxima:
    // 2^-inf = 0 weighs out masked pieces and the empty state (M = -inf)
    const float mref = mb == -INFINITY ? 0.f : mb;
    const float r = fast_exp2(M - mref);
    L *= r;
    A *= r;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float w = fast_exp2(m[k] - mref);
      L += w * l[k];
      A += w * x[k];
    }
    M = mb;
  };
  for (int s0 = sb; s0 < se; s0 += kRedBatch) {
    const int rem = se - s0;   // wave-uniform
    if (rem <= 2) batch(s0, std::integral_constant<int, 2>{});
    else if (rem <= 4) batch(s0, std::integral_constant<int, 4>{});
    else if (rem <= 8) batch(s0, std::integral_constant<int, 8>{});
    else batch(s0, std::integral_constant<int, kRedBatch>{});
  }
  if constexpr (PW > 1) {
    // states of waves 1 .. PW-1, merged by wave 0 (an empty run is M = -inf,
    // L = 0, A = 0 and weighs out)
    __shared__ f32x4 s_a[PW - 1][64];
    __shared__ float s_m[PW - 1][64], s_l[PW - 1][64];
    if (wave > 0) {
      s_a[wave - 1][lane] = A;
      s_m[wave - 1][lane] = M;
      s_l[wave - 1][lane] = L;
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < PW - 1; ++w) {
      const float mw = s_m[w][lane];
      const float mb = fmaxf(M, mw);
      const float mref = mb == -INFINITY ? 0.f : mb;
      const float r0 = fast_exp2(M - mref), r1 = fast_exp2(mw - mref);
      L = L * r0 + s_l[w][lane] * r1;
      A = A * r0 + s_a[w][lane] * r1;
      M = mb;
    }
  }
  if (!work) return;
  const float inv = 1.0f / (L == 0.f ? 1.f : L);
  char* op = a.out + b * a.o_sb + (int64_t)hq * a.o_sh + 4 * li * (int)sizeof(uint16_t);
  *(uint32_t*)op = pack2(OT{}, A[0] * inv, A[1] * inv);
  *(uint32_t*)(op + 4) = pack2(OT{}, A[2] * inv, A[3] * inv);
}

}  // namespace sia
