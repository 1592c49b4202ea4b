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
//  * A work item is (sequence b, split s, unit u) where a unit is one KV head
//    and a group of up to 16 of its query heads.  Each item covers
//    `tps` 16-token tiles of the sequence; `tps` is chosen on the device from
//    kv_len so that the persistent grid (CUs x occupancy work-groups) gets an
//    even share (plan_items below).  The KV of a unit is read once for all of
//    its query heads.
//  * A work-group of NW wave64s takes items round-robin.  Its waves split the
//    item's 16-token tiles (double-buffered in registers); each wave runs its
//    own online softmax and the waves' (m, l, acc) states are merged through
//    LDS.  A sequence that fits one item is normalised and written straight to
//    `out`; otherwise the item writes an fp32 partial and decode_reduce()
//    merges the splits.
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
// Plan header in the workspace (ints): split size, item count, unit blocks per
// (sequence, split), the work counter; the item prefix per sequence follows.
constexpr int kPlanTps = 0, kPlanTotal = 1, kPlanUB = 2, kPlanCounter = 3, kPlanHeader = 4;
constexpr int kTpsMin = 8;         // smallest split, in tiles
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
  float qk_scale;                                    // sm_scale * log2(e)
  float* ws_acc; float* ws_ml; int32_t* ws_plan; int32_t max_items; int32_t G16;
  int32_t tps_force;
  int32_t slots;                                     // persistent work-groups of decode_main
  int32_t scale_vec;                                 // scale rows allow 16-byte vector loads
};

// --------------------------------------------------------------------- plan

__device__ __forceinline__ int seq_tiles(const DecodeArgs& a, int b) {
  int n = a.kv_len[a.kv_per_seq ? b : 0];
  n = n < 0 ? 0 : (n > a.cap_tokens ? a.cap_tokens : n);
  return (n + kTile - 1) / kTile;
}
__device__ __forceinline__ int seq_tokens(const DecodeArgs& a, int b) {
  int n = a.kv_len[a.kv_per_seq ? b : 0];
  return n < 0 ? 0 : (n > a.cap_tokens ? a.cap_tokens : n);
}

// Block-wide reductions over NW waves (red: LDS scratch of >= 2*NW ints).
template <int NW>
__device__ __forceinline__ void block_sum_max(long long& sum, int& mx, int* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int s_lo = (int)sum;  // per-thread partials stay < 2^31 (tiles * units per thread)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    s_lo += __shfl_xor(s_lo, o);
    mx = max(mx, __shfl_xor(mx, o));
  }
  __syncthreads();
  if (lane == 0) { red[wave] = s_lo; red[NW + wave] = mx; }
  __syncthreads();
  long long t = 0; int m = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) { t += red[w]; m = max(m, red[NW + w]); }
  sum = t; mx = m;
}

// Exclusive scan of cnt[0..B) into pre[0..B] (pre[B] = total), in LDS.
template <int NW>
__device__ __forceinline__ void block_scan(const DecodeArgs& a, int tps, int* pre, int* red, int UB) {
  const int T = NW * 64, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (a.B + T - 1) / T;
  const int b0 = tid * per;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    int b = b0 + i;
    if (b < a.B) local += ((pre[b] + tps - 1) / tps) * UB;
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
      run += ((cnt + tps - 1) / tps) * UB;
    }
  }
  if (tid == T - 1) pre[a.B] = run;
  __syncthreads();
}

// Decide tiles-per-split from the device-side lengths and build the item
// prefix (items of sequence b are pre[b] .. pre[b+1]-1, split-major).
//
// Items are taken round-robin by the `gridDim.x` persistent work-groups, so a
// split of t tiles finishes in about ceil(items / slots) * (t + overhead).
// Thread c evaluates "split the longest sequence c+1 ways" and the cheapest
// candidate wins (ties go to the larger split, i.e. fewer partials).  With
// equal lengths this finds the exact balance; with ragged lengths it keeps
// the heaviest slot close to the mean.
template <int NW>
__device__ int plan_items(const DecodeArgs& a, int* pre, int* red, int& tps_out, int quantum, int UB, int slots) {
  const int T = NW * 64;
  // quantum: every wave sharing a unit gets the same number of tiles
  constexpr int kItemOverhead = 8;   // per-item fixed cost, in tiles
  // lengths (in tiles) into pre[] temporarily, and the longest
  int mx = 0;
  for (int b = threadIdx.x; b < a.B; b += T) {
    const int t = seq_tiles(a, b);
    pre[b] = t;
    mx = max(mx, t);
  }
  long long dummy = 0;
  block_sum_max<NW>(dummy, mx, red);
  int tps;
  if (a.tps_force > 0) {
    tps = a.tps_force;
  } else {
    // candidate c = threadIdx.x / 8 + 1 splits of the longest sequence; the 8
    // threads of a candidate sum the item counts of every 8th sequence
    static_assert(NW * 64 >= 8, "need at least 8 threads");
    const int c = threadIdx.x / 8 + 1, j = threadIdx.x & 7;
    int t = (mx + c - 1) / c;
    t = max(t, kTpsMin);
    t = (t + quantum - 1) / quantum * quantum;
    long long items = 0;
    for (int b = j; b < a.B; b += 8) items += (pre[b] + t - 1) / t;
    items += __shfl_xor(items, 1);
    items += __shfl_xor(items, 2);
    items += __shfl_xor(items, 4);
    items *= UB;
    constexpr long long kInf = (1LL << 36) - 1;
    long long cost = (items + slots - 1) / slots * (long long)(t + kItemOverhead);
    if (items > a.max_items || cost > kInf) cost = kInf;
    // arg-min over the block of (cost, -t): ties prefer the larger split
    unsigned long long k = ((unsigned long long)cost << 27) | (unsigned long long)(0x7ffffff - t);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const unsigned long long y = __shfl_xor(k, o);
      k = y < k ? y : k;
    }
    __syncthreads();
    unsigned long long* red64 = (unsigned long long*)red;   // NW 8-byte slots (red is 8-byte aligned)
    if ((threadIdx.x & 63) == 0) red64[threadIdx.x >> 6] = k;
    __syncthreads();
    unsigned long long best = red64[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) best = red64[w] < best ? red64[w] : best;
    tps = 0x7ffffff - (int)(best & 0x7ffffffULL);
  }
  tps = max(tps, kTpsMin);
  tps = (tps + quantum - 1) / quantum * quantum;
  // Grow the split until the partial workspace can hold every item.
  for (int guard = 0; guard < 32; ++guard) {
    long long items = 0;
    for (int b = threadIdx.x; b < a.B; b += T) items += (long long)((pre[b] + tps - 1) / tps) * UB;
    int dm = 0;
    block_sum_max<NW>(items, dm, red);
    if (items <= a.max_items) break;
    tps = min(tps * 2, 1 << 28);
  }
  __syncthreads();
  block_scan<NW>(a, tps, pre, red, UB);
  tps_out = tps;
  return pre[a.B];
}

// -------------------------------------------------------------- tile data

// One 16-token tile's operands as held by one lane.
template <int D, class KV, class ST>
struct Tile {
  static constexpr int KB = (D / 4) * KV::bytes;     // K bytes per lane: token lane16, elems [grp*D/4, +D/4)
  static constexpr int VB = (D / 16) * KV::bytes;    // V bytes per lane per token: elems [lane16*D/16, +D/16)
  static constexpr bool kInt8 = std::is_same<KV, I8>::value;
  Raw<KB> k;
  Raw<VB> v[4];                                      // tokens 4*grp + i
  float ks[4], vs[4];                                // int8 scales of tokens 4*grp + i
};

// Byte offsets of this lane's operands inside one tile (constant per item).
struct LaneOff {
  uint32_t k;       // token lane16, elements [grp*D/4, +D/4)
  uint32_t v[4];    // token 4*grp+i, elements [lane16*D/16, +D/16)
  uint32_t ks, vs;  // scales of tokens 4*grp .. 4*grp+3
};

// Uniform base pointers of one tile (scalar registers).
struct TilePtr {
  const char* k; const char* v; const char* ks; const char* vs;
};

template <class ST>
__device__ __forceinline__ float load_scale(const char* p) {
  if constexpr (std::is_same<ST, F32>::value) return *(const float*)p;
  else return (float)*(const _Float16*)p;
}

// Load this lane's operands of one tile.  FULL: all 16 tokens exist, so no
// per-lane predicate; otherwise tokens >= `valid` read as zero.
template <int D, class KV, class ST, bool FULL>
__device__ __forceinline__ void load_tile(const DecodeArgs& a, const TilePtr& t, const LaneOff& o, int valid,
                                          Tile<D, KV, ST>& c, int lane16, int grp) {
  using C = Tile<D, KV, ST>;
  if (FULL || lane16 < valid) load_raw<C::KB>(c.k, t.k + o.k);
  else zero_raw<C::KB>(c.k);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (FULL || 4 * grp + i < valid) load_raw<C::VB>(c.v[i], t.v + o.v[i]);
    else zero_raw<C::VB>(c.v[i]);
  }
  if constexpr (C::kInt8) {
    if (FULL && std::is_same<ST, F32>::value && a.scale_vec) {
      const f32x4 k4 = __builtin_nontemporal_load((const f32x4*)(t.ks + o.ks));
      const f32x4 v4 = __builtin_nontemporal_load((const f32x4*)(t.vs + o.vs));
#pragma unroll
      for (int i = 0; i < 4; ++i) { c.ks[i] = k4[i]; c.vs[i] = v4[i]; }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = FULL || 4 * grp + i < valid;
        c.ks[i] = ok ? load_scale<ST>(t.ks + o.ks + i * (uint32_t)a.ks_sn) : 0.0f;
        c.vs[i] = ok ? load_scale<ST>(t.vs + o.vs + i * (uint32_t)a.vs_sn) : 0.0f;
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

  f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < KSTEPS; ++j) {
    const u32x4 ka = k_operand<D, KV, ST>(c, j);
    sacc = mfma16x16x32(MT{}, ka, qop[j], sacc);
    if constexpr (QSplit<KV, QT>::value) sacc = mfma16x16x32(MT{}, ka, qop_lo[j], sacc);
  }
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = sacc[i] * qmul;
    if constexpr (kInt8) s[i] *= c.ks[i];
    if (!FULL && tile * kTile + 4 * grp + i >= ntok) s[i] = -INFINITY;
  }
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
    pop_lo[0] = pack2(MT{}, p[0] - lo_f32(MT{}, pop[0]), p[1] - hi_f32(MT{}, pop[0]));
    pop_lo[1] = pack2(MT{}, p[2] - lo_f32(MT{}, pop[1]), p[3] - hi_f32(MT{}, pop[1]));
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
    if constexpr (!kInt8) st.acc[e] = mfma16x16x16(MT{}, va, pop_lo, st.acc[e]);
  }
}

// Q operand for a unit: head col c (lane16), element range of group grp.
// Returns the per-lane score multiplier (sm_scale*log2e, times 2^-shift when
// the query was rescaled to stay inside f16's range).
template <int D, class KV, class QT>
__device__ __forceinline__ float load_q(const DecodeArgs& a, int b, int hq, bool live, int grp,
                                       u32x4* qop, u32x4* qop_lo) {
  using MT = typename MmaOf<KV>::T;
  constexpr int KSTEPS = D / 32;
  constexpr int PER = D / 4;
  float qf[PER];
  const char* qp = a.q + b * a.q_sb + (int64_t)hq * a.q_sh + grp * PER * 2;
#pragma unroll
  for (int w = 0; w < PER / 8; ++w) {
    const u32x4 x = live ? *(const u32x4*)(qp + 16 * w) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qf[8 * w + 2 * i] = lo_f32(QT{}, x[i]);
      qf[8 * w + 2 * i + 1] = hi_f32(QT{}, x[i]);
    }
  }
  float mul = a.qk_scale;
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

// Waves per SIMD each instantiation is compiled for (its VGPR budget).  A
// work-group is NW = 8 waves, so below 4 waves per SIMD a CU holds one group.
template <int D, class KV>
struct DecodeWaves {
  static constexpr int value = D <= 64 ? 4 : (D <= 128 ? 2 : 1);
};

// Geometry of one item inside a work-group of NW waves (all uniform).
//   U >= NW: the item covers NW units (one per wave), phases P = 1.
//   U <  NW: the item covers all U units; P = NW / U waves share a unit and
//            split its tiles by phase (merged through LDS afterwards).
struct ItemShape {
  int units;   // units covered by one item (<= NW)
  int P;       // waves per unit
};
template <int NW>
__device__ __forceinline__ ItemShape item_shape(int U) {
  ItemShape sh;
  if (U >= NW) { sh.units = NW; sh.P = 1; }
  else { sh.units = U; sh.P = NW / U; }
  return sh;
}

template <int D, class KV, class QT, class ST, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(DecodeWaves<D, KV>::value)))
void decode_main(const DecodeArgs a) {
  constexpr int E = D / 16;
  constexpr int KSTEPS = D / 32;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  // LDS: [acc: NW*G16*D f32][m: NW*G16][l: NW*G16][red: 2*NW+2 ints][pre: B+1 ints]
  float* l_acc = (float*)smem;
  float* l_m = l_acc + NW * a.G16 * D;
  float* l_l = l_m + NW * a.G16;
  int* red = (int*)(l_l + NW * a.G16);
  int* pre = red + 2 * NW + 2;

  const ItemShape shape = item_shape<NW>(a.U);
  // the plan (written by decode_plan just before this kernel): split size,
  // item count and the item prefix per sequence
  const int tps = uniform(a.ws_plan[kPlanTps]);
  const int total = uniform(a.ws_plan[kPlanTotal]);
  for (int i = threadIdx.x; i <= a.B; i += NW * 64) pre[i] = a.ws_plan[kPlanHeader + i];
  // Work assignment: group g first takes item g; items past the grid are
  // handed out by an atomic counter (zeroed by decode_plan), so a group that
  // finishes early takes more and ragged batches stay balanced.  Only those
  // late, naturally staggered requests touch the counter: a burst of
  // same-address atomics from every group at launch costs more than it saves.
  int* l_item = red;   // LDS slot broadcasting the next item
  const bool steal = total > (int)gridDim.x;
  __syncthreads();
  int next_item = blockIdx.x;

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane16 = lane & 15, grp = lane >> 4;
  using TileT = Tile<D, KV, ST>;
  LaneOff lo;
  lo.k = (uint32_t)(lane16 * a.k_sn) + (uint32_t)(grp * TileT::KB);
#pragma unroll
  for (int i = 0; i < 4; ++i) lo.v[i] = (uint32_t)((4 * grp + i) * a.v_sn) + (uint32_t)(lane16 * TileT::VB);
  lo.ks = (uint32_t)(4 * grp * a.ks_sn);
  lo.vs = (uint32_t)(4 * grp * a.vs_sn);
  const int uin = wave / shape.P;        // unit slot of this wave inside an item
  const int phase = wave - uin * shape.P;

  while (next_item < total) {
    const int item = uniform(next_item);
    // request the following item now; its index is only needed at the end
    int stolen = 0;
    if (steal && threadIdx.x == 0) stolen = (int)gridDim.x + atomicAdd(&a.ws_plan[kPlanCounter], 1);
    // item -> (b, split, unit block): b is the largest index with pre[b] <= item
    int blo = 0, bhi = a.B;
    while (bhi - blo > 1) { const int mid = (blo + bhi) >> 1; if (pre[mid] <= item) blo = mid; else bhi = mid; }
    const int b = uniform(blo);
    const int rem = uniform(item - pre[b]);
    const int split = rem / a.UB, ublk = rem - split * a.UB;
    const int unit = ublk * shape.units + uin;
    const bool wave_live = uin < shape.units && unit < a.U;
    const int hkv = unit / a.HG, hg = unit - hkv * a.HG;
    const int ntok = uniform(seq_tokens(a, b));
    const int ntile = (ntok + kTile - 1) / kTile;
    const int nsplit = (ntile + tps - 1) / tps;
    const int t_lo = split * tps;
    const int t_hi = min(t_lo + tps, ntile);
    const int nh = wave_live ? min(16, a.G - 16 * hg) : 0;    // live head columns of this wave's unit
    const bool live = lane16 < nh;
    const int hq = live ? hkv * a.G + 16 * hg + lane16 : 0;

    WaveState<D> st;
    st.m = -INFINITY; st.l = 0.f; st.sexp = -100;
#pragma unroll
    for (int e = 0; e < E; ++e) st.acc[e] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (wave_live) {
      u32x4 qop[KSTEPS], qop_lo[KSTEPS];
      const float qmul = load_q<D, KV, QT>(a, b, hq, live, grp, qop, qop_lo);

      // This wave takes tiles t_lo + phase, + P, ...: `nfull` full tiles
      // (double-buffered) and possibly the sequence's partial last tile.
      const int P = shape.P;
      const bool paged = a.bt != nullptr;
      const int t_first = t_lo + phase;
      const int t_full = min(t_hi, ntok / kTile);
      const int nfull = t_first < t_full ? (t_full - t_first + P - 1) / P : 0;
      const int nt = t_first < t_hi ? (t_hi - t_first + P - 1) / P : 0;
      const int64_t rowk = paged ? 0 : (int64_t)b * a.k_s0, rowv = paged ? 0 : (int64_t)b * a.v_s0;
      const int64_t rowks = paged ? 0 : (int64_t)b * a.ks_s0, rowvs = paged ? 0 : (int64_t)b * a.vs_s0;
      const char* kb = a.k + rowk + (int64_t)hkv * a.k_sh;
      const char* vb = a.v + rowv + (int64_t)hkv * a.v_sh;
      const char* ksb = a.ks + rowks + (int64_t)hkv * a.ks_sh;
      const char* vsb = a.vs + rowvs + (int64_t)hkv * a.vs_sh;
      const int tpp_mask = (1 << a.lg_tiles_per_page) - 1;
      auto tile_ptr = [&](int t, int phys) {
        TilePtr tp;
        int64_t ok, ov, oks, ovs;
        if (paged) {
          const int off = (t & tpp_mask) * kTile;
          ok = (int64_t)phys * a.k_s0 + off * a.k_sn;
          ov = (int64_t)phys * a.v_s0 + off * a.v_sn;
          oks = (int64_t)phys * a.ks_s0 + off * a.ks_sn;
          ovs = (int64_t)phys * a.vs_s0 + off * a.vs_sn;
        } else {
          ok = (int64_t)t * kTile * a.k_sn;
          ov = (int64_t)t * kTile * a.v_sn;
          oks = (int64_t)t * kTile * a.ks_sn;
          ovs = (int64_t)t * kTile * a.vs_sn;
        }
        tp.k = kb + ok; tp.v = vb + ov; tp.ks = ksb + oks; tp.vs = vsb + ovs;
        return tp;
      };
      // page ids of this wave's tiles [w0, w0 + 64) in lanes 0..63
      auto page_ids = [&](int w0, int wn) {
        int pg = 0;
        if (paged && lane < wn) {
          const int t = t_first + (w0 + lane) * P;
          pg = a.bt[(int64_t)b * a.bt_sb + (int64_t)(t >> a.lg_tiles_per_page) * a.bt_sl];
          pg = ((unsigned)pg < (unsigned long long)a.num_pages) ? pg : 0;   // never read outside the pool
        }
        return pg;
      };
      TileT bufA, bufB;
      for (int w0 = 0; w0 < nfull; w0 += 64) {
        const int wn = min(64, nfull - w0);
        const int pg = page_ids(w0, wn);
        int k = 0;
        load_tile<D, KV, ST, true>(a, tile_ptr(t_first + w0 * P, __builtin_amdgcn_readlane(pg, 0)), lo, 16,
                                   bufA, lane16, grp);
        while (true) {
          if (k + 1 < wn)
            load_tile<D, KV, ST, true>(a, tile_ptr(t_first + (w0 + k + 1) * P, __builtin_amdgcn_readlane(pg, k + 1)),
                                       lo, 16, bufB, lane16, grp);
          compute_tile<D, KV, QT, ST, true>(bufA, qop, qop_lo, qmul, 0, ntok, grp, st);
          if (++k >= wn) break;
          if (k + 1 < wn)
            load_tile<D, KV, ST, true>(a, tile_ptr(t_first + (w0 + k + 1) * P, __builtin_amdgcn_readlane(pg, k + 1)),
                                       lo, 16, bufA, lane16, grp);
          compute_tile<D, KV, QT, ST, true>(bufB, qop, qop_lo, qmul, 0, ntok, grp, st);
          if (++k >= wn) break;
        }
      }
      if (nt > nfull) {  // the sequence's partial last tile belongs to this wave
        const int t = t_first + nfull * P;
        const int pg = page_ids(nfull, 1);
        load_tile<D, KV, ST, false>(a, tile_ptr(t, __builtin_amdgcn_readlane(pg, 0)), lo, ntok - t * kTile,
                                    bufA, lane16, grp);
        compute_tile<D, KV, QT, ST, false>(bufA, qop, qop_lo, qmul, t, ntok, grp, st);
      }
    }

    const float lsum = wave_sum_xor16_32(st.l);
    const float unscale = std::is_same<KV, I8>::value ? ldexpf(1.0f, st.sexp - 4) : 1.0f;
    const bool direct = nsplit == 1;
    // partial slot of (item, unit slot, head col)
    const int64_t pslot = ((int64_t)item * NW + uin) * a.G16;
    if (shape.P == 1) {
      // one wave owns each unit: write straight from registers
      if (live) {
        if (direct) {
          const float inv = unscale / (lsum == 0.f ? 1.f : lsum);
          char* op = a.out + b * a.o_sb + (int64_t)hq * a.o_sh + grp * (D / 4) * 2;
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < E; e += 2) {
              const uint32_t w = pack2(QT{}, st.acc[e][i] * inv, st.acc[e + 1][i] * inv);
              *(uint32_t*)(op + (i * E + e) * 2) = w;
            }
        } else {
          float* dst = a.ws_acc + (pslot + lane16) * D + grp * (D / 4);
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < E; e += 4)
              *(f32x4*)(dst + i * E + e) = f32x4{st.acc[e][i] * unscale, st.acc[e + 1][i] * unscale,
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
        float* dst = l_acc + (wave * a.G16 + lane16) * D + grp * (D / 4);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < E; ++e) dst[i * E + e] = st.acc[e][i] * unscale;
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
          const int64_t ps = ((int64_t)item * NW + us) * a.G16 + cc;
          a.ws_acc[ps * D + d] = A;
          if (d == 0) { a.ws_ml[ps * 2 + 0] = M; a.ws_ml[ps * 2 + 1] = L; }
        }
      }
    }
    if (steal) {
      if (threadIdx.x == 0) l_item[0] = stolen;
      __syncthreads();
      next_item = l_item[0];
      __syncthreads();   // l_item and the merge LDS are free for the next item
    } else {
      if (shape.P > 1) __syncthreads();   // merge LDS free for reuse
      next_item += gridDim.x;
    }
  }
}

// One work-group: decide the split from the device-side lengths, write the
// item prefix and zero the work counter for decode_main.
template <int NW>
__global__ __launch_bounds__(NW * 64) void decode_plan(const DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int* red = (int*)smem;            // 2*NW+2 ints (8-byte aligned)
  int* pre = red + 2 * NW + 2;      // B+1 ints
  const ItemShape shape = item_shape<NW>(a.U);
  int tps;
  const int total = plan_items<NW>(a, pre, red, tps, shape.P, a.UB, a.slots);
  for (int i = threadIdx.x; i <= a.B; i += NW * 64) a.ws_plan[kPlanHeader + i] = pre[i];
  if (threadIdx.x == 0) {
    a.ws_plan[kPlanTps] = tps;
    a.ws_plan[kPlanTotal] = total;
    a.ws_plan[kPlanUB] = a.UB;
    a.ws_plan[kPlanCounter] = 0;
  }
}

// Merge split-K partials of one (sequence, query head) per wave; writes zeros
// for empty sequences and skips sequences the main kernel wrote directly.
template <int D, class OT, int NW>
__global__ __launch_bounds__(256) void decode_reduce(const DecodeArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= a.B * a.Hq) return;
  const int b = row / a.Hq, hq = row - b * a.Hq;
  const int p0 = a.ws_plan[kPlanHeader + b], p1 = a.ws_plan[kPlanHeader + b + 1];
  const int nsplit = (p1 - p0) / a.UB;
  if (nsplit == 1) return;
  const int hkv = hq / a.G, gi = hq - hkv * a.G, hg = gi >> 4, cc = gi & 15;
  const int unit = hkv * a.HG + hg;
  const ItemShape shape = item_shape<NW>(a.U);
  const int ublk = unit / shape.units, uin = unit - ublk * shape.units;
  char* op = a.out + b * a.o_sb + (int64_t)hq * a.o_sh;
  auto slot = [&](int s) { return ((int64_t)(p0 + s * a.UB + ublk) * NW + uin) * a.G16 + cc; };
  // (m, l) of up to 64 splits per pass, one split per lane
  float M = -INFINITY;
  for (int s0 = 0; s0 < nsplit; s0 += 64) {
    const int s = s0 + lane;
    const float m = s < nsplit ? a.ws_ml[slot(s) * 2] : -INFINITY;
    M = fmaxf(M, m);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
  constexpr int PER = (D + 63) / 64;
  float A[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) A[i] = 0.f;
  float L = 0.f;
  if (M != -INFINITY) {
    for (int s0 = 0; s0 < nsplit; s0 += 64) {
      const int s = s0 + lane;
      float wt = 0.f, lw = 0.f;
      if (s < nsplit) {
        const float m = a.ws_ml[slot(s) * 2];
        wt = m == -INFINITY ? 0.f : fast_exp2(m - M);
        lw = wt * a.ws_ml[slot(s) * 2 + 1];
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) lw += __shfl_xor(lw, o);
      L += lw;
      const int n = min(64, nsplit - s0);
#pragma unroll 4
      for (int j = 0; j < n; ++j) {
        const float w = __shfl(wt, j);
        const float* src = a.ws_acc + slot(s0 + j) * D;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int d = lane + 64 * i;
          if (d < D) A[i] += w * src[d];
        }
      }
    }
  }
  const float inv = 1.0f / (L == 0.f ? 1.f : L);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + 64 * i;
    if (d < D) store_out(OT{}, op + d * (int)sizeof(uint16_t), A[i] * inv);
  }
}

}  // namespace sia
