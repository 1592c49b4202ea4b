// Causal / full flash-attention forward (prefill, any Tq) for gfx950.
//
// Semantics follow the reference kernel kernels/attention_kernel.py:91-232:
// query row i sits at absolute position (Tk - Tq) + i and, when causal, sees
// keys j <= (Tk - Tq) + i (bottom-right alignment); a row with no visible key
// is written as zeros; GQA maps query head hq to KV head hq / (Hq / Hkv);
// The reference rounds P to the input dtype before PV (tl.dot(p.to(v.dtype),
// v)); here P and V are rounded to f16 for that product whatever the input
// dtype (bf16 P alone costs up to ~2^-9 |v| on rows with few keys), V values
// saturate at the f16 range (+-65504), and the row sum is taken over the
// rounded weights.  Accumulation is fp32.
//
// Structure (MI355X-first):
//  * prefill_pack_v converts V once per call into f16 "V^T block images":
//    one 64-key block per image, laid out exactly as the main kernel's LDS
//    wants it, so no work-group converts or transposes V again (each V block
//    is read by every query block and every query head of its KV head).
//  * A work-group of prefill_fwd is 8 waves (two per SIMD) of 32 query rows
//    each: the same rows of hpw query heads that share one KV head, 32 *
//    8 / hpw rows per head (hpw = 4 at G = 4: 64 rows x 4 heads).  Every
//    wave of a causal work-group then sees the same key blocks, so no wave
//    idles while the last one finishes.  It walks key blocks of BN = 64 through a
//    four-stage LDS ring per tensor filled by buffer_load ... lds (global ->
//    LDS DMA, no VGPR staging): three blocks are in flight while one is
//    computed, every wait is a constant vmcnt, and the per-step barrier
//    carries no memory fence (a fence would drain the ring).
//  * K stages are row-major with an XOR swizzle of their 16-byte chunks, so
//    each DMA instruction reads whole rows (coalesced) and the MFMA operand
//    reads stay free of bank conflicts; V^T images are chunk-major.
//  * Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (keys as rows,
//    its 32 queries as columns), so every lane owns one query: the row max is
//    a lane-local v_maximum3 tree plus one v_permlane32_swap, and P^T feeds
//    O^T += V^T P^T straight from registers (the key order of its k-slots
//    matches the S^T output layout; the V^T images store keys in that order).
//  * Software pipeline: the MFMAs of the next block's scores are interleaved
//    (sched_group_barrier) with the exponentials of the current block, whose
//    PV MFMAs follow; the loop is unrolled by four so stage arrays and score
//    registers are fixed per step at compile time.
//  * Blocks are issued heaviest-first (the causal diagonal makes late query
//    blocks the longest), and every work-group of one (b, KV head) is placed
//    on the same XCD so their K/V tiles are served by one L2.
#pragma once

#include "sia_common.hpp"

namespace sia {

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32x32x16(F16, u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}
__device__ __forceinline__ f32x16 mfma32x32x16(BF16, u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

struct PrefillArgs {
  const char* q; int64_t q_sb, q_sh, q_sm;     // byte strides; head_dim contiguous
  const char* k; int64_t k_sb, k_sh, k_sn;
  const char* vimg;                             // V^T block images (prefill_pack_v)
  const char* v; int64_t v_sb, v_sh, v_sn;      // raw V (variant 2: images built in LDS)
  char* out; int64_t o_sb, o_sh, o_sm;
  int32_t B, Hq, Hkv, G, Tq, Tk, causal;
  float qk_scale;                               // sm_scale * log2(e)
  int32_t nqblk;                                // ceil(Tq / rows per head per work-group)
  int32_t nkb;                                  // ceil(Tk / 64)
  int32_t hpw_lg;                               // log2 of the query heads per work-group (hpw)
  int32_t nunit;                                // work-groups per query block: B * Hkv * (G / hpw)
  int32_t remap;                                // XCD-aware block order (nunit % 8 == 0)
  int32_t fold;                                 // CU count when the grid fills two work-groups per CU, else 0
  FastDiv dU, dU8, dBH, dHkv;                   // divisions by nunit, nunit / 8, B * Hkv, Hkv
  // rotary embedding of q at load (prefill_fwd<D, T, true> only): query row
  // i of sequence b sits at position start_host + start_pos[b or 0] + i
  // (start_pos NULL: 0) and is rotated by row pos of the cos/sin tables
  // (first D/2 columns; a position outside the table rotates to zeros)
  const char* cs; const char* sn; int64_t tab_rs;
  int32_t Tc, tab_dt, interleaved;
  const int32_t* start_pos; int32_t start_host, pos_per_seq;
};

struct PackArgs {
  const char* v; int64_t v_sb, v_sh, v_sn;      // byte strides; head_dim contiguous
  char* vimg;
  int32_t Hkv, Tk, nkb;
  int64_t nblocks;                              // B * Hkv * nkb
};

constexpr int kPfBN = 64;               // keys per block
constexpr int kBufferFlags = 0x00020000;   // gfx9 raw buffer resource word 3 (32-bit data, no swizzle)

// Per-head-dim configuration of prefill_fwd.
//  * D = 128: 8 waves (two per SIMD, 256 VGPRs each) and a four-stage K/V ring
//    (three blocks in flight); one work-group (128 KB of LDS) per CU.
//    Variant 1 (VAR = 1, chosen by the host when the 8-wave grid would not
//    exceed the CU count, e.g. one sequence of up to 2048 tokens): 4 waves
//    and a two-stage ring, so twice the work-groups, and a causal work-group
//    covers half the rows (B1 T = 1024: 30.5 -> 25.6 us per call).
//    Variant 2 (D = 32 and 64 too) is variant 1 without prefill_pack_v: V blocks come into the
//    ring as raw rows, every work-group converts each bfloat16 block to f16
//    in LDS, and the PV product reads it with transposed reads (more vector
//    work per block, one launch less per call; chosen for short key ranges,
//    where the call is launch- and latency-bound).
//    float16 at D = 32 ... 128 needs no V^T images in any variant: raw V rows
//    and transposed LDS reads (kTrV in prefill_fwd).
//  * D <= 64: 4 waves with the same register budget, so two work-groups share
//    a CU and one's prologue and epilogue overlap the other's key loop (MHA
//    D = 64 at T = 1024: 88 -> 70 us per call); a two-stage ring at D = 64,
//    four stages below, where blocks are small (measured best of the two).
//  * D = 256: the O^T accumulators alone take 128 registers per lane, so 4
//    waves run one per SIMD with 512 registers, and the 32 KB blocks fit LDS
//    as a two-stage ring.
// The PV product works on 32-dimension tiles, so V images are at least 32
// dimensions wide (D = 16 is zero-padded).
template <int D, int VAR = 0>
struct PfCfg {
  static constexpr bool small = VAR >= 1;
  static constexpr bool packv = VAR == 2;                 // V^T images built in LDS from raw V rows
  static constexpr int waves = D == 128 && !small ? 8 : 4;
  static constexpr int stages = small ? 2 : D == 128 || D < 64 ? 4 : 2;
  static constexpr int wpe = D <= 128 ? 2 : 1;          // waves per SIMD the registers are budgeted for
  static constexpr int DV = D < 32 ? 32 : D;             // V^T image dimensions
  static constexpr int kblk = kPfBN * D * 2;             // bytes of one K block
  static constexpr int vblk = kPfBN * DV * 2;            // bytes of one V^T image
  static constexpr int kdma = kblk / 1024;               // 1 KB DMA instructions per K block
  static constexpr int vdma = vblk / 1024;
  static constexpr int kper = (kdma + waves - 1) / waves;   // per wave (waves past the count issue
  static constexpr int vper = (vdma + waves - 1) / waves;   // empty transfers into a dummy area)
  static constexpr bool dummy = kper * waves != kdma || vper * waves != vdma;
};

// Waves per work-group of prefill_fwd at head_dim D (host side).
inline int pf_waves(int D, int var = 0) { return D == 128 && var == 0 ? 8 : 4; }
// Query heads per work-group: the largest power of two that divides the GQA
// group size G and is at most the wave count (host side).
inline int pf_heads_per_group(int D, int G, int var = 0) {
  int h = 1;
  while (2 * h <= pf_waves(D, var) && G % (2 * h) == 0) h *= 2;
  return h;
}

// Key (0..63 within its block) held by element i (0..7) of image chunk c: the
// keys of 16-key group c/2 in the order of the S^T output registers of lanes
// of half c%2, i.e. 4 (c%2) + {0, 1, 2, 3, 8, 9, 10, 11}.
__device__ __forceinline__ int image_key(int c, int i) { return 16 * (c >> 1) + 4 * (c & 1) + (i & 3) + 8 * (i >> 2); }

// One 16-bit V element (raw bits) as f16 bits: bf16 is widened to f32,
// clamped to the f16 range and rounded (the PV product runs in f16 so that P
// keeps 11 significant bits).
__device__ __forceinline__ uint32_t elem_f16(F16, uint32_t bits) { return bits; }
__device__ __forceinline__ uint32_t elem_f16(BF16, uint32_t bits) {
  const float f = __builtin_amdgcn_fmed3f(__builtin_bit_cast(float, bits << 16), -65504.0f, 65504.0f);
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// V (B, Hkv, Tk, D) -> images [B][Hkv][nkb]: image chunk x = c * DV + d (16
// bytes at x * 16) holds keys image_key(c, 0..7) of dimension d as f16; keys
// at or past Tk and dimensions past D are zero.  One work-group per image:
// the 64 x D block is read with coalesced 16-byte loads into LDS (rows padded
// by 8 bytes so the 8 rows one output chunk gathers sit in different banks),
// then every thread assembles whole output chunks, so each store instruction
// of a wave writes one contiguous 1 KB run.
template <int D, class T>
__global__ __launch_bounds__(256) void prefill_pack_v(const PackArgs a) {
  constexpr int DV = PfCfg<D>::DV;
  constexpr int RS = D + 4;                       // LDS row stride in 16-bit elements
  constexpr int IN = kPfBN * D / 8;               // 16-byte input chunks per block
  constexpr int OUT = 8 * DV;                     // 16-byte output chunks per image
  __shared__ __attribute__((aligned(16))) uint16_t tile[kPfBN * RS];
  const uint32_t blk = blockIdx.x;
  const uint32_t bh = blk / (uint32_t)a.nkb;
  const int kb = (int)(blk - bh * (uint32_t)a.nkb);
  const uint32_t b = bh / (uint32_t)a.Hkv;
  const int hkv = (int)(bh - b * (uint32_t)a.Hkv);
  const char* src = a.v + (int64_t)b * a.v_sb + (int64_t)hkv * a.v_sh;
#pragma unroll
  for (int i = 0; i < (IN + 255) / 256; ++i) {
    const int q = threadIdx.x + 256 * i;
    if (q < IN) {
      const int row = q / (D / 8), c8 = q % (D / 8);
      const int key = kb * kPfBN + row;
      const u32x4 w = key < a.Tk ? *(const u32x4*)(src + (int64_t)key * a.v_sn + c8 * 16) : u32x4{0u, 0u, 0u, 0u};
      uint32_t* t = (uint32_t*)(tile + row * RS + c8 * 8);   // 8-byte aligned (RS * 2 % 8 == 0)
      *(u32x2*)t = u32x2{w[0], w[1]};
      *(u32x2*)(t + 2) = u32x2{w[2], w[3]};
    }
  }
  __syncthreads();
  char* dst = a.vimg + (int64_t)blk * PfCfg<D>::vblk;
#pragma unroll
  for (int i = 0; i < OUT / 256; ++i) {
    const int x = threadIdx.x + 256 * i;
    const int c = x / DV, d = x % DV;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (d < D) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t lo = elem_f16(T{}, tile[image_key(c, 2 * m) * RS + d]);
        const uint32_t hi = elem_f16(T{}, tile[image_key(c, 2 * m + 1) * RS + d]);
        w[m] = lo | (hi << 16);
      }
    }
    *(u32x4*)(dst + (int64_t)x * 16) = w;
  }
}

// Rotary prologue variants of prefill_fwd: q rotated as it is loaded, with
// split-half pairs (i, i + D/2) or interleaved pairs (2i, 2i + 1), from
// cos/sin tables in q's dtype or in fp32.
enum : int { kRopeNone = 0, kRopeSplit16 = 1, kRopeInter16 = 2, kRopeSplit32 = 3, kRopeInter32 = 4 };

// The cos/sin entries one lane needs to rotate its Q operand (qop[j] holds
// q[d], d = 16 j + 8 h + [0, 8)): split-half pairs (d, d + D/2) use columns
// 16 j + 8 h + [0, 8) for j < D/32 (D = 16: columns 0-7 in both half-waves);
// interleaved pairs (2i, 2i + 1) use columns 8 j + 4 h + [0, 4) for j < D/16.
// They are fetched into registers together with q, before the first K/V
// transfers are issued, and used once those are in flight: every variant
// issues a fixed number of loads, so the wait before the rotation covers q
// and the tables alone.
template <int D, int ROPE>
struct RopeQ {
  static constexpr int EW = ROPE >= kRopeSplit32 ? 2 : 1;             // words per two entries
  static constexpr int NW = (D / 8 > 4 ? D / 8 : 4) * EW;             // words per table
  uint32_t c[ROPE ? NW : 1], s[ROPE ? NW : 1];
  bool ok;                                                           // the position has a table row
};

template <int D, int ROPE>
__device__ __forceinline__ void rope_q_fetch(const PrefillArgs& a, RopeQ<D, ROPE>& r, int64_t pos, int h) {
  constexpr int KST = D / 16;
  constexpr int ES = ROPE >= kRopeSplit32 ? 4 : 2;                    // table entry bytes
  r.ok = pos >= 0 && pos < a.Tc;
  const int64_t ro = (int64_t)(r.ok ? pos : 0) * a.tab_rs;
  const char* crow = a.cs + ro;
  const char* srow = a.sn + ro;
  // n 16-byte or 8-byte pieces from column col of both rows into words w0..
  auto take = [&](int col, int w0, int bytes) {
#pragma unroll
    for (int off = 0; off < bytes; off += 16) {
      if (bytes - off >= 16) {
        const u32x4 cv = *(const u32x4*)(crow + ES * col + off), sv = *(const u32x4*)(srow + ES * col + off);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          r.c[w0 + off / 4 + e] = cv[e];
          r.s[w0 + off / 4 + e] = sv[e];
        }
      } else {
        const u32x2 cv = *(const u32x2*)(crow + ES * col + off), sv = *(const u32x2*)(srow + ES * col + off);
        r.c[w0 + off / 4] = cv[0]; r.c[w0 + off / 4 + 1] = cv[1];
        r.s[w0 + off / 4] = sv[0]; r.s[w0 + off / 4 + 1] = sv[1];
      }
    }
  };
  if constexpr (ROPE == kRopeInter16 || ROPE == kRopeInter32) {
#pragma unroll
    for (int j = 0; j < KST; ++j) take(8 * j + 4 * h, 2 * RopeQ<D, ROPE>::EW * j, 4 * ES);
  } else {
    constexpr int NQ = KST >= 2 ? KST / 2 : 1;
#pragma unroll
    for (int j = 0; j < NQ; ++j) take(KST >= 2 ? 16 * j + 8 * h : 0, 4 * RopeQ<D, ROPE>::EW * j, 8 * ES);
  }
}

// N consecutive entries from fetched words w (16-bit tables hold q's dtype T)
template <int N, bool F32T, class T>
__device__ __forceinline__ void tab_vals(const uint32_t* w, float* x) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    if constexpr (F32T) {
      x[2 * i] = __builtin_bit_cast(float, w[2 * i]);
      x[2 * i + 1] = __builtin_bit_cast(float, w[2 * i + 1]);
    } else {
      x[2 * i] = lo_f32(T{}, w[i]);
      x[2 * i + 1] = hi_f32(T{}, w[i]);
    }
  }
}

// Rotate this lane's Q operand in registers.  Split-half pairs sit in qop[j]
// and qop[j + D/32] of the same lane (for D = 16, in the lanes l and l ^ 32);
// interleaved pairs sit in one word.  The arithmetic is rope_rotate's, then
// a round to T: the same bits as the rotation kernels produce.  A position
// without a table row rotates q to zeros.
template <int D, class T, int ROPE>
__device__ __forceinline__ void rope_q_apply(const PrefillArgs& a, u32x4* qop, const RopeQ<D, ROPE>& r, int h) {
  constexpr int KST = D / 16;
  constexpr bool F32T = ROPE >= kRopeSplit32;
  constexpr int EW = RopeQ<D, ROPE>::EW;
  const uint32_t ok = r.ok ? 0xffffffffu : 0u;   // a mask, not a branch around the rotation
  if constexpr (ROPE == kRopeInter16 || ROPE == kRopeInter32) {
#pragma unroll
    for (int j = 0; j < KST; ++j) {
      float c[4], sn[4];
      tab_vals<4, F32T, T>(r.c + 2 * EW * j, c);
      tab_vals<4, F32T, T>(r.s + 2 * EW * j, sn);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float y0, y1;
        rope_rotate(lo_f32(T{}, qop[j][w]), hi_f32(T{}, qop[j][w]), c[w], sn[w], y0, y1);
        qop[j][w] = pack2(T{}, y0, y1) & ok;
      }
    }
  } else if constexpr (KST >= 2) {
#pragma unroll
    for (int j = 0; j < KST / 2; ++j) {
      float c[8], sn[8];
      tab_vals<8, F32T, T>(r.c + 4 * EW * j, c);
      tab_vals<8, F32T, T>(r.s + 4 * EW * j, sn);
      u32x4& xa = qop[j];
      u32x4& xb = qop[j + KST / 2];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float a0, b0, a1, b1;
        rope_rotate(lo_f32(T{}, xa[w]), lo_f32(T{}, xb[w]), c[2 * w], sn[2 * w], a0, b0);
        rope_rotate(hi_f32(T{}, xa[w]), hi_f32(T{}, xb[w]), c[2 * w + 1], sn[2 * w + 1], a1, b1);
        xa[w] = pack2(T{}, a0, a1) & ok;
        xb[w] = pack2(T{}, b0, b1) & ok;
      }
    }
  } else {
    // D = 16: dims 0-7 in lanes 0-31, their partners 8-15 in lanes 32-63
    float c[8], sn[8];
    tab_vals<8, F32T, T>(r.c, c);
    tab_vals<8, F32T, T>(r.s, sn);
    u32x4 other;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const auto x = __builtin_amdgcn_permlane32_swap(qop[0][w], qop[0][w], false, false);
      other[w] = h ? (uint32_t)x[0] : (uint32_t)x[1];
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float o0, o1, t0, t1;
      if (h == 0) {
        rope_rotate(lo_f32(T{}, qop[0][w]), lo_f32(T{}, other[w]), c[2 * w], sn[2 * w], o0, t0);
        rope_rotate(hi_f32(T{}, qop[0][w]), hi_f32(T{}, other[w]), c[2 * w + 1], sn[2 * w + 1], o1, t1);
      } else {
        rope_rotate(lo_f32(T{}, other[w]), lo_f32(T{}, qop[0][w]), c[2 * w], sn[2 * w], t0, o0);
        rope_rotate(hi_f32(T{}, other[w]), hi_f32(T{}, qop[0][w]), c[2 * w + 1], sn[2 * w + 1], t1, o1);
      }
      qop[0][w] = pack2(T{}, o0, o1) & ok;
    }
  }
}

template <int P>
struct PfParity {
  static constexpr int value = P;
};

// Combine lanes l and l ^ 32 (the two halves of the wave) without LDS:
// v_permlane32_swap of x with itself yields {x[l % 32], x[l % 32 + 32]}.
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                 false, false);
  return __builtin_elementwise_maximum(__builtin_bit_cast(float, (uint32_t)r[0]),
                                       __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                                 false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Work-group barrier for the K/V ring.  __syncthreads() carries a release
// fence, which on this target waits for every DMA still in flight (vmcnt(0))
// and would drain the ring each step.  The hand-offs here are ordered
// explicitly instead: a stage's DMA is retired by the wave's own vmcnt wait
// before it arrives, and its LDS reads of a stage are complete (lgkmcnt(0))
// before another wave may refill it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// vmcnt(N): at most N vector memory instructions of this wave still
// outstanding (gfx9 s_waitcnt: vmcnt bits 3:0 and 15:14, expcnt and lgkmcnt
// left at their no-wait maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// (one template argument each: __launch_bounds__ is a macro)
template <int C> constexpr int kPfThreads = PfCfg<C / 4, C % 4>::waves * 64;
template <int C> constexpr int kPfWpe = PfCfg<C / 4, C % 4>::wpe;

template <int D, class T, int ROPE, int VAR>
__global__ __launch_bounds__(kPfThreads<4 * D + VAR>) __attribute__((amdgpu_waves_per_eu(kPfWpe<4 * D + VAR>)))
void prefill_fwd(const PrefillArgs a) {
  using C = PfCfg<D, VAR>;
  constexpr int NW = C::waves, S = C::stages, DV = C::DV;
  constexpr int KST = D / 16;                   // QK k-steps
  constexpr int ET = DV / 32;                   // O^T d-tiles
  constexpr int KB = C::kblk, VB = C::vblk;
  constexpr int NK = C::kper, NV = C::vper;     // DMA instructions per wave per block
  static_assert(S == 2 || S == 4, "ring depth");
  // float16 at D = 32 ... 128: V needs no conversion, so its blocks come
  // into the ring as raw rows and the PV product reads its A operand with
  // transposed LDS reads (ds_read_b64_tr_b16) instead of from V^T images: no
  // prefill_pack_v launch.  (bfloat16 V is converted to float16 for the PV
  // product, which keeps P at 11 significant bits; a bfloat16 P misses the
  // 2e-3 output bar.  D = 16 keeps the images, zero-padded to the 32-wide PV
  // tile.  D = 256, one wave per SIMD, lost 11% to the two reads per operand
  // against the repack's one launch.)
  constexpr bool kTrV = (std::is_same<T, F16>::value && D >= 32 && D <= 128) || C::packv;
  constexpr bool kRawV = kTrV;                  // raw V rows in the V stages
  // K stages: swizzled row-major (below); V^T image chunk c of dimension d at
  // c * D * 16 + d * 16
  // (distinct arrays per stage: the compiler then sees that a DMA into one
  // stage never aliases the LDS reads of another and adds no waits)
  __shared__ __attribute__((aligned(1024))) char lk0[KB], lk1[KB], lk2[S > 2 ? KB : 16], lk3[S > 2 ? KB : 16];
  __shared__ __attribute__((aligned(1024))) char lv0[VB], lv1[VB], lv2[S > 2 ? VB : 16], lv3[S > 2 ? VB : 16];
  // destination of the empty transfers of waves past a block's DMA count
  __shared__ __attribute__((aligned(1024))) char ldummy[C::dummy ? 1024 : 16];
  auto kstage = [&](auto s) -> char* {
    constexpr int I = decltype(s)::value % S;
    return I == 0 ? lk0 : I == 1 ? lk1 : I == 2 ? lk2 : lk3;
  };
  auto vstage = [&](auto s) -> char* {
    constexpr int I = decltype(s)::value % S;
    return I == 0 ? lv0 : I == 1 ? lv1 : I == 2 ? lv2 : lv3;
  };

  // ---- block -> (query block, unit), heaviest first.  A unit is (b, KV
  // head, group of hpw query heads); u = hgrp * B * Hkv + b * Hkv + hkv, so
  // with the XCD-aware order (block index % 8 = XCD) every unit of one (b,
  // KV head) lands on one XCD when B * Hkv % 8 == 0.
  // (both orders computed and one selected: a branch here made the compiler
  // load the kernel arguments in four dependent rounds instead of two)
  // A grid of more work-groups than CUs but at most two per CU is resident
  // at once: the first `fold` work-groups take one slot of every CU, and
  // work-group fold + i the second slot of work-group i's CU.  Those are
  // numbered lightest-first, so every CU pairs a heavy and a light group
  // (per XCD with the XCD-aware order, whose slots fold the same way).
  int ql, u;
  {
    const int lin = blockIdx.x;
    const int nall = a.nqblk * a.nunit;
    const int xcd = lin & 7;
    const int slot0 = lin >> 3, f8 = a.fold >> 3;
    const int slot = a.fold && slot0 >= f8 ? f8 + ((nall >> 3) - 1 - slot0) : slot0;
    const int lin1 = a.fold && lin >= a.fold ? a.fold + (nall - 1 - lin) : lin;
    const int ql8 = fdiv(slot, a.dU8);
    const int u8 = xcd + 8 * (slot - ql8 * (a.nunit >> 3));
    const int ql1 = fdiv(lin1, a.dU);
    const int u1 = lin1 - ql1 * a.nunit;
    ql = a.remap ? ql8 : ql1;
    u = a.remap ? u8 : u1;
  }
  const int bhn = a.B * a.Hkv;
  const int hgrp = fdiv(u, a.dBH);
  const int bh = u - hgrp * bhn;
  const int b = fdiv(bh, a.dHkv);
  const int hkv = bh - b * a.Hkv;
  const int qblk = a.nqblk - 1 - ql;
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int off = a.Tk - a.Tq;                           // bottom-right causal offset
  // This wave's head (wave % hpw) and 32-row group (wave / hpw) of the
  // work-group's rpg = NW / hpw row groups per head.  With 8 waves, waves w
  // and w + 4 share a SIMD; under a causal mask later row groups see more key
  // blocks, so with several row groups the second wave of each SIMD takes
  // them in reverse and every SIMD carries the same number of key blocks.
  const int rpg = NW >> a.hpw_lg;
  const int hw = wave & ((1 << a.hpw_lg) - 1);
  const int r0 = wave >> a.hpw_lg;
  const int rg = NW == 8 && wave >= NW / 2 && rpg > 1 ? rpg - 1 - (r0 - rpg / 2) : r0;
  const int hq = hkv * a.G + (hgrp << a.hpw_lg) + hw;
  const int q0 = qblk * 32 * rpg;                        // the work-group's first row (every head)
  const int qi = q0 + rg * 32 + l32;                     // this lane's query row

  // ---- Q^T operand (B of S^T = K Q^T): query qi, d = 16 j + 8 h + [0, 8)
  // (loaded by load_q below, after the first K block's transfers are issued)
  u32x4 qop[KST];
  RopeQ<D, ROPE> rq;   // rotation inputs (applied once the first K/V transfers are issued)
  auto load_q = [&]() {
    const char* qp = a.q + b * a.q_sb + (int64_t)hq * a.q_sh + (int64_t)min(qi, a.Tq - 1) * a.q_sm + 16 * h;
#pragma unroll
    for (int j = 0; j < KST; ++j) qop[j] = *(const u32x4*)(qp + 32 * j);   // (rows past Tq read row Tq - 1; never stored)
    if constexpr (ROPE != kRopeNone) {
      const int64_t base = (int64_t)a.start_host + (a.start_pos != nullptr ? a.start_pos[a.pos_per_seq ? b : 0] : 0);
      rope_q_fetch<D, ROPE>(a, rq, base + qi, h);
    }
  };

  const int kend = a.causal ? min(a.Tk, off + q0 + 32 * rpg) : a.Tk;
  const int nblk = kend > 0 ? (kend + kPfBN - 1) / kPfBN : 0;   // key blocks of the work-group
  const int wrow0 = q0 + rg * 32;                        // this wave's first row
  const int wend = a.causal ? min(a.Tk, off + wrow0 + 32) : a.Tk;   // keys this wave can see
  const int wblk = wend > 0 ? min(nblk, (wend + kPfBN - 1) / kPfBN) : 0;   // blocks this wave computes
  // blocks [0, wfull) are visible to every row of the wave: no mask
  const int lim_all = a.causal ? min(a.Tk - 1, off + wrow0) : a.Tk - 1;
  const int wfull = lim_all >= 0 ? (lim_all + 1) / kPfBN : 0;
  const int lim = a.causal ? min(a.Tk - 1, off + qi) : a.Tk - 1;   // this lane's last visible key

  const char* kb = a.k + b * a.k_sb + (int64_t)hkv * a.k_sh;
  const char* vimg = a.vimg + ((int64_t)b * a.Hkv + hkv) * a.nkb * VB;
  // K stages are row-major with an XOR swizzle: 16-byte chunk c of key row r
  // sits in slot c ^ (r % NC) of the row's RB bytes.  A DMA instruction then
  // reads whole rows (16 lanes per 256-byte row at D = 128: coalesced), and
  // the 8 lanes an LDS read serves at a time, which hold 8 consecutive rows,
  // hit 8 different bank groups.  k_voff[i]: this lane's byte offset inside
  // the block for DMA instruction i of the wave.
  constexpr int RB = 2 * D, NC = D / 8, ROWS_PER_DMA = 1024 / RB;
  int k_voff[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int r = (wave * NK + i) * ROWS_PER_DMA + lane / NC;
    k_voff[i] = r * (int)a.k_sn + (((lane % NC) ^ (r % NC)) * 16);
  }
  // raw V rows land in the V stages like K rows.  Variant 2 uses the K
  // swizzle.  The transposed reads (kTrV) use their own: one such read takes
  // 32 dimensions (4 chunks) of 8 consecutive rows, 32 chunk reads that
  // should cover the 16 chunk-wide bank groups of a 256-byte bank sweep twice
  // each.  Rows of 256 bytes (D = 128) start a sweep each, and slot
  // c ^ (4 (r % 4) + (r / 4) % 2) spreads them (the K swizzle, c ^ r % 16,
  // would put them on 8 groups: 4-way conflicts); 128-byte rows (D = 64)
  // share a sweep in pairs and take c ^ 4 ((r / 2) % 2); 64-byte rows
  // (D = 32) already cover a sweep in 4 rows.
  auto vswz = [](int r) -> int {
    if constexpr (!kTrV) return r % NC;
    else if constexpr (NC >= 16) return 4 * (r & 3) + ((r >> 2) & 1);
    else if constexpr (NC == 8) return 4 * ((r >> 1) & 1);
    else return 0;
  };
  const char* vb = kRawV ? a.v + b * a.v_sb + (int64_t)hkv * a.v_sh : nullptr;
  int v_voff[NK];
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const int r = (wave * NK + i) * ROWS_PER_DMA + lane / NC;
    v_voff[i] = kRawV ? r * (int)a.v_sn + (((lane % NC) ^ vswz(r)) * 16) : 0;
  }
  // kTrV: lane L of each 16-lane group gives the address of key row
  // (L % 16) / 4 of the group's 4 and dimensions 4 (L % 4) .. + 4 of its 16;
  // the read returns to lane L dimension L % 16 of the group at those 4 keys.
  // Groups (L / 16) cover dimensions 16 ((L / 16) % 2) of the d-tile and
  // keys 4 h, so lane (l32, h) gets dimension l32 of the tile at keys
  // 4 h + [0, 4) of the k-slot (+ 8 for the second read): the image order.
  // v_tr[e]: this lane's address for d-tile e within the first 16 keys (the
  // swizzle depends on the row's low 3 bits only, which k-slot and second
  // read, +16 and +8 rows, leave alone).
  int v_tr[kTrV ? ET : 1];
  if constexpr (kTrV) {
    const int trk = (lane & 15) >> 2, trj = lane & 3, trx = 2 * ((lane >> 4) & 1) + (trj >> 1);
    const int row = 4 * h + trk, f = vswz(row);
#pragma unroll
    for (int e = 0; e < ET; ++e) {
      v_tr[e] = row * RB + (((4 * e + trx) ^ f) * 16) + 8 * (trj & 1);
      // (held whole: split into a row part and a chunk part, each read paid
      // a v_or to join them, 32 per block step)
      asm volatile("" : "+v"(v_tr[e]));
    }
  }
  // A operand of PV slot x (k-slot x / ET, d-tile x % ET) from V stage Vst:
  // one V^T image chunk, or two transposed reads of raw rows (kTrV)
  auto pv_a = [&](const char* Vst, int x) -> u32x4 {
    if constexpr (kTrV) {
      typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
      const char* p = Vst + v_tr[x % ET] + (x / ET) * 16 * RB;
      const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p));
      const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 8 * RB)));
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    } else {
      return *(const u32x4*)(Vst + h * DV * 16 + l32 * 16 + (x / ET) * 2 * DV * 16 + (x % ET) * 512);
    }
  };
  // QK operand addresses: k-step j reads chunk 2 j + h of row l32 (tile 0)
  // and row l32 + 32 (tile 1: + 32 RB, same swizzle since 32 % NC == 0)
  int k_rd[KST];
#pragma unroll
  for (int j = 0; j < KST; ++j) k_rd[j] = l32 * RB + (((2 * j + h) ^ (l32 % NC)) * 16);

  // DMA of K block `blk` / V^T image `blk` into its ring stage (blk % S):
  // wave w moves 1 KB pieces [w NK, (w+1) NK) of the block (rows past Tk
  // read as zero through the buffer bound) and the same range of the image.
  // A block past the work-group's last one, and a piece past the block's end
  // (waves beyond the DMA count at small head_dim), is issued with an empty
  // buffer range: the hardware drops every out-of-range read (no memory
  // traffic) and what it fills is never read, so every wave issues the same
  // instruction count per group and the waits below are constants.
  // (one transfer instruction each: the ring refills are spread over the
  // MFMA stream, see `qk`)
  auto issue_k1 = [&](int blk, char* LK, int i) {
    const bool live = blk < nblk;
    const int key0 = live ? blk * kPfBN : 0;
    const int rows = live ? min(kPfBN, a.Tk - key0) : 0;
    {
      const int c = wave * NK + i;
      const bool real = c < C::kdma;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(kb + (int64_t)key0 * a.k_sn), 0, real ? rows * (int)a.k_sn : 0, kBufferFlags);
      // (every argument through a plain local: an expression such as an array
      // element or a conditional passed straight to this builtin makes the
      // host compilation pass drop the kernel's launch stub)
      const int voff = k_voff[i];
      char* dst = real ? LK + c * 1024 : ldummy;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, dst, 16, voff, 0, 0, 0);
    }
  };
  auto issue_v1 = [&](int blk, char* LV, int i) {
    const bool live = blk < nblk;
    if constexpr (kRawV) {
      const int key0 = live ? blk * kPfBN : 0;
      const int rows = live ? min(kPfBN, a.Tk - key0) : 0;
      const int c = wave * NK + i;
      const bool real = c < C::kdma;
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(vb + (int64_t)key0 * a.v_sn), 0, real ? rows * (int)a.v_sn : 0, kBufferFlags);
      const int voff = v_voff[i];
      char* dst = real ? LV + c * 1024 : ldummy;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, dst, 16, voff, 0, 0, 0);
    } else {
      const int c = wave * NV + i;
      const bool real = c < C::vdma;
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(vimg + (live ? (int64_t)blk * VB : 0)), 0, live && real ? VB : 0, kBufferFlags);
      char* dst = real ? LV + c * 1024 : ldummy;
      const int soff = real ? c * 1024 : 0;
      const int voff = lane * 16;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, dst, 16, voff, soff, 0, 0);
    }
  };
  auto issue_k = [&](int blk, char* LK) {
#pragma unroll
    for (int i = 0; i < NK; ++i) issue_k1(blk, LK, i);
  };
  auto issue_v = [&](int blk, char* LV) {
#pragma unroll
    for (int i = 0; i < NV; ++i) issue_v1(blk, LV, i);
  };
  // Variant 2 with bfloat16 V: convert the raw V block of stage LV to f16 in
  // place (the transposed reads then take it as they take float16 V).  Every
  // thread converts its own 16-byte chunks (bf16 bits as f32, clamped to the
  // f16 range, both halves rounded in one packed conversion: prefill_pack_v's
  // arithmetic), so one barrier after the writes suffices.
  auto pack_vstage = [&](char* LV) {
    if constexpr (C::packv && std::is_same<T, BF16>::value) {
      constexpr int CH = VB / 16 / (NW * 64);
      static_assert(CH * 16 * NW * 64 == VB, "variant 2 geometry");
      __builtin_amdgcn_sched_barrier(0);
      // (t passes through an empty asm so that the address arithmetic stays
      // inside this step: hoisted out of the key loop, its registers would be
      // held across every block)
      int t = threadIdx.x;
      asm volatile("" : "+v"(t));
      u32x4 w[CH];
#pragma unroll
      for (int i = 0; i < CH; ++i) w[i] = *(const u32x4*)(LV + (t + i * NW * 64) * 16);
#pragma unroll
      for (int i = 0; i < CH; ++i)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint32_t x = w[i][m];
          const float f0 = __builtin_bit_cast(float, x << 16), f1 = __builtin_bit_cast(float, x & 0xffff0000u);
          w[i][m] = pack2(F16{}, __builtin_amdgcn_fmed3f(f0, -65504.0f, 65504.0f),
                          __builtin_amdgcn_fmed3f(f1, -65504.0f, 65504.0f));
        }
#pragma unroll
      for (int i = 0; i < CH; ++i) *(u32x4*)(LV + (t + i * NW * 64) * 16) = w[i];
      ring_barrier();     // the whole converted block is written before any wave reads it
      // (nothing of the block step that follows is scheduled into the
      // conversion, where its registers would add to it)
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // A work step's ring refill: NP single transfers (K pieces, then V
  // pieces).  On the four-stage ring they are issued from inside the QK
  // product so that the memory pipeline takes them while the MFMAs run
  // (issued back to back after the barrier, the eight waves' transfers queue
  // up and stall every wave's issue); they have two blocks of lead there.
  // The two-stage ring has one block of lead, so its refills go out right
  // after the barrier (issued from the QK product, the last transfers have
  // only the PV half of a block to land: a D = 256 causal prefill of 4096
  // tokens takes 181 us that way against 154 us with the refills up front).
  constexpr int NP = NK + NV;
  constexpr bool kInlineRefill = S == 4;

  f32x16 o[ET];
#pragma unroll
  for (int e = 0; e < ET; ++e) o[e] = f32x16{};
  float m = -INFINITY, l = 0.f;

  // S^T = K Q^T for the 64 keys of one K stage: two 32-key tiles (raw scores;
  // the scale is folded into the exponent, c > 0 keeps the max)
  // (piece(p) issues transfer p of the step's ring refill; transfer p goes
  // after k-step p KST / NP)
  auto qk = [&](const char* K, f32x16& s0, f32x16& s1, auto piece) {
    s0 = f32x16{};
    s1 = f32x16{};
#pragma unroll
    for (int j = 0; j < KST; ++j) {
      const u32x4 a0 = *(const u32x4*)(K + k_rd[j]);
      const u32x4 a1 = *(const u32x4*)(K + k_rd[j] + 32 * RB);
      s0 = mfma32x32x16(T{}, a0, qop[j], s0);
      s1 = mfma32x32x16(T{}, a1, qop[j], s1);
#pragma unroll
      for (int p = 0; p < NP; ++p)
        if ((p * KST) / NP == j) piece(p);
    }
  };
  auto no_piece = [](int) {};
  // keys past this lane's last visible key -> -inf (diagonal / ragged blocks)
  // (each compare feeds its select at once: compares hoisted ahead of the
  // selects would hold 32 lane masks in scalar registers)
  auto mask = [&](f32x16& s0, f32x16& s1, int key0) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int key = key0 + ((j & 15) >> 2) * 8 + 4 * h + (j & 3);
      if (key > lim) s0[j] = -INFINITY;
      if (key + 32 > lim) s1[j] = -INFINITY;
    }
  };
  // row max over the 64 keys: a lane-local tree plus the partner half of the wave
  // (a three-input tree, 32 values in 16 v_maximum3; pairs of two-input
  // maxima had compiled to 21, several of them with a repeated operand)
  auto rowmax = [&](const f32x16& s0, const f32x16& s1) {
    auto mx3 = [](float x, float y, float z) {
      return __builtin_elementwise_maximum(__builtin_elementwise_maximum(x, y), z);
    };
    float v[32];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      v[j] = s0[j];
      v[16 + j] = s1[j];
    }
    float t[12];
#pragma unroll
    for (int i = 0; i < 10; ++i) t[i] = mx3(v[3 * i], v[3 * i + 1], v[3 * i + 2]);
    t[10] = v[30];
    t[11] = v[31];
    float u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = mx3(t[3 * i], t[3 * i + 1], t[3 * i + 2]);
    return half_swap_max(__builtin_elementwise_maximum(mx3(u[0], u[1], u[2]), u[3]));
  };
  // lazy running max: (l, o) are rescaled only when the block max exceeds m by
  // 2^8 (p <= 2^8 otherwise, well inside f16)
  auto raise_max = [&](float rmax) {
    const float smax = rmax * a.qk_scale;
    if (__any(smax > m + 8.0f)) {
      const float m_new = __builtin_elementwise_maximum(m, smax);
      const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m - m_new);   // row still sees nothing
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int e = 0; e < ET; ++e) o[e] *= alpha;
    }
  };
  // The work of one key block j (sa = raw scores of block j in, sb = scores
  // of block j + 1 out): the QK MFMAs of S_{j+1} and the PV MFMAs of block j
  // form one stream of NS MFMA slots, each reading its A operand from LDS
  // two slots ahead (an LDS read takes ~64 cycles, one MFMA slot of a wave
  // ~48 with two waves per SIMD, so a read issued one slot ahead stalls
  // every MFMA).  The exponentials of block j run under the QK slots
  // (P_j k-slots 0-2) and the first PV slots (k-slot 3), whose MFMAs need
  // them in that order; the next block's row max, which needs all of
  // S_{j+1}, fills the last PV slots.
  constexpr int NQK = 2 * KST, NPV = 4 * ET, NS = NQK + NPV;
  constexpr int PD = 2;                                  // LDS operand reads in flight ahead of the MFMA
  auto work = [&](auto parity, int j, f32x16& sa0, f32x16& sa1, f32x16& sb0, f32x16& sb1, float& rmax,
                  auto piece) {
    constexpr int P = decltype(parity)::value;           // j % S, known at compile time
    if (j >= wblk) {
      // (a wave past its last block still moves its share of the ring)
#pragma unroll
      for (int p = 0; p < NP; ++p) piece(p);
    } else {
      raise_max(rmax);
      // S_{j+1} is computed even on the wave's last block (its stage then
      // holds another block or stale keys and the scores are discarded):
      // one code path keeps the accumulators in place across iterations
      const char* K = kstage(PfParity<P + 1>{});
      const char* Vst = vstage(PfParity<P>{});
      // A operand of slot i: K rows (k-step i / 2, tile i % 2), then V^T
      // chunks (k-slot x / ET, d-tile x % ET)
      auto rd = [&](int i) -> u32x4 {
        if (i < NQK) return *(const u32x4*)(K + k_rd[i >> 1] + (i & 1) * 32 * RB);
        return pv_a(Vst, i - NQK);
      };
      const float mu = m == -INFINITY ? 0.f : m;           // rows with nothing visible yet
      const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
      u32x4 pop[4];
      float lb[4];
      // P_j k-slot ks = 2^(s c - m) rounded to f16, packed as the B operand
      // of the PV product (keys of S^T output registers 8 (ks % 2) .. + 8 of
      // tile ks / 2); its row sum is taken over the rounded weights
      auto ex = [&](int ks) {
        lb[ks] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j0 = (ks & 1) * 8 + 2 * i;
          const float x0 = ks < 2 ? sa0[j0] : sa1[j0];
          const float x1 = ks < 2 ? sa0[j0 + 1] : sa1[j0 + 1];
          const float p0 = fast_exp2(__builtin_fmaf(x0, a.qk_scale, -mu));
          const float p1 = fast_exp2(__builtin_fmaf(x1, a.qk_scale, -mu));
          const uint32_t w = pack2(F16{}, p0, p1);
          lb[ks] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), ones, lb[ks], false);
          pop[ks][i] = w;
        }
      };
      u32x4 buf[PD + 1];
#pragma unroll
      for (int i = 0; i < PD; ++i) buf[i] = rd(i);
      sb0 = f32x16{};
      sb1 = f32x16{};
      ex(0);
      ex(1);
      ex(2);
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        if (i + PD < NS) buf[(i + PD) % (PD + 1)] = rd(i + PD);
        const u32x4 av = buf[i % (PD + 1)];
        if (i < NQK) {
          if ((i & 1) == 0) sb0 = mfma32x32x16(T{}, av, qop[i >> 1], sb0);
          else sb1 = mfma32x32x16(T{}, av, qop[i >> 1], sb1);
          if (i & 1) {
#pragma unroll
            for (int p = 0; p < NP; ++p)
              if ((p * KST) / NP == (i >> 1)) piece(p);
          }
        } else {
          const int x = i - NQK;
          o[x % ET] = mfma32x32x16(F16{}, av, pop[x / ET], o[x % ET]);
        }
        if (i == NQK - 1) ex(3);
      }
      l += (lb[0] + lb[1]) + (lb[2] + lb[3]);
      // the next block's row max (unmasked; redone below on masked blocks)
      rmax = rowmax(sb0, sb1);
      // slot pattern: two reads ahead, then per slot one MFMA, the read two
      // slots on, the ring transfers after this k-step (QK slots), and the
      // VALU work: exponentials (transcendental unit) and the other VALU
      // instructions counted apart.  24 exponentials of P_j (k-slots 0-2)
      // and their 48 fma/pack/row-sum instructions go under the QK slots, 8
      // (k-slot 3) and 16 under the first half of the PV slots, the row max
      // (~19 instructions with the swap and the rescale test) under the rest.
      constexpr int TQ = (24 + NQK - 1) / NQK, VQ = (48 + NQK - 1) / NQK;
      constexpr int TP = (8 + 2 * ET - 1) / (2 * ET), VP1 = (16 + 2 * ET - 1) / (2 * ET);
      constexpr int VP2 = (24 + 2 * ET - 1) / (2 * ET);
      __builtin_amdgcn_sched_group_barrier(0x100, PD, 0);
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (i + PD < NS) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          if (kTrV && i + PD >= NQK) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // (two transposed reads)
        }
        if (kInlineRefill && i < NQK && (i & 1)) {
#pragma unroll
          for (int p = 0; p < NP; ++p)
            if ((p * KST) / NP == (i >> 1)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
        if (i < NQK) {
          __builtin_amdgcn_sched_group_barrier(0x400, TQ, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, VQ, 0);
        } else if (i < NQK + 2 * ET) {
          __builtin_amdgcn_sched_group_barrier(0x400, TP, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, VP1, 0);
        } else {
          __builtin_amdgcn_sched_group_barrier(0x002, VP2, 0);
        }
      }
      // (keeps the row sum inside this scheduling region: otherwise it sinks
      // below the branch that follows, where nothing overlaps it)
      asm volatile("" : "+v"(l));
      // (the scores of block wblk are discarded: no mask for them)
      if (j + 1 >= wfull && j + 1 < wblk) {
        mask(sb0, sb1, (j + 1) * kPfBN);
        rmax = rowmax(sb0, sb1);
      }
    }
  };

  f32x16 s0 = f32x16{}, s1 = f32x16{}, n0 = f32x16{}, n1 = f32x16{};
  float rmax = -INFINITY;
  auto first_scores = [&]() {
    if (wblk > 0) {
      qk(lk0, s0, s1, no_piece);
      if (wfull == 0) mask(s0, s1, 0);
      rmax = rowmax(s0, s1);
    }
  };
  // The work-group's last key block T = nblk - 1 runs after the loop: its
  // PV product alone (no next block's scores to compute).  When every row of
  // the wave sees at most the block's first 32 keys (a causal diagonal block
  // whose second half lies past the wave's rows, or a ragged last block), the
  // second key tile's weights are all zero and its exponentials and PV MFMAs
  // are skipped.  Its V stage is picked at run time (one block per group).
  const int wlim = a.causal ? min(a.Tk - 1, off + wrow0 + 31) : a.Tk - 1;   // the wave's last visible key
  auto work_last = [&](const char* Vstage, int j, const f32x16& sa0, const f32x16& sa1) {
    if (j >= wblk) return;
    raise_max(rmax);
    const float mu = m == -INFINITY ? 0.f : m;
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    u32x4 pop[4];
    float lb[4];
    auto ex = [&](int ks) {
      lb[ks] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j0 = (ks & 1) * 8 + 2 * i;
        const float x0 = ks < 2 ? sa0[j0] : sa1[j0];
        const float x1 = ks < 2 ? sa0[j0 + 1] : sa1[j0 + 1];
        const float p0 = fast_exp2(__builtin_fmaf(x0, a.qk_scale, -mu));
        const float p1 = fast_exp2(__builtin_fmaf(x1, a.qk_scale, -mu));
        const uint32_t w = pack2(F16{}, p0, p1);
        lb[ks] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), ones, lb[ks], false);
        pop[ks][i] = w;
      }
    };
    auto rdv = [&](int x) { return pv_a(Vstage, x); };
    auto pv = [&](auto nks) {
      constexpr int NX = decltype(nks)::value * ET;
      u32x4 buf[3];
      buf[0] = rdv(0);
      buf[1] = rdv(1);
#pragma unroll
      for (int ks = 0; ks < decltype(nks)::value; ++ks) ex(ks);
#pragma unroll
      for (int x = 0; x < NX; ++x) {
        if (x + 2 < NX) buf[(x + 2) % 3] = rdv(x + 2);
        o[x % ET] = mfma32x32x16(F16{}, buf[x % 3], pop[x / ET], o[x % ET]);
      }
    };
    if (wlim < j * kPfBN + 32) {
      pv(std::integral_constant<int, 2>{});
      l += lb[0] + lb[1];
    } else {
      pv(std::integral_constant<int, 4>{});
      l += (lb[0] + lb[1]) + (lb[2] + lb[3]);
    }
  };
  // scores of block nfb (the last): in s after an even number of full blocks, in n after an odd one
  const int nfb = nblk > 0 ? nblk - 1 : 0;
  auto last_block = [&](const char* Vstage) {
    f32x16 t0, t1;
    const bool in_n = (nfb & 1) != 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      t0[i] = in_n ? n0[i] : s0[i];
      t1[i] = in_n ? n1[i] : s1[i];
    }
    work_last(Vstage, nfb, t0, t1);
  };

  if constexpr (S == 4) {
    // Four-stage ring, one barrier per two key blocks.  Block j needs K_{j+1}
    // (scores of the next block) and V_j.  The barrier before blocks j, j+1
    // (j even) retires blocks j-2, j-1; the stages they read are refilled
    // with K_{j+3}, K_{j+4}, V_{j+2}, V_{j+3} from inside the two blocks'
    // QK products: two blocks of lead, waited for (vmcnt(0)) at the next
    // barrier.
    auto super = [&](auto parity, int j, bool second) {
      constexpr int P = decltype(parity)::value;          // 0 or 2
      wait_vmcnt<0>();                                      // this wave's DMA of blocks j, j+1 landed
      ring_barrier();                                     // everyone's landed; blocks j-2, j-1 retired
      // refills: K_{j+3}, V_{j+2} from block j's QK, K_{j+4}, V_{j+3} from
      // block j+1's (all into stages retired at this barrier)
      auto piece0 = [&](int p) {
        if (p < NK) issue_k1(j + 3, kstage(PfParity<P + 3>{}), p);
        else issue_v1(j + 2, vstage(PfParity<P + 2>{}), p - NK);
      };
      auto piece1 = [&](int p) {
        if (p < NK) issue_k1(j + 4, kstage(PfParity<P>{}), p);
        else issue_v1(j + 3, vstage(PfParity<P + 3>{}), p - NK);
      };
      work(PfParity<P>{}, j, s0, s1, n0, n1, rmax, piece0);
      if (second) {
        work(PfParity<P + 1>{}, j + 1, n0, n1, s0, s1, rmax, piece1);
      } else {
#pragma unroll
        for (int p = 0; p < NP; ++p) piece1(p);
      }
    };
    // Prologue: K_0's transfers first, then q (its 32 rows per load
    // instruction take the memory pipeline a while), then V_0, K_1, K_2,
    // V_1.  The first scores wait for K_0 and q only; the rest land under
    // them.  (Loads retire in order, so vmcnt(later) covers exactly K_0 and
    // q.)
    if (nblk > 0) {
      if constexpr (ROPE == kRopeNone) {
        // q comes through LDS: each wave's 32 rows by 1 KB LDS DMA (whole
        // rows, swizzled like the K stages) into a stage the first blocks do
        // not use yet (V_1's, K_3's, V_2's, V_3's; 2 waves each), then read in
        // the operand layout.  Loaded straight into registers, each of a
        // wave's q instructions touched 32 rows (256 cache-line requests per
        // wave instead of 64), and the memory pipeline worked through them
        // ahead of the ring's first transfers.  Rows past Tq read as zeros.
        issue_k(0, lk0);
        issue_v(0, lv0);
        issue_k(1, lk1);
        issue_k(2, lk2);
        char* qst = ((wave >> 1) == 0 ? lv1 : (wave >> 1) == 1 ? lk3 : (wave >> 1) == 2 ? lv2 : lv3) +
                    (wave & 1) * 32 * RB;
        {
          const int r0w = q0 + rg * 32;
          const int nrow = max(0, min(32, a.Tq - r0w));
          const int bytes = nrow > 0 ? (nrow - 1) * (int)a.q_sm + RB : 0;
          const __amdgpu_buffer_rsrc_t rsq = __builtin_amdgcn_make_buffer_rsrc(
              (void*)(a.q + b * a.q_sb + (int64_t)hq * a.q_sh + (int64_t)min(r0w, a.Tq - 1) * a.q_sm), 0, bytes,
              kBufferFlags);
#pragma unroll
          for (int i = 0; i < 32 * RB / 1024; ++i) {
            const int r = i * ROWS_PER_DMA + lane / NC;
            const int voff = r * (int)a.q_sm + (((lane % NC) ^ (r % NC)) * 16);
            char* dst = qst + i * 1024;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsq, dst, 16, voff, 0, 0, 0);
          }
        }
        wait_vmcnt<0>();                                  // this wave's q (and K_0 .. K_2, V_0) landed
#pragma unroll
        for (int j = 0; j < KST; ++j) qop[j] = *(const u32x4*)(qst + k_rd[j]);
        ring_barrier();                                   // every wave's q read and K_0 landed
        issue_v(1, lv1);                                  // into the q stage just read
        first_scores();
      } else {
        issue_k(0, lk0);
        load_q();
        __builtin_amdgcn_sched_barrier(0);
        issue_v(0, lv0);
        issue_k(1, lk1);
        issue_k(2, lk2);
        issue_v(1, lv1);
        wait_vmcnt<2 * NK + 2 * NV>();
        rope_q_apply<D, T, ROPE>(a, qop, rq, h);
        ring_barrier();
        first_scores();
      }
    } else {
      load_q();
    }
    // blocks 0 .. nblk - 2 in full steps, then the last block's PV product
    int j = 0;
    for (; j + 3 < nfb; j += 4) {
      super(PfParity<0>{}, j, true);
      super(PfParity<2>{}, j + 2, true);
    }
    if (j < nfb) super(PfParity<0>{}, j, j + 1 < nfb);
    if (j + 2 < nfb) super(PfParity<2>{}, j + 2, false);
    if (nblk > 0) {
      wait_vmcnt<0>();                                      // this wave's part of V_{nblk-1} landed
      ring_barrier();
      const int st = nfb & 3;
      last_block(st == 0 ? lv0 : st == 1 ? lv1 : st == 2 ? lv2 : lv3);
    }
  } else {
    // Two-stage ring, one barrier per block: the barrier before block j
    // retires block j - 1, whose stages block j's QK product refills with
    // K_{j+2} and V_{j+1}.
    auto step = [&](auto parity, int j, f32x16& sa0, f32x16& sa1, f32x16& sb0, f32x16& sb1) {
      constexpr int P = decltype(parity)::value;
      wait_vmcnt<0>();                                      // this wave's part of K_{j+1}, V_j landed
      ring_barrier();
      issue_k(j + 2, kstage(PfParity<P>{}));             // K_{j+2}, V_{j+1} into the stages retired here
      issue_v(j + 1, vstage(PfParity<P + 1>{}));
      pack_vstage(vstage(PfParity<P>{}));                // variant 2: V_j's image (its rows have landed)
      work(parity, j, sa0, sa1, sb0, sb1, rmax, no_piece);
    };
    // Prologue as on the four-stage ring: K_0, q, then V_0 and K_1 landing
    // under the first scores.
    if (nblk > 0) {
      issue_k(0, lk0);
      load_q();
      __builtin_amdgcn_sched_barrier(0);
      issue_v(0, lv0);
      issue_k(1, lk1);
      wait_vmcnt<NK + NV>();
      if constexpr (ROPE != kRopeNone) rope_q_apply<D, T, ROPE>(a, qop, rq, h);
      ring_barrier();
      first_scores();
    } else {
      load_q();
    }
    int j = 0;
    for (; j + 1 < nfb; j += 2) {
      step(PfParity<0>{}, j, s0, s1, n0, n1);
      step(PfParity<1>{}, j + 1, n0, n1, s0, s1);
    }
    if (j < nfb) step(PfParity<0>{}, j, s0, s1, n0, n1);
    if (nblk > 0) {
      wait_vmcnt<0>();                                      // this wave's part of V_{nblk-1} landed
      ring_barrier();
      char* vlast = (nfb & 1) ? lv1 : lv0;
      pack_vstage(vlast);   // (variant 2; one copy: a stage picked by a branch here kept the scores on the stack)
      last_block(vlast);
    }
  }

  // ---- normalise and store.  The lane owns query qi, d = 32 e + 8 (j / 4) +
  // 4 h + j % 4 of O^T; the wave's 32 x D tile goes through LDS (16-byte
  // chunks swizzled by row) so that every global store writes whole rows.
  wait_vmcnt<0>();                                         // every ring transfer (empty ones fill zeros) landed
  ring_barrier();                                        // every wave is done with the ring
  {
    constexpr int NCH = D / 8;                           // 16-byte chunks per row
    char* tile = (wave >> 1) == 0 ? lk0 : (wave >> 1) == 1 ? lk1 : (wave >> 1) == 2 ? lk2 : lk3;
    tile += (wave & 1) * 32 * RB;
    const float lt = half_swap_sum(l);
    const float inv = lt == 0.f ? 0.f : 1.0f / lt;
#pragma unroll
    for (int e = 0; e < ET; ++e)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        if (32 * e + 8 * g4 >= D) continue;            // zero-padded image dimensions (D = 16)
        u32x2 w;
        w[0] = pack2(T{}, o[e][4 * g4 + 0] * inv, o[e][4 * g4 + 1] * inv);
        w[1] = pack2(T{}, o[e][4 * g4 + 2] * inv, o[e][4 * g4 + 3] * inv);
        *(u32x2*)(tile + l32 * RB + (((4 * e + g4) ^ (l32 % NCH)) * 16) + h * 8) = w;
      }
    constexpr int RPI = 64 / NCH;                        // rows per 64-lane pass
    const int c = lane % NCH;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int row = i * RPI + lane / NCH;
      const u32x4 w = *(const u32x4*)(tile + row * RB + ((c ^ (row % NCH)) * 16));
      const int qrow = q0 + rg * 32 + row;
      if (qrow < a.Tq)
        *(u32x4*)(a.out + b * a.o_sb + (int64_t)hq * a.o_sh + (int64_t)qrow * a.o_sm + c * 16) = w;
    }
  }
}

}  // namespace sia
