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
//  * A work-group is 4 waves x 32 query rows (BM = 128) of one (b, hq); it
//    walks key blocks of BN = 64 staged in LDS, double-buffered: K row-major
//    and V transposed (V^T, key-contiguous, f16), both with padded rows so
//    the MFMA operand reads are bank-conflict free.  V is transposed (and
//    converted) in registers before its LDS write.
//  * Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (keys as rows,
//    its 32 queries as columns), so every lane owns one query: the row max is
//    a lane-local max plus one xor-32 exchange, and P^T feeds O^T += V^T P^T
//    straight from registers (the key order of its k-slots matches the S^T
//    output layout, and the V^T reads use the same order).
//  * Blocks are issued heaviest-first (the causal diagonal makes late query
//    blocks the longest), and the query heads that share a KV head are placed
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
  const char* v; int64_t v_sb, v_sh, v_sn;
  char* out; int64_t o_sb, o_sh, o_sm;
  int32_t B, Hq, Hkv, G, Tq, Tk, causal;
  float qk_scale;                               // sm_scale * log2(e)
  int32_t nqblk;                                // ceil(Tq / 128)
  int32_t remap;                                // XCD-aware block order
};

constexpr int kPfBM = 128;   // query rows per work-group (4 waves x 32)
constexpr int kPfBN = 64;    // keys per block

template <int D>
struct PrefillLds {
  static constexpr int KROW = D + 8;          // padded K row (elements)
  static constexpr int VROW = kPfBN + 4;      // padded V^T row (elements)
  static constexpr int KSZ = kPfBN * KROW;
  static constexpr int VSZ = D * VROW;
};

// Cooperative global -> register load of one K/V block (256 threads).
template <int D>
struct KvRegs {
  static constexpr int KCH = D / 32;          // 16-byte K chunks per thread
  static constexpr int VGRP = (16 * (D / 8) + 255) / 256;   // (4-key, 8-d) V groups per thread
  u32x4 k[KCH];
  u32x4 v[VGRP][4];
};

template <int D>
__device__ __forceinline__ void load_kv_block(const PrefillArgs& a, const char* kb, const char* vb, int key0,
                                              KvRegs<D>& r) {
  const int t = threadIdx.x;
  const bool full = key0 + kPfBN <= a.Tk;          // uniform: no per-key predicate needed
  {
    const int key = key0 + (t >> 2);
    const int d0 = (t & 3) * (D / 4);
    const char* src = kb + (int64_t)(full ? key : min(key, a.Tk - 1)) * a.k_sn + d0 * 2;
#pragma unroll
    for (int c = 0; c < KvRegs<D>::KCH; ++c) {
      const u32x4 x = *(const u32x4*)(src + 16 * c);
      r.k[c] = (full || key < a.Tk) ? x : u32x4{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int g = 0; g < KvRegs<D>::VGRP; ++g) {
    const int idx = t + 256 * g;
    const int c8 = idx % (D / 8), kg = idx / (D / 8);
    if (kg < 16) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int key = key0 + 4 * kg + rr;
        const u32x4 x = *(const u32x4*)(vb + (int64_t)(full ? key : min(key, a.Tk - 1)) * a.v_sn + c8 * 16);
        r.v[g][rr] = (full || key < a.Tk) ? x : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
}

// Element `hs` (0 low, 1 high) of two packed 16-bit words as one f16 pair.
// bf16 sources are widened to f32, clamped to the f16 range and rounded: the
// PV product runs in f16 so that P keeps 11 significant bits.
__device__ __forceinline__ uint32_t to_f16_pair(F16, uint32_t a, uint32_t b, int hs) { return gather16(a, b, hs); }
__device__ __forceinline__ uint32_t to_f16_pair(BF16, uint32_t a, uint32_t b, int hs) {
  const float fa = __builtin_bit_cast(float, hs ? (a & 0xffff0000u) : (a << 16));
  const float fb = __builtin_bit_cast(float, hs ? (b & 0xffff0000u) : (b << 16));
  return pack2(F16{}, __builtin_amdgcn_fmed3f(fa, -65504.0f, 65504.0f),
               __builtin_amdgcn_fmed3f(fb, -65504.0f, 65504.0f));
}

template <int D, class T>
__device__ __forceinline__ void store_kv_block(const KvRegs<D>& r, uint16_t* lk, uint16_t* lv) {
  using L = PrefillLds<D>;
  const int t = threadIdx.x;
  {
    const int key = t >> 2;
    const int d0 = (t & 3) * (D / 4);
#pragma unroll
    for (int c = 0; c < KvRegs<D>::KCH; ++c) *(u32x4*)(lk + key * L::KROW + d0 + 8 * c) = r.k[c];
  }
#pragma unroll
  for (int g = 0; g < KvRegs<D>::VGRP; ++g) {
    const int idx = t + 256 * g;
    const int c8 = idx % (D / 8), kg = idx / (D / 8);
    if (kg < 16) {
      // 4 keys x 8 d -> for each d one 64-bit word holding the 4 keys
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int p = x >> 1, hs = x & 1;
        u32x2 w;
        w[0] = to_f16_pair(T{}, r.v[g][0][p], r.v[g][1][p], hs);
        w[1] = to_f16_pair(T{}, r.v[g][2][p], r.v[g][3][p], hs);
        *(u32x2*)(lv + (c8 * 8 + x) * L::VROW + 4 * kg) = w;
      }
    }
  }
}

template <int D, class T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prefill_fwd(const PrefillArgs a) {
  using L = PrefillLds<D>;
  constexpr int KST = D / 16;    // QK k-steps
  constexpr int ET = D / 32;     // O^T d-tiles
  __shared__ __attribute__((aligned(16))) uint16_t lk[2][L::KSZ];
  __shared__ __attribute__((aligned(16))) uint16_t lv[2][L::VSZ];

  // ---- block -> (query block, b, hq), heaviest first, KV-head groups per XCD
  int lin = blockIdx.x;
  if (a.remap) {
    const int xcd = lin & 7, slot = lin >> 3;
    lin = ((slot / a.G) * 8 + xcd) * a.G + slot % a.G;
  }
  const int g = lin % a.G;
  int rest = lin / a.G;
  const int hkv = rest % a.Hkv;
  rest /= a.Hkv;
  const int b = rest % a.B;
  const int qblk = a.nqblk - 1 - rest / a.B;
  const int hq = hkv * a.G + g;

  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int off = a.Tk - a.Tq;                           // bottom-right causal offset
  const int q0 = qblk * kPfBM;
  const int qi = q0 + wave * 32 + l32;                   // this lane's query row

  // ---- Q^T operand (B of S^T = K Q^T): query qi, d = 16 j + 8 h + [0, 8)
  u32x4 qop[KST];
  {
    const char* qp = a.q + b * a.q_sb + (int64_t)hq * a.q_sh + (int64_t)min(qi, a.Tq - 1) * a.q_sm + 16 * h;
#pragma unroll
    for (int j = 0; j < KST; ++j) qop[j] = qi < a.Tq ? *(const u32x4*)(qp + 32 * j) : u32x4{0u, 0u, 0u, 0u};
  }

  const int kend = a.causal ? min(a.Tk, off + q0 + kPfBM) : a.Tk;
  const int nblk = kend > 0 ? (kend + kPfBN - 1) / kPfBN : 0;
  const int wrow0 = q0 + wave * 32;                      // this wave's first row
  const int wend = a.causal ? min(a.Tk, off + wrow0 + 32) : a.Tk;   // keys this wave can see

  const char* kb = a.k + b * a.k_sb + (int64_t)hkv * a.k_sh;
  const char* vb = a.v + b * a.v_sb + (int64_t)hkv * a.v_sh;

  f32x16 o[ET];
#pragma unroll
  for (int e = 0; e < ET; ++e) o[e] = f32x16{};
  float m = -INFINITY, l = 0.f;

  // Two register staging sets: block it+2 is requested while block it is
  // computed and block it+1 (already in registers) is written to LDS after it.
  KvRegs<D> kvA, kvB;
  if (nblk > 0) {
    load_kv_block<D>(a, kb, vb, 0, kvA);
    store_kv_block<D, T>(kvA, lk[0], lv[0]);
  }
  if (nblk > 1) load_kv_block<D>(a, kb, vb, kPfBN, kvB);
  __syncthreads();

  auto step = [&](int it, KvRegs<D>& refill, const KvRegs<D>& next) {
    const int buf = it & 1;
    const int key0 = it * kPfBN;
    if (it + 2 < nblk) load_kv_block<D>(a, kb, vb, key0 + 2 * kPfBN, refill);
      if (key0 < wend) {
        const uint16_t* K = lk[buf];
        const uint16_t* V = lv[buf];
        // ---- S^T = K Q^T for keys [key0, key0 + 64): two 32-key tiles
        f32x16 s0 = f32x16{}, s1 = f32x16{};
  #pragma unroll
        for (int j = 0; j < KST; ++j) {
          const u32x4 a0 = *(const u32x4*)(K + l32 * L::KROW + 16 * j + 8 * h);
          const u32x4 a1 = *(const u32x4*)(K + (32 + l32) * L::KROW + 16 * j + 8 * h);
          s0 = mfma32x32x16(T{}, a0, qop[j], s0);
          s1 = mfma32x32x16(T{}, a1, qop[j], s1);
        }
        // raw scores; the scale is folded into the exponent (c > 0 keeps the max)
        float sc[32];
  #pragma unroll
        for (int j = 0; j < 16; ++j) { sc[j] = s0[j]; sc[16 + j] = s1[j]; }
        // mask keys past Tk and, on the causal diagonal, keys after the row's position
        const bool need_mask = key0 + kPfBN > a.Tk || (a.causal && key0 + kPfBN - 1 > off + wrow0);
        if (need_mask) {
          const int lim = a.causal ? min(a.Tk - 1, off + qi) : a.Tk - 1;
  #pragma unroll
          for (int j = 0; j < 32; ++j) {
            const int key = key0 + (j >> 4) * 32 + ((j & 15) >> 2) * 8 + 4 * h + (j & 3);
            if (key > lim) sc[j] = -INFINITY;
          }
        }
        float rmax = fmaxf(sc[0], sc[1]);
  #pragma unroll
        for (int j = 2; j < 32; j += 2) rmax = fmaxf(rmax, fmaxf(sc[j], sc[j + 1]));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 32));         // the partner lane holds the other 32 keys
        const float smax = rmax * a.qk_scale;
        if (__any(smax > m + 8.0f)) {                      // lazy max (p <= 2^8 otherwise)
          const float m_new = fmaxf(m, smax);
          const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m - m_new);   // row still sees nothing
          m = m_new;
          l *= alpha;
  #pragma unroll
          for (int e = 0; e < ET; ++e) o[e] *= alpha;
        }
        const float mu = m == -INFINITY ? 0.f : m;         // rows with nothing visible yet
        const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
        u32x4 pop[4];
  #pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j0 = (ks >> 1) * 16 + (ks & 1) * 8 + 2 * i;
            const float p0 = fast_exp2(__builtin_fmaf(sc[j0], a.qk_scale, -mu));
            const float p1 = fast_exp2(__builtin_fmaf(sc[j0 + 1], a.qk_scale, -mu));
            const uint32_t w = pack2(F16{}, p0, p1);
            // the row sum is taken over the rounded weights the MFMA uses, so the
            // output stays an exact convex combination of V rows
            l = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), ones, l, false);
            pop[ks][i] = w;
          }
        }
        // ---- O^T += V^T P^T
  #pragma unroll
        for (int e = 0; e < ET; ++e) {
  #pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const uint16_t* vp = V + (32 * e + l32) * L::VROW + (ks >> 1) * 32 + (ks & 1) * 16 + 4 * h;
            const u32x2 lo = *(const u32x2*)vp;
            const u32x2 hi = *(const u32x2*)(vp + 8);
            const u32x4 va = u32x4{lo[0], lo[1], hi[0], hi[1]};
            o[e] = mfma32x32x16(F16{}, va, pop[ks], o[e]);
          }
        }
      }
    // buffer buf^1 was last read before the previous barrier: refill it now
    if (it + 1 < nblk) store_kv_block<D, T>(next, lk[buf ^ 1], lv[buf ^ 1]);
    __syncthreads();
  };
  for (int it = 0; it < nblk; it += 2) {
    step(it, kvA, kvB);
    if (it + 1 < nblk) step(it + 1, kvB, kvA);
  }

  // ---- normalise and store: lane owns query qi, d = 32 e + 8 (j / 4) + 4 h + j % 4
  const float lt = l + __shfl_xor(l, 32);
  if (qi < a.Tq) {
    const float inv = lt == 0.f ? 0.f : 1.0f / lt;
    char* op = a.out + b * a.o_sb + (int64_t)hq * a.o_sh + (int64_t)qi * a.o_sm;
#pragma unroll
    for (int e = 0; e < ET; ++e)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2 w;
        w[0] = pack2(T{}, o[e][4 * g4 + 0] * inv, o[e][4 * g4 + 1] * inv);
        w[1] = pack2(T{}, o[e][4 * g4 + 2] * inv, o[e][4 * g4 + 3] * inv);
        *(u32x2*)(op + (32 * e + 8 * g4 + 4 * h) * 2) = w;
      }
  }
}

}  // namespace sia
