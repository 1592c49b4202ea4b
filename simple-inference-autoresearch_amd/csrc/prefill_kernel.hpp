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
//  * A work-group of prefill_fwd is 4 waves x 32 query rows (BM = 128) of one
//    (b, hq); it walks key blocks of BN = 64 through two LDS stages filled by
//    buffer_load ... lds (global -> LDS DMA: no VGPR staging, no VALU), the
//    next block's DMA in flight while the current one is computed.
//  * LDS is chunk-major: the 16-byte chunk c of row r sits at byte
//    c * rows * 16 + r * 16, so the 32 lanes that read one MFMA operand read
//    32 consecutive chunks (no bank conflict, no swizzle arithmetic) and
//    every LDS address is a per-lane base plus an immediate.
//  * Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16 (keys as rows,
//    its 32 queries as columns), so every lane owns one query: the row max is
//    a lane-local v_maximum3 tree plus one v_permlane32_swap, and P^T feeds
//    O^T += V^T P^T straight from registers (the key order of its k-slots
//    matches the S^T output layout; the V^T images store keys in that order).
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
  const char* vimg;                             // V^T block images (prefill_pack_v)
  char* out; int64_t o_sb, o_sh, o_sm;
  int32_t B, Hq, Hkv, G, Tq, Tk, causal;
  float qk_scale;                               // sm_scale * log2(e)
  int32_t nqblk;                                // ceil(Tq / 128)
  int32_t nkb;                                  // ceil(Tk / 64)
  int32_t remap;                                // XCD-aware block order
};

struct PackArgs {
  const char* v; int64_t v_sb, v_sh, v_sn;      // byte strides; head_dim contiguous
  char* vimg;
  int32_t Hkv, Tk, nkb;
  int64_t nblocks;                              // B * Hkv * nkb
};

constexpr int kPfBM = 128;   // query rows per work-group (4 waves x 32)
constexpr int kPfBN = 64;    // keys per block
constexpr int kBufferFlags = 0x00020000;   // gfx9 raw buffer resource word 3 (32-bit data, no swizzle)

// Bytes of one K block (64 rows of D) and of one V^T block image.
template <int D>
constexpr int pf_block_bytes() { return kPfBN * D * 2; }

// Key (0..63 within its block) held by element i (0..7) of image chunk c: the
// keys of 16-key group c/2 in the order of the S^T output registers of lanes
// of half c%2, i.e. 4 (c%2) + {0, 1, 2, 3, 8, 9, 10, 11}.
__device__ __forceinline__ int image_key(int c, int i) { return 16 * (c >> 1) + 4 * (c & 1) + (i & 3) + 8 * (i >> 2); }

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

// V (B, Hkv, Tk, D) -> images [B][Hkv][nkb]: image chunk c of dimension d
// (16 bytes at (c * D + d) * 16) holds keys image_key(c, 0..7) of d as f16;
// keys at or past Tk are zero.  One thread makes 8 (d) x 8 (keys).
template <int D, class T>
__global__ __launch_bounds__(256) void prefill_pack_v(const PackArgs a) {
  constexpr int DG = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t blk = gid / (8 * DG);
  if (blk >= a.nblocks) return;
  const int r = (int)(gid % (8 * DG));
  const int c = r / DG, dg = r % DG;
  const int kb = (int)(blk % a.nkb);
  const int64_t bh = blk / a.nkb;
  const int hkv = (int)(bh % a.Hkv);
  const int64_t b = bh / a.Hkv;
  const char* src = a.v + b * a.v_sb + (int64_t)hkv * a.v_sh + dg * 16;
  u32x4 in[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = kb * kPfBN + image_key(c, i);
    in[i] = key < a.Tk ? *(const u32x4*)(src + (int64_t)key * a.v_sn) : u32x4{0u, 0u, 0u, 0u};
  }
  char* dst = a.vimg + blk * pf_block_bytes<D>() + (int64_t)(c * D + 8 * dg) * 16;
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    u32x4 w;
#pragma unroll
    for (int m = 0; m < 4; ++m) w[m] = to_f16_pair(T{}, in[2 * m][x >> 1], in[2 * m + 1][x >> 1], x & 1);
    *(u32x4*)(dst + 16 * x) = w;
  }
}

template <int S>
struct PfStage {
  static constexpr int value = S;
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

template <int D, class T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prefill_fwd(const PrefillArgs a) {
  constexpr int KST = D / 16;                   // QK k-steps
  constexpr int ET = D / 32;                    // O^T d-tiles
  constexpr int BLK = pf_block_bytes<D>();
  constexpr int NDMA = BLK / 1024 / 4;          // 1 KB DMA instructions per wave per tensor and block
  // chunk-major stages: K chunk c of key row r at c * 1024 + r * 16 (64 rows);
  // V^T image chunk c of dimension d at c * D * 16 + d * 16
  __shared__ __attribute__((aligned(1024))) char lk0[BLK], lk1[BLK], lv0[BLK], lv1[BLK];

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
  const char* vimg = a.vimg + ((int64_t)b * a.Hkv + hkv) * a.nkb * BLK;
  const int k_voff = lane * (int)a.k_sn;                // DMA lane = key row

  // DMA of block `blk` into one stage: wave w moves K chunks [w NDMA, (w+1) NDMA)
  // (64 rows each; rows past Tk read as zero through the buffer bound) and the
  // same range of 1 KB pieces of the V^T image.
  auto issue = [&](int blk, char* LK, char* LV) {
    const int key0 = blk * kPfBN;
    const int rows = min(kPfBN, a.Tk - key0);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(kb + (int64_t)key0 * a.k_sn), 0, rows * (int)a.k_sn, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)(vimg + (int64_t)blk * BLK), 0, BLK, kBufferFlags);
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      const int c = wave * NDMA + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, LK + c * 1024, 16, k_voff, c * 16, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, LV + c * 1024, 16, lane * 16, c * 1024, 0, 0);
    }
  };

  f32x16 o[ET];
#pragma unroll
  for (int e = 0; e < ET; ++e) o[e] = f32x16{};
  float m = -INFINITY, l = 0.f;

  auto compute = [&](const char* K, const char* V, int key0) {
    // ---- S^T = K Q^T for keys [key0, key0 + 64): two 32-key tiles
    f32x16 s0 = f32x16{}, s1 = f32x16{};
    const char* kr = K + h * 1024 + l32 * 16;
#pragma unroll
    for (int j = 0; j < KST; ++j) {
      const u32x4 a0 = *(const u32x4*)(kr + j * 2048);
      const u32x4 a1 = *(const u32x4*)(kr + j * 2048 + 512);
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
    float mx[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      mx[j] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(sc[4 * j], sc[4 * j + 1]),
                                            __builtin_elementwise_maximum(sc[4 * j + 2], sc[4 * j + 3]));
    float rmax = __builtin_elementwise_maximum(
        __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx[0], mx[1]),
                                      __builtin_elementwise_maximum(mx[2], mx[3])),
        __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx[4], mx[5]),
                                      __builtin_elementwise_maximum(mx[6], mx[7])));
    rmax = half_swap_max(rmax);                        // the partner lane holds the other 32 keys
    const float smax = rmax * a.qk_scale;
    if (__any(smax > m + 8.0f)) {                      // lazy max (p <= 2^8 otherwise)
      const float m_new = __builtin_elementwise_maximum(m, smax);
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
    // ---- O^T += V^T P^T: operand chunk 2 ks + h of dimension 32 e + l32
    const char* vr = V + h * D * 16 + l32 * 16;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int e = 0; e < ET; ++e) {
        const u32x4 va = *(const u32x4*)(vr + ks * 2 * D * 16 + e * 512);
        o[e] = mfma32x32x16(F16{}, va, pop[ks], o[e]);
      }
    }
  };

  // One pipeline step: start the DMA of block it + 1 into the other stage
  // (last read before the previous barrier), compute block it, then wait for
  // this wave's DMA and meet the other waves (their DMA done, their reads of
  // this stage finished).
  auto step = [&](auto stage, int it) {
    constexpr int S = decltype(stage)::value;
    if (it + 1 < nblk) issue(it + 1, S ? lk0 : lk1, S ? lv0 : lv1);
    const int key0 = it * kPfBN;
    if (key0 < wend) compute(S ? lk1 : lk0, S ? lv1 : lv0, key0);
    __builtin_amdgcn_s_waitcnt(0x0f70);                // vmcnt(0)
    __syncthreads();
  };

  if (nblk > 0) {
    issue(0, lk0, lv0);
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
  }
  for (int it = 0; it < nblk; it += 2) {
    step(PfStage<0>{}, it);
    if (it + 1 < nblk) step(PfStage<1>{}, it + 1);
  }

  // ---- normalise and store: lane owns query qi, d = 32 e + 8 (j / 4) + 4 h + j % 4
  const float lt = half_swap_sum(l);
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
