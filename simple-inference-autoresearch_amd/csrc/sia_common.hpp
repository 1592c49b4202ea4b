// Shared device/host helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "sia_attention.h"

namespace sia {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// Element-type tags.  `bytes` is the storage size; the MFMA input type of a
// 16-bit tag is itself, int8 K/V feed the f16 MFMA after an exact conversion.
struct F16 { static constexpr int bytes = 2; static constexpr int code = SIA_F16; };
struct BF16 { static constexpr int bytes = 2; static constexpr int code = SIA_BF16; };
struct I8 { static constexpr int bytes = 1; static constexpr int code = SIA_I8; };
struct F32 { static constexpr int bytes = 4; static constexpr int code = SIA_F32; };

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float to_f32(F16, uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}
__device__ __forceinline__ float to_f32(BF16, uint16_t bits) {
  return __builtin_bit_cast(float, (uint32_t)bits << 16);
}

// Round-to-nearest-even conversions of two floats into one packed 16-bit pair
// (low half = a).
__device__ __forceinline__ uint32_t pack2(F16, float a, float b) {
  f16x2 h = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint32_t pack2(BF16, float a, float b) {
  bf16x2 h = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ float lo_f32(F16, uint32_t w) { return to_f32(F16{}, (uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float hi_f32(F16, uint32_t w) { return to_f32(F16{}, (uint16_t)(w >> 16)); }
__device__ __forceinline__ float lo_f32(BF16, uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float hi_f32(BF16, uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__device__ __forceinline__ void store_out(F16, char* p, float x) {
  *(_Float16*)p = (_Float16)x;
}
__device__ __forceinline__ void store_out(BF16, char* p, float x) {
  *(__bf16*)p = (__bf16)x;
}
__device__ __forceinline__ void store_out(F32, char* p, float x) { *(float*)p = x; }

// Four signed int8 in `w`, bytes (b0, b1) or (b2, b3), to an exact f16 pair.
// 0x64XX as f16 is 1024 + XX; biasing the byte by 0x80 maps x in [-128,127] to
// 1152 + x, which is exact, and the packed subtraction of 1152 is exact too.
__device__ __forceinline__ uint32_t i8pair_to_f16x2(uint32_t w_xor80, uint32_t sel) {
  uint32_t biased = __builtin_amdgcn_perm(0x64646464u, w_xor80, sel);
  f16x2 h = __builtin_bit_cast(f16x2, biased);
  const f16x2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  return __builtin_bit_cast(uint32_t, h + bias);
}
// Byte `e` of words a (low half) and b (high half) as an exact f16 pair.
__device__ __forceinline__ uint32_t i8gather_to_f16x2(uint32_t a, uint32_t b, int e) {
  // selector: result byte0 = a.byte(e), byte1 = 0, byte2 = b.byte(e), byte3 = 0
  const uint32_t sel = (uint32_t)e | 0x0c00u | ((uint32_t)(4 + e) << 16) | 0x0c000000u;
  uint32_t w = __builtin_amdgcn_perm(b, a, sel) ^ 0x64806480u;
  f16x2 h = __builtin_bit_cast(f16x2, w);
  const f16x2 bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  return __builtin_bit_cast(uint32_t, h + bias);
}
// Half `hsel` (0 = low, 1 = high) of words a and b as one packed pair.
__device__ __forceinline__ uint32_t gather16(uint32_t a, uint32_t b, int hsel) {
  return __builtin_amdgcn_perm(b, a, hsel ? 0x07060302u : 0x05040100u);
}

// ---------------------------------------------------------------------- MFMA

__device__ __forceinline__ f32x4 mfma16x16x32(F16, u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x32(BF16, u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// 16x16x64 int8 -> int32 (exact): A/B hold 16 bytes per lane.  Both
// operands use the same lane/byte -> k map, so any consistent placement of
// the contraction index in the two operands gives the same dot products.
__device__ __forceinline__ i32x4 mfma16x16x64_i8(u32x4 a, u32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                               0);
}

// 16x16x16: A/B hold 4 elements (2 words) per lane, k = 4*(lane/16) + i.
__device__ __forceinline__ f32x4 mfma16x16x16(F16, u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                               __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16x16x16(BF16, u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                   __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}

// ------------------------------------------------------------------ wave ops

__device__ __forceinline__ float wave_max_xor16_32(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float wave_sum_xor16_32(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
// A 64-bit value the compiler must keep in scalar registers (computed by
// the scalar unit, then added to per-lane addresses with one vector op).
__device__ __forceinline__ uint64_t uniform64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Division by a divisor fixed for the whole launch, as a multiply-high and a
// shift (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, the round-up method with an N + 1-bit
// multiplier): with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
// x / d = (umulhi(x, m) + x) >> l for 0 <= x < 2^32; the sum fits 32 bits
// because callers keep x < 2^31.  The scalar unit does it in three
// instructions instead of the ~25 dependent ones of a runtime division.
struct FastDiv {
  uint32_t m;
  uint32_t l;
};
inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while (l < 32 && (1ull << l) < d) ++l;
  const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return FastDiv{(uint32_t)m, l};
}
__device__ __forceinline__ int fdiv(int x, FastDiv f) {
  return (int)((__umulhi((uint32_t)x, f.m) + (uint32_t)x) >> f.l);
}

// One rotary-embedding pair: oa = xa c - xb s, ob = xb c + xa s in fp32 with
// every product and sum rounded on its own.  hipcc contracts a*b - c*d into
// an FMA by default (and __fmul_rn is a plain multiply in this toolchain), so
// the contraction is switched off here: the result is a fixed function of
// the inputs, shared by every kernel that rotates q or k.
__device__ __forceinline__ void rope_rotate(float xa, float xb, float c, float s, float& oa, float& ob) {
#pragma clang fp contract(off)
  oa = xa * c - xb * s;
  ob = xb * c + xa * s;
}

// ------------------------------------------------------------------- loads

template <int BYTES>
struct Raw {
  static_assert(BYTES % 4 == 0 || BYTES == 2 || BYTES == 1, "raw size");
  static constexpr int W = BYTES >= 4 ? BYTES / 4 : 1;
  uint32_t w[W];
};

// Streaming (non-temporal) loads: K/V bytes are read exactly once per call, so
// they should not displace anything in L2 / MALL (measured on MI355X: a plain
// streaming read reaches ~6.3 TB/s, the non-temporal one ~7.1 TB/s).
template <int BYTES>
__device__ __forceinline__ void load_raw(Raw<BYTES>& r, const char* p) {
  if constexpr (BYTES % 16 == 0) {
#pragma unroll
    for (int i = 0; i < BYTES / 16; ++i) {
      const u32x4 x = __builtin_nontemporal_load((const u32x4*)(p + 16 * i));
      r.w[4 * i + 0] = x[0];
      r.w[4 * i + 1] = x[1];
      r.w[4 * i + 2] = x[2];
      r.w[4 * i + 3] = x[3];
    }
  } else if constexpr (BYTES == 8) {
    const u32x2 x = __builtin_nontemporal_load((const u32x2*)p);
    r.w[0] = x[0];
    r.w[1] = x[1];
  } else if constexpr (BYTES == 4) {
    r.w[0] = __builtin_nontemporal_load((const uint32_t*)p);
  } else {
    static_assert(BYTES % 16 == 0 || BYTES == 8 || BYTES == 4, "unsupported load width");
  }
}

template <int BYTES>
__device__ __forceinline__ void zero_raw(Raw<BYTES>& r) {
#pragma unroll
  for (int i = 0; i < Raw<BYTES>::W; ++i) r.w[i] = 0u;
}

}  // namespace sia
