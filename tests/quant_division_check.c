/* CPU check of the int8 KV quantisation arithmetic used by the gfx950 kernel
 * (csrc/kv_write.hip, div_by_scale): x / scale evaluated as q0 = RN(x * inv),
 * r = fma(-q0, scale, x), q = fma(r, inv, q0) with inv = RN(1 / scale) must
 * give the same int8 code, rint(x / scale) clamped to [-127, 127] with NaN -> 0,
 * as the correctly rounded division of model/kv_cache.py:58-67.  scale =
 * RN(amax / 127) with amax floored at 1e-8 rounded to the source dtype.
 *
 * Usage: quant_division_check STRIDE SAMPLES
 *   bf16 and fp16: every |x| <= amax (both signs) for every STRIDE-th amax
 *   pattern; fp32: SAMPLES random pairs plus SAMPLES/10 pairs within 3 ulps of
 *   a .5 tie.  Prints the counts and exits 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bf16(uint32_t h) { return from_bits(h << 16); }
static float f16(uint32_t h) {
  const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
  const float v = e == 0 ? ldexpf((float)m, -24) : ldexpf((float)(m | 0x400), e - 25);
  return (h & 0x8000) ? -v : v;
}
static int clamp_code(float q) {
  if (q != q) return 0;
  q = fminf(fmaxf(q, -127.f), 127.f);
  return (int)q;
}
static int code_div(float x, float s) { return clamp_code(rintf(x / s)); }
static int code_fma(float x, float s, float inv) {
  const float q0 = x * inv;
  const float r = fmaf(-q0, s, x);
  return clamp_code(rintf(fmaf(r, inv, q0)));
}

static long bad = 0, pairs = 0;
static void check(float x, float s, float inv) {
  ++pairs;
  if (code_div(x, s) != code_fma(x, s, inv)) {
    if (bad < 5) printf("mismatch x=%a scale=%a\n", x, s);
    ++bad;
  }
}

static void sweep16(float (*cv)(uint32_t), uint32_t lim, float floor_v, int stride, const char* name) {
  const long b0 = bad, p0 = pairs;
  for (uint32_t a = 0; a < lim; a += stride) {
    float amax = cv(a);
    if (!(amax > 0)) continue;
    if (amax < floor_v) amax = floor_v;
    const float s = amax / 127.0f, inv = 1.0f / s;
    for (uint32_t b = 0; b < lim; ++b) {
      const float x = cv(b);
      if (x > amax) break;
      check(x, s, inv);
      check(-x, s, inv);
    }
  }
  printf("%s: %ld pairs, %ld mismatches\n", name, pairs - p0, bad - b0);
}

int main(int argc, char** argv) {
  const int stride = argc > 1 ? atoi(argv[1]) : 1;
  const long samples = argc > 2 ? atol(argv[2]) : 1000000;
  /* 1e-8 rounded to bf16 (nearest even); fp16 rounds it to 0 */
  uint32_t u = to_bits(1e-8f);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  sweep16(bf16, 0x7f80, from_bits(u), stride, "bf16");
  sweep16(f16, 0x7c00, 0.0f, stride, "fp16");

  uint64_t st = 88172645463325252ull;
  const long b0 = bad, p0 = pairs;
  for (long i = 0; i < samples; ++i) {
    st ^= st << 13; st ^= st >> 7; st ^= st << 17;
    float amax = from_bits((uint32_t)(st >> 32) & 0x7fffffffu), x = from_bits((uint32_t)st & 0x7fffffffu);
    if (!(amax > 0) || isinf(amax) || isnan(amax) || isnan(x) || isinf(x)) continue;
    if (amax < 1e-8f) amax = 1e-8f;
    if (x > amax) x = fmodf(x, amax);
    const float s = amax / 127.0f, inv = 1.0f / s;
    check(x, s, inv);
    check(-x, s, inv);
  }
  for (long i = 0; i < samples / 10; ++i) {
    st ^= st << 13; st ^= st >> 7; st ^= st << 17;
    const float amax = from_bits(0x32000000u + (uint32_t)(st % 0x1d000000u));   /* ~7e-9 .. 3e8 */
    const float s = amax / 127.0f, inv = 1.0f / s;
    const int k = (int)((st >> 40) % 127);
    const uint32_t ux = to_bits(((float)k + 0.5f) * s);
    for (int d = -3; d <= 3; ++d) {
      const float x = from_bits(ux + d);
      if (x <= amax) { check(x, s, inv); check(-x, s, inv); }
    }
  }
  printf("fp32: %ld pairs, %ld mismatches\n", pairs - p0, bad - b0);
  return bad != 0;
}
