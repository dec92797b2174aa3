/* CPU model of the device fp16 narrowings in mtorch_amd/csrc/common.h, checked over all 2^32
 * float bit patterns: f2h_fast (short common path + generic fallback) must equal f2h_generic,
 * and f2h_generic must equal mtorch's rounding (round to nearest, ties away from zero, overflow
 * to inf, NaN keeping the top payload bits; tensor.cpp:276-315, restated in oracle/oracle.c).
 * f2h_nonnan (integer and fma steps, no hardware conversion) must equal f2h_generic on every
 * non-NaN pattern, with fp32 denormal inputs kept or flushed to zero; f2h_rtz_prep followed by
 * the round-toward-zero conversion on every finite pattern below 65520 in magnitude.
 * The hardware conversion v_cvt_f16_f32 rounds to nearest-even; F16C's _cvtss_sh with
 * round-to-nearest is the same IEEE operation.  fmaf is the correctly rounded fused multiply-add
 * that v_fma_f32 computes. */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static inline uint32_t rne(uint32_t bits) {
  float f;
  memcpy(&f, &bits, 4);
  return (uint32_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
}

static uint32_t f2h_generic(uint32_t bits) {
  const uint32_t raw = (bits >> 23) & 0xffu;
  uint32_t h = rne(bits);
  const int d = 126 - (int)raw;
  const uint32_t sh = (uint32_t)(d < 13 ? 13 : (d > 24 ? 24 : d));
  const uint32_t sig = (bits & 0x7fffffu) | 0x800000u;
  const int tie_even = (sig & ((2u << sh) - 1u)) == (1u << (sh - 1u));
  h += (raw - 102u <= 40u && tie_even) ? 1u : 0u;
  const uint32_t payload = (bits & 0x7fffffu) >> 13;
  const uint32_t nan_bits = ((bits >> 16) & 0x8000u) | 0x7c00u | (payload != 0u ? payload : 0x200u);
  return (bits & 0x7fffffffu) > 0x7f800000u ? nan_bits : (h & 0xffffu);
}

static uint32_t f2h_fast(uint32_t bits) {
  const uint32_t a = bits & 0x7fffffffu;
  const int common = a == 0u || a - 0x38800000u < 0x0f000000u;
  if (!common) return f2h_generic(bits);
  return (rne(bits) + ((bits & 0x3fffu) == 0x1000u ? 1u : 0u)) & 0xffffu;
}

static uint32_t f2h_nonnan(uint32_t bits, int flush) {
  float v;
  memcpy(&v, &bits, 4);
  const uint32_t t = ((bits - 0x37fff000u) >> 13) & 0x3ffffu;
  const uint32_t hn = t < 0x7c00u ? t : 0x7c00u;
  float av = fabsf(v);
  if (flush && (bits & 0x7f800000u) == 0u) av = 0.0f;
  const uint32_t hs = (uint32_t)fmaf(av, 16777216.0f, 0x1.fffffep-2f);
  return (av < 0x1p-14f ? hs : hn) | ((bits >> 16) & 0x8000u);
}

/* f2h_rtz_prep + v_cvt_pkrtz_f16_f32: value + copysign(offset, value) in fp32 (round to nearest
 * even), then the conversion rounding toward zero (F16C's _cvtss_sh with _MM_FROUND_TO_ZERO is
 * the same IEEE operation).  Claimed equal to f2h_generic for every finite |value| < 65520, with
 * fp32 denormals kept or flushed (inputs and results) to zero. */
static uint32_t f2h_rtz(uint32_t bits, int flush) {
  float v;
  memcpy(&v, &bits, 4);
  if (flush && (bits & 0x7f800000u) == 0u) v = (bits & 0x80000000u) ? -0.0f : 0.0f;
  int off = (int)(bits & 0x7f800000u) - (11 << 23);
  off = off > 0x32ffffff ? off : 0x32ffffff; /* 2^-25 - 2^-49 */
  const uint32_t ob = (bits & 0x80000000u) | (uint32_t)off;
  float o;
  memcpy(&o, &ob, 4);
  float t = v + o;
  uint32_t tb;
  memcpy(&tb, &t, 4);
  if (flush && (tb & 0x7f800000u) == 0u) t = (tb & 0x80000000u) ? -0.0f : 0.0f;
  return (uint32_t)_cvtss_sh(t, _MM_FROUND_TO_ZERO) & 0xffffu;
}

/* mtorch's scalar rule, written independently of the hardware conversion */
static uint32_t f2h_reference(uint32_t bits) {
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t a = bits & 0x7fffffffu;
  if (a > 0x7f800000u) {
    const uint32_t payload = (bits & 0x7fffffu) >> 13;
    return sign | 0x7c00u | (payload != 0u ? payload : 0x200u);
  }
  if (a == 0x7f800000u) return sign | 0x7c00u;
  const int exponent = (int)(a >> 23) - 127 + 15;
  uint32_t mantissa = a & 0x7fffffu;
  if (exponent <= 0) {
    if (exponent < -10) return sign;
    mantissa |= 0x800000u;
    const int shift = 14 - exponent;
    uint32_t h = mantissa >> shift;
    const uint32_t rem = mantissa & ((1u << shift) - 1u);
    if (rem >= (1u << (shift - 1))) h += 1u; /* half or more: away from zero */
    return sign | h;
  }
  uint32_t r = ((uint32_t)exponent << 10) + ((mantissa + 0x1000u) >> 13);
  return sign | (r >= 0x7c00u ? 0x7c00u : r);
}

int main(void) {
  uint64_t bad_fast = 0, bad_ref = 0, bad_nonnan = 0, bad_rtz = 0;
  for (uint64_t i = 0; i <= 0xffffffffull; ++i) {
    const uint32_t b = (uint32_t)i;
    const uint32_t g = f2h_generic(b);
    if (f2h_fast(b) != g && bad_fast++ < 5) printf("fast %08x: %04x vs %04x\n", b, f2h_fast(b), g);
    if (f2h_reference(b) != g && bad_ref++ < 5) printf("ref %08x: %04x vs %04x\n", b, f2h_reference(b), g);
    if ((b & 0x7fffffffu) <= 0x7f800000u && (f2h_nonnan(b, 0) != g || f2h_nonnan(b, 1) != g) && bad_nonnan++ < 5)
      printf("nonnan %08x: %04x / %04x vs %04x\n", b, f2h_nonnan(b, 0), f2h_nonnan(b, 1), g);
    if ((b & 0x7fffffffu) < 0x477ff000u && (f2h_rtz(b, 0) != g || f2h_rtz(b, 1) != g) && bad_rtz++ < 5)
      printf("rtz %08x: %04x / %04x vs %04x\n", b, f2h_rtz(b, 0), f2h_rtz(b, 1), g);
  }
  printf("fast!=generic %llu, reference!=generic %llu, nonnan!=generic %llu, rtz!=generic %llu\n",
         (unsigned long long)bad_fast, (unsigned long long)bad_ref, (unsigned long long)bad_nonnan,
         (unsigned long long)bad_rtz);
  return (bad_fast || bad_ref || bad_nonnan || bad_rtz) ? 1 : 0;
}
