// Shared definitions for libmthip: dtype codes, error plumbing, stream access and the
// device-side fp16 conversion that follows mtorch's rounding rule.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <string>

#include "../../include/mthip.h"

namespace mthip {

// ---- errors -----------------------------------------------------------------------------
// Every C entry point returns 0 on success; on failure it stores a message retrievable
// through mthip_last_error() (thread-local) and returns a non-zero status.
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define MTHIP_CHECK_HIP(expr)                                                                  \
  do {                                                                                         \
    hipError_t _e = (expr);                                                                    \
    if (_e != hipSuccess)                                                                      \
      return ::mthip::fail(MTHIP_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(_e)); \
  } while (0)

#define MTHIP_REQUIRE(cond, msg)                                        \
  do {                                                                  \
    if (!(cond)) return ::mthip::fail(MTHIP_ERR_INVALID, (msg));        \
  } while (0)

// Per-device in-order stream (created on first use, default priority, non-blocking with
// respect to the legacy null stream).  Returns nullptr and sets the error on failure.
hipStream_t stream_for(int device);
// Makes `device` current for the calling host thread; returns 0 or an error status.
int use_device(int device);
// After a kernel launch: turns a launch error into a status.
int check_launch(const char* what);
// 65536-entry fp16 table of erf-gelu indexed by the input's bits, bit-identical to evaluating
// it; filled on first use per device (nullptr if that failed).
const uint16_t* gelu_f16_lookup(int device, hipStream_t s);
// The fp16 SiLU of every half value (silu_half), filled once per device (norm.hip).
const uint16_t* silu_f16_lookup(int device, hipStream_t s);

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Division of a 32-bit unsigned value by a run-time invariant d >= 1 as a multiply-high, add
// and shift (Granlund & Montgomery, "Division by invariant integers using multiplication",
// PLDI 1994, round-up variant): with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1,
// n / d = (mulhi(n, m) + n) >> l for every n < 2^32.  Kernels divide tile and pixel indices
// this way instead of through the ~100-instruction generic division.
struct FastDiv {
  uint32_t d, m, l;
  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t divisor) : d(divisor), m(0), l(0) {
    while ((uint64_t(1) << l) < (uint64_t)d) ++l;
    m = (uint32_t)(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint64_t t = __umulhi(n, m);
    return (uint32_t)((t + n) >> l);
  }
  __device__ __forceinline__ uint32_t mod(uint32_t n) const { return n - div(n) * d; }
};

// ---- device fp16 conversion ------------------------------------------------------------
// mtorch's float_to_half_bits (tensor.cpp:276-315) rounds the magnitude half-away-from-zero
// (add 0x1000 then drop 13 bits), shifts subnormals before rounding and flushes anything
// below 2^-25 to a signed zero.  The hardware v_cvt_f16_f32 rounds to nearest-even, so every
// kernel that narrows to fp16 uses this integer restatement instead.
__device__ __forceinline__ uint16_t f2h_bits(float value) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t raw_exponent = (bits >> 23) & 0xffu;
  uint32_t mantissa = bits & 0x7fffffu;
  if (raw_exponent == 0xffu) {
    if (mantissa == 0) return (uint16_t)(sign | 0x7c00u);
    const uint32_t payload = mantissa >> 13;
    return (uint16_t)(sign | 0x7c00u | (payload == 0 ? 0x0200u : payload));
  }
  int32_t exponent = (int32_t)raw_exponent - 112;  // -127 + 15
  if (exponent <= 0) {
    if (exponent < -10) return (uint16_t)sign;
    mantissa = (mantissa | 0x800000u) >> (1 - exponent);
    return (uint16_t)(sign | ((mantissa + 0x1000u) >> 13));
  }
  // Normal range: rounding may carry into the exponent; a carry out of exponent 30 gives
  // 0x7c00 (inf), which is exactly what adding the rounded mantissa bits produces.
  const uint32_t rounded = ((uint32_t)exponent << 10) + ((mantissa + 0x1000u) >> 13);
  return (uint16_t)(sign | (rounded >= 0x7c00u ? 0x7c00u : rounded));
}

// The hardware conversion (v_cvt_f16_f32, round to nearest-even) of exactly `value`.  The empty
// asm hides where the value came from: given a product of two widened halves, the compiler
// otherwise folds the multiply and this conversion into v_fma_mix(a, b, +0), whose +0 addend
// turns a -0 product into +0.
__device__ __forceinline__ uint32_t cvt_f16_rne(float value) {
  asm("" : "+v"(value));
  return __builtin_bit_cast(uint16_t, (_Float16)value);
}

// Bit-identical to f2h_bits for every input, and branch-free.  mtorch's rule is round-to-nearest
// with ties away from zero, overflowing to inf; the hardware conversion (v_cvt_f16_f32, with
// fp16 subnormals) rounds to nearest-even and overflows the same way.  The two differ only on exact ties whose kept LSB is 0, where
// RNE keeps the smaller magnitude: with sh discarded significand bits (13 for normal halves,
// up to 24 for the smallest subnormal, biased float exponent 102..142), such a tie has
// significand & (2^(sh+1) - 1) == 2^(sh-1), and one ulp is added to the magnitude.  NaNs keep
// the top payload bits as mtorch does (the hardware would set the quiet bit).
__device__ __forceinline__ uint16_t f2h_generic(float value) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t raw = (bits >> 23) & 0xffu;
  uint32_t h = cvt_f16_rne(value);
  const int d = 126 - (int)raw;
  const uint32_t sh = (uint32_t)(d < 13 ? 13 : (d > 24 ? 24 : d));
  const uint32_t sig = (bits & 0x7fffffu) | 0x800000u;
  const bool tie_even = (sig & ((2u << sh) - 1u)) == (1u << (sh - 1u));
  h += (raw - 102u <= 40u && tie_even) ? 1u : 0u;
  const uint32_t payload = (bits & 0x7fffffu) >> 13;
  const uint32_t nan_bits = ((bits >> 16) & 0x8000u) | 0x7c00u | (payload != 0u ? payload : 0x200u);
  return (uint16_t)((bits & 0x7fffffffu) > 0x7f800000u ? nan_bits : h);
}

// f2h_generic with a short common path, for streaming kernels (one or a few values per lane
// between loads, many waves per SIMD): for zero and |value| in [2^-14, 2^16) the result is a
// normal half (or the overflow to inf), 13 significand bits are discarded, and the RNE result
// needs the extra ulp exactly when those bits are 0x1000 with the kept LSB 0, i.e.
// (bits & 0x3fff) == 0x1000 (inside [65520, 65536) the discarded bits are >= 0x3000, so inf is
// never bumped).  Subnormal results, |value| >= 2^16, infinities and NaNs take f2h_generic, on a
// branch the whole wave skips unless one of its lanes needs it.  Equal to f2h_generic for all
// 2^32 inputs (tests/f2h_fast_model.c checks both exhaustively with a CPU model of the hardware
// conversion).
//
// Epilogues that narrow dozens of values per lane at one or two waves per SIMD (GEMM, conv,
// attention) use f2h_nonnan below instead: no branch per value, so the conversions interleave,
// where one scalar branch per value would serialise them.
__device__ __forceinline__ uint16_t f2h_fast(float value) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t a = bits & 0x7fffffffu;
  const bool common = a == 0u || a - 0x38800000u < 0x0f000000u;
  uint32_t h = cvt_f16_rne(value);
  h += (bits & 0x3fffu) == 0x1000u ? 1u : 0u;
  if (__builtin_amdgcn_ballot_w64(!common)) {
    const uint32_t g = f2h_generic(value);
    h = common ? h : g;
  }
  return (uint16_t)h;
}

// mtorch's fp16 narrowing for every value except NaN (which gives an infinity), branch-free and
// without the hardware conversion: about 10 VALU operations against f2h_generic's ~20.
//  * |value| >= 2^-14 (normal halves, overflow): adding 0x1000 to the bit pattern rounds the 13
//    discarded significand bits half-up in magnitude (a carry moves into the exponent);
//    subtracting (127 - 15) << 23 at the same time rebiases the exponent, and results from
//    65520 up (and inf) clamp to 0x7c00.
//  * |value| < 2^-14 (subnormal halves): the result counts units of 2^-24, floor(|v| * 2^24 +
//    0.5).  fma(|v|, 2^24, 0.5 - 2^-25) produces that floor exactly under round-to-nearest-even
//    (the sum of 0.5 itself and the float just below 2^-25, scaled, would round up to 1).
// Epilogues narrow with it, record whether any lane met a NaN, and redo their values with
// f2h_generic in the rare wave that did.  Equal to f2h_generic for every non-NaN float, with or
// without fp32 denormal flushing (tests/f2h_fast_model.c checks all 2^32 patterns).
__device__ __forceinline__ uint32_t f2h_nonnan(float value) {
  const uint32_t bits = __float_as_uint(value);
  const uint32_t hn = min(((bits - 0x37fff000u) >> 13) & 0x3ffffu, 0x7c00u);
  const float av = __builtin_fabsf(value);
  const uint32_t hs = (uint32_t)__builtin_fmaf(av, 16777216.0f, 0x1.fffffep-2f);
  return (av < 0x1p-14f ? hs : hn) | ((bits >> 16) & 0x8000u);
}

// mtorch's fp16 narrowing for finite |value| < 65520 as one float add and the hardware's
// round-toward-zero conversion (v_cvt_pkrtz_f16_f32, two values per instruction): adding half
// the fp16 spacing at |value| with value's sign and truncating gives the half-away-from-zero
// result.  For a float exponent e >= -14 the offset is u/2 = 2^(e-11), a multiple of value's
// float ulp: the sum is exact unless it carries into the next binade, where its rounding cannot
// reach the next fp16 value.  Below, the spacing is 2^-24 and the offset 2^-25 - 2^-49: a sum
// that lands 2^-49 under a multiple of 2^-24 rounds up onto it (its ulp is >= 2^-47 there), so
// ties still truncate upward while every value under a tie stays under, and |value| < 2^-25
// stays below 2^-24 (a result of 0).  As bits: 2^(e-11) is the exponent field minus 11 << 23,
// which for e < -116 wraps negative; a signed integer max against the bits of 2^-25 - 2^-49
// orders these positive floats as floats (and needs no NaN canonicalisation, unlike a float
// max of bits).  About 5 VALU operations per value against f2h_nonnan's ~10.  NaN, infinities and |value| >= 65520 (where the
// conversion saturates at 65504) are not covered: callers keep a running maximum of |value|
// (maximum propagates NaN) and redo a wave that met one with f2h_nonnan / f2h_generic.
// tests/f2h_fast_model.c checks every covered pattern, with fp32 denormals kept or flushed.
__device__ __forceinline__ float f2h_rtz_prep(float value) {
  const uint32_t bits = __float_as_uint(value);
  const int off = max((int)(bits & 0x7f800000u) - (11 << 23), 0x32ffffff);  // 0x32ffffff: 2^-25 - 2^-49
  return value + __uint_as_float((bits & 0x80000000u) | (uint32_t)off);
}

// Two values narrowed by f2h_rtz_prep + the round-toward-zero conversion, packed low | high << 16.
__device__ __forceinline__ uint32_t f2h_rtz_pack(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(f2h_rtz_prep(lo), f2h_rtz_prep(hi)));
}

// The largest |value| seen so far, NaN once any value was NaN: the covering test for the
// f2h_rtz_* narrowings is !(running < 65520).
__device__ __forceinline__ float abs_max_nan(float running, float value) {
  return __builtin_elementwise_maximum(running, __builtin_fabsf(value));
}

// (float)a.half + (float)b.half for fp16 halves of two packed registers (AHI / BHI: the high
// half) as one v_fma_mix_f32, a * 1.0 + b with both operands widened exactly: the same single
// rounding as widening both and adding.  A sum of two halves is 0 or at least 2^-24 in magnitude,
// never an fp32 denormal, so the denormal mode does not enter.
template <bool AHI, bool BHI>
__device__ __forceinline__ float add_halves(uint32_t a, uint32_t b) {
  float d;
  if constexpr (AHI && BHI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  else if constexpr (AHI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  else if constexpr (BHI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(d) : "v"(a), "v"(b));
  return d;
}

// acc + (float)a.half and acc + (float)a.half * (float)a.half (HI: the high half), each with one
// rounding as one v_fma_mix_f32: a half times 1.0 or times itself is exact in fp32, so these
// equal widening, (squaring,) and adding.  For sums of halves and of squares of halves (every
// term 0 or at least 2^-48 in magnitude, partial sums multiples of 2^-48) no fp32 denormal
// arises, so the denormal mode does not enter.
template <bool HI>
__device__ __forceinline__ float acc_add_half(float acc, uint32_t a) {
  float d;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(a), "v"(acc));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(a), "v"(acc));
  return d;
}
template <bool HI>
__device__ __forceinline__ float acc_add_sq_half(float acc, uint32_t a) {
  float d;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(d) : "v"(a), "v"(acc));
  else
    asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel_hi:[1,1,0]" : "=v"(d) : "v"(a), "v"(acc));
  return d;
}

// (float)a.half * (float)b.half, exact (a product of two halves fits a float, normal or 0), as
// one v_fma_mix_f32 with a -0.0 addend, which leaves every product as it is (a +0 addend would
// turn a -0 product into +0).
template <bool AHI, bool BHI>
__device__ __forceinline__ float mul_halves(uint32_t a, uint32_t b) {
  float d;
  const float nz = -0.0f;
  if constexpr (AHI && BHI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(d) : "v"(a), "v"(b), "v"(nz));
  else if constexpr (AHI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,1,0]" : "=v"(d) : "v"(a), "v"(b), "v"(nz));
  else if constexpr (BHI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[1,1,0]" : "=v"(d) : "v"(a), "v"(b), "v"(nz));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,1,0]" : "=v"(d) : "v"(a), "v"(b), "v"(nz));
  return d;
}

// Exact widening; finite values and infinities match tensor.cpp:317-344 bit for bit.
__device__ __forceinline__ float h2f_bits(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Exact widening including NaN payloads (integer restatement of tensor.cpp:317-344),
// used by the dtype-cast kernel where bit-exactness covers every pattern.
__device__ __forceinline__ float h2f_exact(uint16_t value) {
  const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
  const uint32_t exponent = (value >> 10) & 0x1fu;
  const uint32_t mantissa = value & 0x03ffu;
  if (exponent == 31) return __uint_as_float(sign | 0x7f800000u | (mantissa << 13));
  return (float)__builtin_bit_cast(_Float16, value);
}

// Element load/store in the op's dtype, computing in fp32.
template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
  // Value as the reference would read it back after storing (identity for fp32).
  static __device__ __forceinline__ float round_trip(float v) { return v; }
};
template <>
struct Elem<uint16_t> {
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return h2f_bits(p[i]); }
  static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) { p[i] = f2h_fast(v); }
  static __device__ __forceinline__ float round_trip(float v) { return h2f_bits(f2h_fast(v)); }
};

}  // namespace mthip
