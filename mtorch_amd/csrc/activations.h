// Activation functions shared by the elementwise kernels and the GEMM/conv/norm epilogues,
// each evaluated the way mtorch's Linux CPU path evaluates it for the given storage dtype.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "common.h"

namespace mthip {
// These run inside kernels built with contraction on (the GEMM epilogues): every body turns
// it off so each multiply and add rounds separately, as the reference's x86-64 build (no FMA)
// evaluates them.

// fp32 GELU exactly as the reference's Linux fp32 path: truncated series for |x| <= 1,
// else Abramowitz-Stegun 7.1.26 erf (tensor.cpp:17132-17154, 17265-17273).
__device__ __forceinline__ float gelu_ref_f32(float x) {
#pragma clang fp contract(off)
  if (fabsf(x) <= 1.0f) {
    const float inv_sqrt_two_pi = 0.39894228040143267794f;
    const float x2 = x * x;
    const float series =
        1.0f + x2 * (-1.0f / 6.0f + x2 * (1.0f / 40.0f + x2 * (-1.0f / 336.0f + x2 * (1.0f / 3456.0f + x2 * (-1.0f / 42240.0f)))));
    return 0.5f * x + inv_sqrt_two_pi * x2 * series;
  }
  const float v = x * 0.70710678118654752440f;
  const float sign = v < 0.0f ? -1.0f : 1.0f;
  const float ax = fabsf(v);
  const float t = 1.0f / (1.0f + 0.3275911f * ax);
  const float poly = (((((1.061405429f * t + -1.453152027f) * t + 1.421413741f) * t + -0.284496736f) * t + 0.254829592f) * t);
  const float erfv = sign * (1.0f - poly * expf(-ax * ax));
  return 0.5f * x * (1.0f + erfv);
}

// fp16 GELU: the reference evaluates 0.5*x*(1+erf(x/sqrt 2)) in double (tensor.cpp:17103-17113,
// 17225-17235); doubles are cheap next to the HBM traffic of this op.
__device__ __forceinline__ float gelu_ref_f16(float xf) {
#pragma clang fp contract(off)
  const double x = (double)xf;
  return (float)(0.5 * x * (1.0 + erf(x * 0.70710678118654752440)));
}

__device__ __forceinline__ float gelu_tanh_f32(float x) {
#pragma clang fp contract(off)
  return 0.5f * x * (1.0f + tanhf(0.79788456080286535588f * (x + 0.044715f * x * x * x)));
}

__device__ __forceinline__ float gelu_tanh_f16(float xf) {
#pragma clang fp contract(off)
  const double x = (double)xf;
  return (float)(0.5 * x * (1.0 + tanh(0.79788456080286535588 * (x + 0.044715 * x * x * x))));
}

// fp16 SiLU of a half h: the reference's f2h(x / (1 + expf(-x))) (tensor.cpp:16500-16538) for
// all 65536 inputs (checked exhaustively against the oracle by a GPU test), from the native
// 2^x and reciprocal instead of expf and an IEEE divide.  The inputs where the native form's
// result differs are pinned: x <= -60 (finite), where x e^x underflows to -0; +-0; 0xc173,
// whose exact quotient lies within an fp32 ulp of an fp16 rounding tie; NaNs (the quieted
// input, as x86 propagates it).  All but 0xc173 have |h| = 0 or |x| > 60 (and x > 60 keeps the
// native result), so one unsigned compare finds them and a wave-uniform branch, taken only by
// waves holding such an input, applies the pins.
__device__ __forceinline__ uint16_t silu_half(uint16_t h) {
#pragma clang fp contract(off)
  const float x = h2f_bits(h);
  const float e = __builtin_amdgcn_exp2f(-x * 1.44269504088896341f);
  uint32_t r = f2h_fast(x * __builtin_amdgcn_rcpf(1.0f + e));
  r = h == 0xc173u ? 0xb15du : r;
  const uint32_t a = h & 0x7fffu;
  const bool rare = a - 1u >= 0x5380u;  // a == 0 (wraps) or a >= 0x5381 (|x| > 60, inf, NaN)
  if (__builtin_amdgcn_ballot_w64(rare)) {
    if (rare) {
      if (a == 0u)
        r = h;  // +-0
      else if (a > 0x7c00u)
        r = h | 0x200u;  // NaN: the quieted input
      else if ((h & 0x8000u) && h != 0xfc00u)
        r = 0x8000u;  // finite x < -60: x e^x underflows to -0
    }
  }
  return (uint16_t)r;
}

template <typename T>
__device__ __forceinline__ float apply_unary(int op, float x);

template <>
__device__ __forceinline__ float apply_unary<float>(int op, float x) {
#pragma clang fp contract(off)
  switch (op) {
    case MTHIP_UNARY_SILU: return x / (1.0f + expf(-x));
    case MTHIP_UNARY_GELU: return gelu_ref_f32(x);
    case MTHIP_UNARY_GELU_TANH: return gelu_tanh_f32(x);
    case MTHIP_UNARY_EXP: return (float)exp((double)x);
    case MTHIP_UNARY_SIN: return (float)sin((double)x);
    case MTHIP_UNARY_COS: return (float)cos((double)x);
    case MTHIP_UNARY_NEG: return -x;
    case MTHIP_UNARY_SIGMOID: return (float)(1.0 / (1.0 + exp(-(double)x)));
    default: return x > 0.0f ? x : 0.0f;
  }
}

// x is a half value (every caller narrows first), so the fp16 forms may key on its bits.
template <>
__device__ __forceinline__ float apply_unary<uint16_t>(int op, float x) {
#pragma clang fp contract(off)
  switch (op) {
    case MTHIP_UNARY_SILU: return h2f_bits(silu_half(f2h_fast(x)));
    case MTHIP_UNARY_GELU: return gelu_ref_f16(x);
    case MTHIP_UNARY_GELU_TANH: return gelu_tanh_f16(x);
    default: return apply_unary<float>(op, x);
  }
}


// Activation codes of the fused epilogues (MTHIP_ACT_*) mapped onto the unary ops.
template <typename T>
__device__ __forceinline__ float apply_act(int act, float x) {
  switch (act) {
    case MTHIP_ACT_GELU: return apply_unary<T>(MTHIP_UNARY_GELU, x);
    case MTHIP_ACT_GELU_TANH: return apply_unary<T>(MTHIP_UNARY_GELU_TANH, x);
    case MTHIP_ACT_SILU: return apply_unary<T>(MTHIP_UNARY_SILU, x);
    default: return x;
  }
}

}  // namespace mthip
