/*
 * CPU oracle for mtorch's SD-UNet hot path -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates the reference's x86-64 Linux scalar code path, operation by operation, in the
 * same accumulation order and precision.  Every function names the reference lines it
 * follows.  Build with -ffp-contract=off so that no multiply-add is fused: the reference's
 * Linux build (g++ -O3, default x86-64 ISA) has no FMA instructions either.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 conversion */

/* tensor.cpp:276-315.  Round-half-away-from-zero on the magnitude (add 0x1000, shift 13);
 * subnormals are shifted first (truncating) and then rounded the same way; values whose
 * half exponent is below -10 flush to a signed zero; NaN keeps its payload or becomes 0x200. */
uint16_t orc_f2h(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof(bits));
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t raw_exponent = (bits >> 23) & 0xffu;
  uint32_t mantissa = bits & 0x7fffffu;
  if (raw_exponent == 0xffu) {
    if (mantissa == 0) return (uint16_t)(sign | 0x7c00u);
    const uint32_t payload = mantissa >> 13;
    return (uint16_t)(sign | 0x7c00u | (payload == 0 ? 0x0200u : payload));
  }
  int32_t exponent = (int32_t)raw_exponent - 127 + 15;
  if (exponent <= 0) {
    if (exponent < -10) return (uint16_t)sign;
    mantissa = (mantissa | 0x800000u) >> (1 - exponent);
    return (uint16_t)(sign | ((mantissa + 0x1000u) >> 13));
  }
  if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  mantissa += 0x1000u;
  if (mantissa & 0x800000u) {
    mantissa = 0;
    ++exponent;
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  }
  return (uint16_t)(sign | ((uint32_t)exponent << 10) | (mantissa >> 13));
}

/* tensor.cpp:317-344: exact widening (subnormals normalised). */
float orc_h2f(uint16_t value) {
  const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
  uint32_t exponent = (value >> 10) & 0x1fu;
  uint32_t mantissa = value & 0x03ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      exponent = 1;
      while ((mantissa & 0x0400u) == 0) {
        mantissa <<= 1;
        --exponent;
      }
      mantissa &= 0x03ffu;
      bits = sign | ((exponent + 127 - 15) << 23) | (mantissa << 13);
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 127 - 15) << 23) | (mantissa << 13);
  }
  float result;
  memcpy(&result, &bits, sizeof(result));
  return result;
}

void orc_f2h_array(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_f2h(src[i]);
}

void orc_h2f_array(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_h2f(src[i]);
}

/* storage_set_unchecked, Float16 case (tensor.cpp:593-597). */
uint16_t orc_d2h(double value) { return orc_f2h((float)value); }

/* storage_get_unchecked widening (tensor.cpp:559-575). */
static double load_d(int dtype, const void* p, int64_t i) {
  if (dtype == ORC_F16) return (double)orc_h2f(((const uint16_t*)p)[i]);
  return (double)((const float*)p)[i];
}

/* storage_set_unchecked narrowing (tensor.cpp:593-600). */
static void store_d(int dtype, void* p, int64_t i, double value) {
  if (dtype == ORC_F16)
    ((uint16_t*)p)[i] = orc_d2h(value);
  else
    ((float*)p)[i] = (float)value;
}

/* ------------------------------------------------------------------ RNG */

void orc_rng_seed(orc_rng* rng, uint64_t seed) {
  rng->state = seed;
  rng->has_spare_normal = 0;
  rng->spare_normal = 0.0;
}

/* splitmix64 (module.cpp:76-82). */
uint64_t orc_rng_next_u64(orc_rng* rng) {
  rng->state += 0x9E3779B97F4A7C15ULL;
  uint64_t z = rng->state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/* 53-bit uniform, zero mapped to 2^-53 (module.cpp:84-88). */
double orc_rng_uniform_open(orc_rng* rng) {
  const double k = 1.0 / 9007199254740992.0;
  const double v = (double)(orc_rng_next_u64(rng) >> 11) * k;
  return v <= 0.0 ? k : v;
}

/* Marsaglia polar method (module.cpp:90-102). */
void orc_rng_normal_pair(orc_rng* rng, double* first, double* second) {
  double u, v, r2;
  do {
    u = 2.0 * orc_rng_uniform_open(rng) - 1.0;
    v = 2.0 * orc_rng_uniform_open(rng) - 1.0;
    r2 = u * u + v * v;
  } while (r2 >= 1.0 || r2 <= 0.0);
  const double s = sqrt(-2.0 * log(r2) / r2);
  *first = u * s;
  *second = v * s;
}

/* Spare-normal cache (module.cpp:104-115). */
double orc_rng_next_normal(orc_rng* rng) {
  if (rng->has_spare_normal) {
    rng->has_spare_normal = 0;
    return rng->spare_normal;
  }
  double a, b;
  orc_rng_normal_pair(rng, &a, &b);
  rng->spare_normal = b;
  rng->has_spare_normal = 1;
  return a;
}

/* fill_random_normal_contiguous<float> (module.cpp:117-144). */
void orc_fill_normal_f32(orc_rng* rng, float* dst, int64_t n, double mean, double std) {
  int64_t i = 0;
  if (rng->has_spare_normal && n > 0) {
    dst[i++] = (float)(mean + std * rng->spare_normal);
    rng->has_spare_normal = 0;
  }
  while (i + 1 < n) {
    double a, b;
    orc_rng_normal_pair(rng, &a, &b);
    dst[i++] = (float)(mean + std * a);
    dst[i++] = (float)(mean + std * b);
  }
  if (i < n) {
    double a, b;
    orc_rng_normal_pair(rng, &a, &b);
    dst[i++] = (float)(mean + std * a);
    rng->spare_normal = b;
    rng->has_spare_normal = 1;
  }
}

/* fp16 randn / normal_: set_at_linear(i, mean + std * next_standard_normal) (module.cpp:173-177,
 * 270-272).  For randn mean=0, std=1 so the value is the normal itself. */
void orc_fill_normal_f16(orc_rng* rng, uint16_t* dst, int64_t n, double mean, double std) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_d2h(mean + std * orc_rng_next_normal(rng));
}

/* fill_random_uniform_contiguous<float> (module.cpp:146-157). */
void orc_fill_uniform_f32(orc_rng* rng, float* dst, int64_t n, double from, double to) {
  const double scale = to - from;
  for (int64_t i = 0; i < n; ++i) dst[i] = (float)(from + scale * orc_rng_uniform_open(rng));
}

/* uniform_ fallback through set_at_linear (module.cpp:361-364). */
void orc_fill_uniform_f16(orc_rng* rng, uint16_t* dst, int64_t n, double from, double to) {
  const double scale = to - from;
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_d2h(from + scale * orc_rng_uniform_open(rng));
}

/* ------------------------------------------------------------------ GEMM family */

/* linear, Linux path (tensor.cpp:31653-31672): per output a double dot product in
 * in-feature order, then the bias added in double (value_for_broadcast), then narrowed. */
int orc_linear(int dtype, const void* x, const void* w, const void* b, void* y,
               int64_t M, int64_t N, int64_t K) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double total = 0.0;
      for (int64_t k = 0; k < K; ++k) total += load_d(dtype, x, m * K + k) * load_d(dtype, w, n * K + k);
      if (b) total += load_d(dtype, b, n);
      store_d(dtype, y, m * N + n, total);
    }
  }
  return 0;
}

/* matmul: fp32 2-D per-output double sum (tensor.cpp:24983-24996); fp16 2-D accumulates a
 * double array k-outer (:25049-25063), which adds the same terms to each output in the same
 * k order; batched_matmul per-output double sum (:24830-24845).  All three therefore reduce
 * to: double sum over k ascending, narrowed once. */
int orc_matmul(int dtype, const void* a, const void* b, void* c, int64_t batch,
               int64_t M, int64_t N, int64_t K, int64_t a_bstride, int64_t b_bstride) {
  for (int64_t bi = 0; bi < batch; ++bi) {
    for (int64_t m = 0; m < M; ++m) {
      for (int64_t n = 0; n < N; ++n) {
        double total = 0.0;
        for (int64_t k = 0; k < K; ++k)
          total += load_d(dtype, a, bi * a_bstride + m * K + k) * load_d(dtype, b, bi * b_bstride + k * N + n);
        store_d(dtype, c, (bi * M + m) * N + n, total);
      }
    }
  }
  return 0;
}

/* addmm (tensor.cpp:25253-25258, 25320-25334): the result is first filled with
 * narrow(beta * in) and then each element becomes narrow(stored + alpha * dot). */
int orc_addmm(int dtype, const void* in_mn, const void* a, const void* b, void* out,
              int64_t M, int64_t N, int64_t K, double beta, double alpha) {
  for (int64_t i = 0; i < M * N; ++i) store_d(dtype, out, i, beta * load_d(dtype, in_mn, i));
  if (alpha == 0.0) return 0;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double total = 0.0;
      for (int64_t k = 0; k < K; ++k) total += load_d(dtype, a, m * K + k) * load_d(dtype, b, k * N + n);
      store_d(dtype, out, m * N + n, load_d(dtype, out, m * N + n) + alpha * total);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ conv2d */

/* conv2d_output_size (tensor.cpp:25941). */
int64_t orc_conv2d_out_size(int64_t in, int64_t k, int64_t stride, int64_t pad, int64_t dil) {
  return (in + 2 * pad - dil * (k - 1) - 1) / stride + 1;
}

int orc_conv2d(int dtype, const void* x, const void* w, const void* b, void* y,
               int64_t B, int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW,
               int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, int64_t groups) {
  if (groups <= 0 || C % groups != 0 || O % groups != 0) return -1;
  const int64_t OH = orc_conv2d_out_size(H, KH, sh, ph, dh);
  const int64_t OW = orc_conv2d_out_size(W, KW, sw, pw, dw);
  const int64_t Cg = C / groups;
  const int64_t Og = O / groups;
  const int direct_1x1 = KH == 1 && KW == 1 && ph == 0 && pw == 0 && sh == 1 && sw == 1 && dh == 1 && dw == 1;

  if (dtype == ORC_F16 && groups == 1 && (O <= 4 || direct_1x1) && B > 0 && OH * OW > 0) {
    /* fp16 direct float-accumulate loop (tensor.cpp:27147-27180; the 3x3-same <=1024-pixel
     * scatter variant :27036-27071 adds the same terms per output in the same (c,ky,kx)
     * order).  total starts at the fp16 bias, every product and sum is a float op. */
    const uint16_t* xh = (const uint16_t*)x;
    const uint16_t* wh = (const uint16_t*)w;
    const uint16_t* bh = (const uint16_t*)b;
    uint16_t* yh = (uint16_t*)y;
    for (int64_t n = 0; n < B; ++n)
      for (int64_t o = 0; o < O; ++o) {
        const float bias_value = bh ? orc_h2f(bh[o]) : 0.0f;
        for (int64_t oy = 0; oy < OH; ++oy)
          for (int64_t ox = 0; ox < OW; ++ox) {
            float total = bias_value;
            for (int64_t c = 0; c < C; ++c)
              for (int64_t ky = 0; ky < KH; ++ky) {
                const int64_t iy = oy * sh - ph + ky * dh;
                if (iy < 0 || iy >= H) continue;
                for (int64_t kx = 0; kx < KW; ++kx) {
                  const int64_t ix = ox * sw - pw + kx * dw;
                  if (ix < 0 || ix >= W) continue;
                  const float xv = orc_h2f(xh[((n * C + c) * H + iy) * W + ix]);
                  const float wv = orc_h2f(wh[((o * C + c) * KH + ky) * KW + kx]);
                  const float prod = xv * wv;
                  total = total + prod;
                }
              }
            yh[((n * O + o) * OH + oy) * OW + ox] = orc_f2h(total);
          }
      }
    return 0;
  }

  /* fp32 generic loop (tensor.cpp:27359-27400): double total seeded by the bias, terms in
   * (c, ky, kx) order with out-of-bounds taps skipped, narrowed once.  fp16 inputs that miss
   * the direct loop are cast to fp32, run through this loop and cast back
   * (tensor.cpp:27182-27194), i.e. f2h((float)total). */
  for (int64_t n = 0; n < B; ++n)
    for (int64_t o = 0; o < O; ++o) {
      const int64_t g = o / Og;
      const int64_t c0 = g * Cg;
      for (int64_t oy = 0; oy < OH; ++oy)
        for (int64_t ox = 0; ox < OW; ++ox) {
          double total = b ? load_d(dtype, b, o) : 0.0;
          for (int64_t c = 0; c < Cg; ++c)
            for (int64_t ky = 0; ky < KH; ++ky) {
              const int64_t iy = oy * sh - ph + ky * dh;
              if (iy < 0 || iy >= H) continue;
              for (int64_t kx = 0; kx < KW; ++kx) {
                const int64_t ix = ox * sw - pw + kx * dw;
                if (ix < 0 || ix >= W) continue;
                total += load_d(dtype, x, ((n * C + c0 + c) * H + iy) * W + ix) *
                         load_d(dtype, w, ((o * Cg + c) * KH + ky) * KW + kx);
              }
            }
          store_d(dtype, y, ((n * O + o) * OH + oy) * OW + ox, total);
        }
    }
  return 0;
}

/* ------------------------------------------------------------------ attention */

/* softmax_scores (tensor.cpp:30429-30442): double max, exp(x - max), sum, divide. */
static void softmax_scores(double* s, int64_t n) {
  double mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i) mx = s[i] > mx ? s[i] : mx;
  double total = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    s[i] = exp(s[i] - mx);
    total += s[i];
  }
  for (int64_t i = 0; i < n; ++i) s[i] /= total;
}

/* Generic SDPA loop (tensor.cpp:31158-31207).  fp16 q/k/v are widened to fp32 exactly, the
 * output is computed as fp32 and then narrowed with f2h (tensor.cpp:30969-30982), which equals
 * storing f2h((float)total).  std::max on doubles with -inf start keeps NaN-free rows exact.
 * has_scale = 0 is the reference's scale=None (1/sqrt(E)); any given scale, zero and negative
 * ones included, multiplies the score as given (tensor.cpp:31019, 31182). */
int orc_sdpa(int dtype, const void* q, const void* k, const void* v, void* o,
             int64_t P, int64_t Lq, int64_t Lk, int64_t E, int64_t Ev,
             int mask_kind, const void* mask, int is_causal, int has_scale, double scale) {
  const double s = has_scale ? scale : 1.0 / sqrt((double)E);
  double* scores = (double*)malloc(sizeof(double) * (size_t)(Lk > 0 ? Lk : 1));
  if (!scores) return -1;
  for (int64_t p = 0; p < P; ++p) {
    for (int64_t qi = 0; qi < Lq; ++qi) {
      const int64_t valid = (mask_kind == 0 && is_causal) ? (Lk < qi + 1 ? Lk : qi + 1) : Lk;
      for (int64_t kj = 0; kj < valid; ++kj) {
        double score = 0.0;
        for (int64_t e = 0; e < E; ++e)
          score += load_d(dtype, q, (p * Lq + qi) * E + e) * load_d(dtype, k, (p * Lk + kj) * E + e);
        score *= s;
        if (mask_kind != 0) {
          if (is_causal && kj > qi) score = -INFINITY;
          const int64_t mi = (p * Lq + qi) * Lk + kj;
          if (mask_kind == 1) {
            if (((const uint8_t*)mask)[mi] == 0) score = -INFINITY;
          } else {
            score = score + (double)((const float*)mask)[mi];
          }
        }
        scores[kj] = score;
      }
      for (int64_t kj = valid; kj < Lk; ++kj) scores[kj] = -INFINITY;
      softmax_scores(scores, Lk);
      for (int64_t ev = 0; ev < Ev; ++ev) {
        double total = 0.0;
        for (int64_t kj = 0; kj < Lk; ++kj) total += scores[kj] * load_d(dtype, v, (p * Lk + kj) * Ev + ev);
        const int64_t oi = (p * Lq + qi) * Ev + ev;
        if (dtype == ORC_F16)
          ((uint16_t*)o)[oi] = orc_f2h((float)total);
        else
          ((float*)o)[oi] = (float)total;
      }
    }
  }
  free(scores);
  return 0;
}

/* ------------------------------------------------------------------ normalisation */

int orc_group_norm(int dtype, const void* x, const void* weight, const void* bias, void* y,
                   int64_t B, int64_t C, int64_t inner, int64_t groups, double eps) {
  if (groups <= 0 || C % groups != 0) return -1;
  const int64_t gc_count = C / groups;
  const int64_t group_size = gc_count * inner;
  float* vals = (float*)malloc(sizeof(float) * (size_t)(group_size > 0 ? group_size : 1));
  if (!vals) return -1;
  for (int64_t n = 0; n < B; ++n) {
    for (int64_t g = 0; g < groups; ++g) {
      const int64_t base = (n * C + g * gc_count) * inner;
      if (dtype == ORC_F16)
        orc_h2f_array((const uint16_t*)x + base, vals, group_size);
      else if (group_size > 0)
        memcpy(vals, (const float*)x + base, sizeof(float) * (size_t)group_size);
      /* Sequential fp32 sum and sum of squares, one-pass variance
       * (tensor.cpp:18752-18767 fp16, :18812-18824 fp32). */
      float sum = 0.0f, sumsq = 0.0f;
      for (int64_t i = 0; i < group_size; ++i) {
        const float v = vals[i];
        sum += v;
        const float sq = v * v;
        sumsq += sq;
      }
      const float mean = sum / (float)group_size;
      const float msq = sumsq / (float)group_size;
      float var = msq - mean * mean;
      if (var < 0.0f) var = 0.0f;
      const float inv = 1.0f / sqrtf(var + (float)eps);
      for (int64_t gc = 0; gc < gc_count; ++gc) {
        const int64_t c = g * gc_count + gc;
        const float* src = vals + gc * inner;
        if (dtype == ORC_F16) {
          /* affine_float32_to_half_bits(scale=gamma*inv, shift=beta-mean*gamma*inv)
           * (tensor.cpp:18768-18781, 18493-18518). */
          const float gamma = weight ? orc_h2f(((const uint16_t*)weight)[c]) : 1.0f;
          const float beta = bias ? orc_h2f(((const uint16_t*)bias)[c]) : 0.0f;
          const float scale = gamma * inv;
          const float shift = beta - mean * gamma * inv;
          uint16_t* dst = (uint16_t*)y + base + gc * inner;
          for (int64_t l = 0; l < inner; ++l) {
            const float t = src[l] * scale;
            dst[l] = orc_f2h(t + shift);
          }
        } else {
          /* (x - mean) * inv * gamma + beta (tensor.cpp:18834-18837). */
          const float gamma = weight ? ((const float*)weight)[c] : 1.0f;
          const float beta = bias ? ((const float*)bias)[c] : 0.0f;
          float* dst = (float*)y + base + gc * inner;
          for (int64_t l = 0; l < inner; ++l) {
            const float t = ((src[l] - mean) * inv) * gamma;
            dst[l] = t + beta;
          }
        }
      }
    }
  }
  free(vals);
  return 0;
}

int orc_layer_norm(int dtype, const void* x, const void* weight, const void* bias, void* y,
                   int64_t rows, int64_t N, double eps) {
  float* row = (float*)malloc(sizeof(float) * (size_t)(N > 0 ? N : 1));
  float* wv = (float*)malloc(sizeof(float) * (size_t)(N > 0 ? N : 1));
  float* bv = (float*)malloc(sizeof(float) * (size_t)(N > 0 ? N : 1));
  if (!row || !wv || !bv) {
    free(row);
    free(wv);
    free(bv);
    return -1;
  }
  if (weight) {
    for (int64_t i = 0; i < N; ++i) wv[i] = dtype == ORC_F16 ? orc_h2f(((const uint16_t*)weight)[i]) : ((const float*)weight)[i];
  }
  if (bias) {
    for (int64_t i = 0; i < N; ++i) bv[i] = dtype == ORC_F16 ? orc_h2f(((const uint16_t*)bias)[i]) : ((const float*)bias)[i];
  }
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t base = r * N;
    float mean, inv;
    if (dtype == ORC_F16) {
      /* Two-pass centred variance (tensor.cpp:17531-17545). */
      orc_h2f_array((const uint16_t*)x + base, row, N);
      float sum = 0.0f;
      for (int64_t i = 0; i < N; ++i) sum += row[i];
      mean = sum / (float)N;
      float css = 0.0f;
      for (int64_t i = 0; i < N; ++i) {
        const float c = row[i] - mean;
        const float sq = c * c;
        css += sq;
      }
      float var = css / (float)N;
      if (var < 0.0f) var = 0.0f;
      inv = 1.0f / sqrtf(var + (float)eps);
    } else {
      /* One-pass sum / sum of squares (tensor.cpp:17577-17587). */
      memcpy(row, (const float*)x + base, sizeof(float) * (size_t)N);
      float sum = 0.0f, sumsq = 0.0f;
      for (int64_t i = 0; i < N; ++i) {
        sum += row[i];
        const float sq = row[i] * row[i];
        sumsq += sq;
      }
      mean = sum / (float)N;
      const float msq = sumsq / (float)N;
      float var = msq - mean * mean;
      if (var < 0.0f) var = 0.0f;
      inv = 1.0f / sqrtf(var + (float)eps);
    }
    /* value = (x - mean) * inv; value *= w; value += b (tensor.cpp:17546-17560, 17588-17603). */
    for (int64_t i = 0; i < N; ++i) {
      float value = (row[i] - mean) * inv;
      if (weight) value = value * wv[i];
      if (bias) value = value + bv[i];
      if (dtype == ORC_F16)
        ((uint16_t*)y)[base + i] = orc_f2h(value);
      else
        ((float*)y)[base + i] = value;
    }
  }
  free(row);
  free(wv);
  free(bv);
  return 0;
}

/* ------------------------------------------------------------------ softmax */

int orc_softmax_lastdim(int dtype, const void* x, void* y, int64_t rows, int64_t cols, int rank) {
  float* row = (float*)malloc(sizeof(float) * (size_t)(cols > 0 ? cols : 1));
  if (!row) return -1;
  /* fp16 and fp32 rank>2 multiply by the reciprocal of the total (tensor.cpp:7581-7588,
   * 7789-7796); fp32 rank 1 and rank-2 dim 1 divide by it (tensor.cpp:7535-7537, 7708-7710). */
  const int divide = dtype == ORC_F32 && rank <= 2;
  for (int64_t r = 0; r < rows; ++r) {
    if (dtype == ORC_F16)
      orc_h2f_array((const uint16_t*)x + r * cols, row, cols);
    else
      memcpy(row, (const float*)x + r * cols, sizeof(float) * (size_t)cols);
    float mx = -INFINITY;
    for (int64_t i = 0; i < cols; ++i) mx = row[i] > mx ? row[i] : mx;
    float total = 0.0f;
    for (int64_t i = 0; i < cols; ++i) {
      row[i] = expf(row[i] - mx);
      total += row[i];
    }
    if (divide) {
      for (int64_t i = 0; i < cols; ++i) row[i] = row[i] / total;
    } else {
      const float inv = 1.0f / total;
      for (int64_t i = 0; i < cols; ++i) row[i] = row[i] * inv;
    }
    if (dtype == ORC_F16)
      orc_f2h_array(row, (uint16_t*)y + r * cols, cols);
    else
      memcpy((float*)y + r * cols, row, sizeof(float) * (size_t)cols);
  }
  free(row);
  return 0;
}

/* softmax_impl's generic path (tensor.cpp:15165-15207), taken when the output dtype differs
 * from the input's: the input read as double, e = exp(x - max) stored at the output dtype,
 * the double total of the unstored e, then each stored e read back and divided by the total. */
int orc_softmax_generic(int in_dtype, const void* x, int out_dtype, void* y, int64_t rows, int64_t cols) {
  double* row = (double*)malloc(sizeof(double) * (size_t)(cols > 0 ? cols : 1));
  if (!row) return -1;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < cols; ++i) {
      const int64_t k = r * cols + i;
      row[i] = in_dtype == ORC_F16 ? (double)orc_h2f(((const uint16_t*)x)[k]) : (double)((const float*)x)[k];
    }
    double mx = -INFINITY;
    for (int64_t i = 0; i < cols; ++i) mx = row[i] > mx ? row[i] : mx;
    double total = 0.0;
    for (int64_t i = 0; i < cols; ++i) {
      const double e = exp(row[i] - mx);
      /* set_at_linear narrows double -> float (-> half) (tensor.cpp:593-614) */
      row[i] = out_dtype == ORC_F16 ? (double)orc_h2f(orc_f2h((float)e)) : (double)(float)e;
      total += e;
    }
    for (int64_t i = 0; i < cols; ++i) {
      const float v = (float)(row[i] / total);
      const int64_t k = r * cols + i;
      if (out_dtype == ORC_F16)
        ((uint16_t*)y)[k] = orc_f2h(v);
      else
        ((float*)y)[k] = v;
    }
  }
  free(row);
  return 0;
}

/* ------------------------------------------------------------------ activations */

/* Abramowitz & Stegun 7.1.26 in float (tensor.cpp:17132-17144). */
float orc_fast_erf_float(float value) {
  const float sign = value < 0.0f ? -1.0f : 1.0f;
  const float x = fabsf(value);
  const float p = 0.3275911f;
  const float a1 = 0.254829592f;
  const float a2 = -0.284496736f;
  const float a3 = 1.421413741f;
  const float a4 = -1.453152027f;
  const float a5 = 1.061405429f;
  const float t = 1.0f / (1.0f + p * x);
  const float poly = (((((a5 * t + a4) * t + a3) * t + a2) * t + a1) * t);
  return sign * (1.0f - poly * expf(-x * x));
}

/* Truncated Taylor series of 0.5*x*erf(x/sqrt 2) for |x| <= 1 (tensor.cpp:17146-17154). */
float orc_gelu_unit_polynomial_float(float x) {
  const float inv_sqrt_two_pi = 0.39894228040143267794f;
  const float x2 = x * x;
  const float series =
      1.0f + x2 * (-1.0f / 6.0f + x2 * (1.0f / 40.0f + x2 * (-1.0f / 336.0f + x2 * (1.0f / 3456.0f + x2 * (-1.0f / 42240.0f)))));
  return 0.5f * x + inv_sqrt_two_pi * x2 * series;
}

int orc_gelu(int dtype, const void* x, void* y, int64_t n, int approximate) {
  if (dtype == ORC_F16) {
    /* f2h((float) gelu_value(double)) (tensor.cpp:17225-17235, gelu_value :17103-17113). */
    for (int64_t i = 0; i < n; ++i) {
      const double v = (double)orc_h2f(((const uint16_t*)x)[i]);
      double r;
      if (approximate == 0)
        r = 0.5 * v * (1.0 + erf(v * 0.70710678118654752440));
      else
        r = 0.5 * v * (1.0 + tanh(0.79788456080286535588 * (v + 0.044715 * v * v * v)));
      ((uint16_t*)y)[i] = orc_f2h((float)r);
    }
    return 0;
  }
  const float* src = (const float*)x;
  float* dst = (float*)y;
  if (approximate == 0) {
    /* tensor.cpp:17265-17273 */
    const float sqrt_half = 0.70710678118654752440f;
    for (int64_t i = 0; i < n; ++i) {
      const float v = src[i];
      if (fabsf(v) <= 1.0f)
        dst[i] = orc_gelu_unit_polynomial_float(v);
      else
        dst[i] = 0.5f * v * (1.0f + orc_fast_erf_float(v * sqrt_half));
    }
  } else {
    /* tensor.cpp:17275-17279 */
    const float k = 0.79788456080286535588f;
    for (int64_t i = 0; i < n; ++i) {
      const float v = src[i];
      dst[i] = 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * v * v * v)));
    }
  }
  return 0;
}

int orc_silu(int dtype, const void* x, void* y, int64_t n) {
  if (dtype == ORC_F16) {
    /* e = expf(-x); f2h(x / (1 + e)) (tensor.cpp:16500-16538). */
    for (int64_t i = 0; i < n; ++i) {
      const float v = orc_h2f(((const uint16_t*)x)[i]);
      const float e = expf(-v);
      ((uint16_t*)y)[i] = orc_f2h(v / (1.0f + e));
    }
    return 0;
  }
  /* x / (1 + expf(-x)) (tensor.cpp:16586-16590). */
  for (int64_t i = 0; i < n; ++i) {
    const float v = ((const float*)x)[i];
    ((float*)y)[i] = v / (1.0f + expf(-v));
  }
  return 0;
}

/* ------------------------------------------------------------------ binary / cast */

int orc_binary(int dtype, int op, const void* a, const void* b, void* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float av = dtype == ORC_F16 ? orc_h2f(((const uint16_t*)a)[i]) : ((const float*)a)[i];
    const float bv = dtype == ORC_F16 ? orc_h2f(((const uint16_t*)b)[i]) : ((const float*)b)[i];
    float r;
    if (op == 0)
      r = av + bv;
    else if (op == 1)
      r = av * bv;
    else
      r = av - bv;
    if (dtype == ORC_F16)
      ((uint16_t*)y)[i] = orc_f2h(r);
    else
      ((float*)y)[i] = r;
  }
  return 0;
}

void orc_cast_f32_to_f16(const float* x, uint16_t* y, int64_t n) { orc_f2h_array(x, y, n); }
void orc_cast_f16_to_f32(const uint16_t* x, float* y, int64_t n) { orc_h2f_array(x, y, n); }
