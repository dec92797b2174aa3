// Host-side random number generation with mtorch's generator, so that seeded inputs and
// parameters are bit-identical to what the reference creates before they move to the GPU.
//
//   splitmix64 stream              module.cpp:76-82
//   53-bit open uniform            module.cpp:84-88
//   Marsaglia polar normal pairs   module.cpp:90-102, spare cache :104-115
//   fp32 normal fill (pairs)       module.cpp:117-144
//   fp16 / per-element fills       module.cpp:173-177, 270-272, 361-364 (value -> float -> half)
//   fp32 uniform fill              module.cpp:146-157
#include <cmath>
#include <cstdint>
#include <cstring>
#include <new>

#include "../../include/mthip.h"

namespace {

struct Generator {
  uint64_t state = 0;
  bool has_spare = false;
  double spare = 0.0;

  uint64_t next_u64() {
    state += 0x9E3779B97F4A7C15ULL;
    uint64_t z = state;
    z = (z ^ (z >> 30U)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27U)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31U);
  }

  double uniform_open() {
    constexpr double kScale = 1.0 / 9007199254740992.0;
    const double v = static_cast<double>(next_u64() >> 11U) * kScale;
    return v <= 0.0 ? kScale : v;
  }

  void normal_pair(double& first, double& second) {
    double u, v, r2;
    do {
      u = 2.0 * uniform_open() - 1.0;
      v = 2.0 * uniform_open() - 1.0;
      r2 = u * u + v * v;
    } while (r2 >= 1.0 || r2 <= 0.0);
    const double scale = std::sqrt(-2.0 * std::log(r2) / r2);
    first = u * scale;
    second = v * scale;
  }

  double normal() {
    if (has_spare) {
      has_spare = false;
      return spare;
    }
    double a, b;
    normal_pair(a, b);
    spare = b;
    has_spare = true;
    return a;
  }
};

// float -> binary16 bit pattern with mtorch's rounding (tensor.cpp:276-315): round the
// magnitude half away from zero, shift subnormals first, flush below 2^-25 to signed zero.
uint16_t float_to_half(float value) {
  uint32_t bits;
  std::memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t raw = (bits >> 23) & 0xffu;
  uint32_t man = bits & 0x7fffffu;
  if (raw == 0xffu) {
    if (man == 0) return static_cast<uint16_t>(sign | 0x7c00u);
    const uint32_t payload = man >> 13;
    return static_cast<uint16_t>(sign | 0x7c00u | (payload == 0 ? 0x0200u : payload));
  }
  const int32_t e = static_cast<int32_t>(raw) - 112;
  if (e <= 0) {
    if (e < -10) return static_cast<uint16_t>(sign);
    man = (man | 0x800000u) >> (1 - e);
    return static_cast<uint16_t>(sign | ((man + 0x1000u) >> 13));
  }
  const uint32_t r = (static_cast<uint32_t>(e) << 10) + ((man + 0x1000u) >> 13);
  return static_cast<uint16_t>(sign | (r >= 0x7c00u ? 0x7c00u : r));
}

}  // namespace

extern "C" {

void* mthip_generator_create(uint64_t seed) {
  auto* g = new (std::nothrow) Generator();
  if (g) g->state = seed;
  return g;
}

void mthip_generator_destroy(void* gen) { delete static_cast<Generator*>(gen); }

int mthip_generator_seed(void* gen, uint64_t seed) {
  if (!gen) return MTHIP_ERR_INVALID;
  auto* g = static_cast<Generator*>(gen);
  g->state = seed;
  g->has_spare = false;
  g->spare = 0.0;
  return MTHIP_OK;
}

int mthip_generator_get_state(void* gen, uint64_t* state, int* has_spare, double* spare) {
  if (!gen) return MTHIP_ERR_INVALID;
  auto* g = static_cast<Generator*>(gen);
  if (state) *state = g->state;
  if (has_spare) *has_spare = g->has_spare ? 1 : 0;
  if (spare) *spare = g->spare;
  return MTHIP_OK;
}

int mthip_generator_set_state(void* gen, uint64_t state, int has_spare, double spare) {
  if (!gen) return MTHIP_ERR_INVALID;
  auto* g = static_cast<Generator*>(gen);
  g->state = state;
  g->has_spare = has_spare != 0;
  g->spare = spare;
  return MTHIP_OK;
}

int mthip_rng_normal(void* gen, int dtype, void* host_dst, int64_t n, double mean, double std) {
  if (!gen || (n > 0 && !host_dst) || n < 0) return MTHIP_ERR_INVALID;
  auto* g = static_cast<Generator*>(gen);
  if (dtype == MTHIP_F32) {
    float* dst = static_cast<float*>(host_dst);
    int64_t i = 0;
    if (g->has_spare && n > 0) {
      dst[i++] = static_cast<float>(mean + std * g->spare);
      g->has_spare = false;
    }
    while (i + 1 < n) {
      double a, b;
      g->normal_pair(a, b);
      dst[i++] = static_cast<float>(mean + std * a);
      dst[i++] = static_cast<float>(mean + std * b);
    }
    if (i < n) {
      double a, b;
      g->normal_pair(a, b);
      dst[i++] = static_cast<float>(mean + std * a);
      g->spare = b;
      g->has_spare = true;
    }
    return MTHIP_OK;
  }
  if (dtype == MTHIP_F64) {
    double* dst = static_cast<double*>(host_dst);
    int64_t i = 0;
    if (g->has_spare && n > 0) {
      dst[i++] = mean + std * g->spare;
      g->has_spare = false;
    }
    while (i + 1 < n) {
      double a, b;
      g->normal_pair(a, b);
      dst[i++] = mean + std * a;
      dst[i++] = mean + std * b;
    }
    if (i < n) {
      double a, b;
      g->normal_pair(a, b);
      dst[i++] = mean + std * a;
      g->spare = b;
      g->has_spare = true;
    }
    return MTHIP_OK;
  }
  if (dtype == MTHIP_F16) {
    uint16_t* dst = static_cast<uint16_t*>(host_dst);
    for (int64_t i = 0; i < n; ++i) dst[i] = float_to_half(static_cast<float>(mean + std * g->normal()));
    return MTHIP_OK;
  }
  return MTHIP_ERR_INVALID;
}

int mthip_rng_uniform(void* gen, int dtype, void* host_dst, int64_t n, double from, double to) {
  if (!gen || (n > 0 && !host_dst) || n < 0) return MTHIP_ERR_INVALID;
  auto* g = static_cast<Generator*>(gen);
  const double scale = to - from;
  if (dtype == MTHIP_F32) {
    float* dst = static_cast<float*>(host_dst);
    for (int64_t i = 0; i < n; ++i) dst[i] = static_cast<float>(from + scale * g->uniform_open());
    return MTHIP_OK;
  }
  if (dtype == MTHIP_F64) {
    double* dst = static_cast<double*>(host_dst);
    for (int64_t i = 0; i < n; ++i) dst[i] = from + scale * g->uniform_open();
    return MTHIP_OK;
  }
  if (dtype == MTHIP_F16) {
    uint16_t* dst = static_cast<uint16_t*>(host_dst);
    for (int64_t i = 0; i < n; ++i) dst[i] = float_to_half(static_cast<float>(from + scale * g->uniform_open()));
    return MTHIP_OK;
  }
  return MTHIP_ERR_INVALID;
}

}  // extern "C"
