// group_norm (+ fused SiLU), layer_norm and last-dim softmax: HBM-streaming kernels with
// wave64 shuffle reductions.
//
// group_norm splits every (sample, group) range into chunks of >= 2048 elements (an SD group is
// up to 122,880 elements but there are only B*32 groups): a stats pass writes per-chunk (sum,
// sum of squares), and an apply pass folds the partials of its group(s) with one wave and
// normalises its own chunk -- NCHW, or channels-last through an LDS transpose for the conv that
// follows.  Two launches per group_norm; the apply pass's re-read of the input is served mostly
// by the 256 MB last-level cache.  Statistics follow the reference's one-pass E[x^2] - mean^2
// form (tensor.cpp:18765-18767, 18822-18824) with fp32 tree sums.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <mutex>
#include <type_traits>

#include <algorithm>

#include "activations.h"
#include "common.h"

namespace mthip {
namespace {

// One level of the xor butterfly: v[lane] + v[lane ^ off], for off = 32, 16, 8, 4, 2, 1, with
// the partner fetched by cross-lane VALU moves instead of an LDS permute (ds_bpermute): gfx950's
// v_permlane32_swap / v_permlane16_swap (exchange half-waves / alternate 16-lane rows; the two
// results hold v and its partner, whose sum is the same in either order), DPP row_ror:8 (within
// 16 lanes a rotation by 8 is lane ^ 8), ds_swizzle's xor mode and DPP quad permutes.  The sums
// are those of the shuffle loop, operand for operand.
template <int OFF>
__device__ __forceinline__ float xor_add(float v) {
  const int b = __float_as_int(v);
  if constexpr (OFF == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)b, (unsigned)b, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)b, (unsigned)b, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if constexpr (OFF == 8) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0x128, 0xf, 0xf, false));  // row_ror:8
  } else if constexpr (OFF == 4) {
    return v + __int_as_float(__builtin_amdgcn_ds_swizzle(b, 0x101f));  // xor_mask 4 within 32 lanes
  } else if constexpr (OFF == 2) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0x4e, 0xf, 0xf, false));  // quad_perm [2,3,0,1]
  } else {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, b, 0xb1, 0xf, 0xf, false));  // quad_perm [1,0,3,2]
  }
}

__device__ __forceinline__ float wave_sum(float v) {
  v = xor_add<32>(v);
  v = xor_add<16>(v);
  v = xor_add<8>(v);
  v = xor_add<4>(v);
  v = xor_add<2>(v);
  return xor_add<1>(v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Sum over a 256-thread block; every thread receives the total.
__device__ __forceinline__ float block_sum256(float v, float* scratch /* [4] */) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

// ------------------------------------------------------------------------------ group_norm
// 16-byte vector of T as floats.
template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
  static __device__ __forceinline__ void load(const T* p, float (&f)[N]) { unpack(*reinterpret_cast<const uint4*>(p), f); }
  static __device__ __forceinline__ void unpack(const uint4 r, float (&f)[N]) {
    if constexpr (sizeof(T) == 2) {
      const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[2 * j] = h2f_bits((uint16_t)(w[j] & 0xffffu));
        f[2 * j + 1] = h2f_bits((uint16_t)(w[j] >> 16));
      }
    } else {
      f[0] = __uint_as_float(r.x);
      f[1] = __uint_as_float(r.y);
      f[2] = __uint_as_float(r.z);
      f[3] = __uint_as_float(r.w);
    }
  }
  static __device__ __forceinline__ void store(T* p, const float (&f)[N]) {
    uint4 r;
    if constexpr (sizeof(T) == 2) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = (uint32_t)f2h_fast(f[2 * j]) | ((uint32_t)f2h_fast(f[2 * j + 1]) << 16);
      r = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      r = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
    }
    *reinterpret_cast<uint4*>(p) = r;
  }
};

// The GroupNorm input: NCHW x0[B][C0][HW], optionally followed along channels by x1[B][C1][HW]
// -- the torch.cat([h, skip], dim=1) that feeds an SD up-block ResBlock, read in place.  Within
// each source a group's channels are consecutive planes, so element i of group (b, g) lies at
// i < split ? lo + i : hi + (i - split).
template <typename T>
struct GnSource {
  const T* x0;
  const T* x1;  // nullptr: one source (C1 == 0)
  int64_t C0, C1, gc, HW, groups;
  __device__ __forceinline__ void group(int64_t bg, const T*& lo, const T*& hi, int64_t& split) const {
    const int64_t b = (uint32_t)bg / (uint32_t)groups, c = (bg - b * groups) * gc;
    lo = x0 + (b * C0 + c) * HW;
    const int64_t n0 = c < C0 ? (C0 - c < gc ? C0 - c : gc) : 0;
    split = n0 * HW;
    hi = x1 ? x1 + (b * C1 + (c + n0 - C0)) * HW - split : lo;
  }
  __device__ __forceinline__ const T* channel(int64_t b, int64_t c) const {
    return c < C0 ? x0 + (b * C0 + c) * HW : x1 + (b * C1 + (c - C0)) * HW;
  }
};

// Per-chunk (sum, sum of squares) of one (sample, group) range.  VECT: the range, the chunk
// bounds and the source split are whole 16-byte vectors.
template <typename T, bool VECT, bool CAT>
__global__ __launch_bounds__(256) void group_norm_stats_kernel(const GnSource<T> src, float2* __restrict__ partial,
                                                               int64_t group_size, int64_t chunk, int splits) {
  __shared__ float red[8];
  const int64_t bg = blockIdx.y;
  const int split = blockIdx.x;
  const int64_t begin = (int64_t)split * chunk;
  const int64_t end = min(begin + chunk, group_size);
  const T* lo = src.x0 + bg * group_size;  // one source: the (sample, group) block is contiguous
  const T* hi = lo;
  int64_t cut = group_size;
  if constexpr (CAT) src.group(bg, lo, hi, cut);
  float s = 0.0f, ss = 0.0f;
  if constexpr (VECT) {
    constexpr int V = Vec16<T>::N;
#pragma unroll 4
    for (int64_t i = begin + (int64_t)threadIdx.x * V; i < end; i += 256 * V) {
      float f[V];
      Vec16<T>::load((i < cut ? lo : hi) + i, f);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        s += f[j];
        ss += f[j] * f[j];
      }
    }
  } else {
    for (int64_t i = begin + threadIdx.x; i < end; i += 256) {
      const float v = Elem<T>::load(i < cut ? lo : hi, i);
      s += v;
      ss += v * v;
    }
  }
  s = wave_sum(s);
  ss = wave_sum(ss);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    red[wave] = s;
    red[4 + wave] = ss;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    partial[bg * splits + split] = make_float2(red[0] + red[1] + red[2] + red[3], red[4] + red[5] + red[6] + red[7]);
}

// (mean, 1/sqrt(var + eps)) from a group's sum and sum of squares over n elements.
__device__ __forceinline__ float2 gn_stats(float s, float ss, float n, float eps) {
  const float mean = s / n;
  const float var = fmaxf(0.0f, ss / n - mean * mean);
  return make_float2(mean, 1.0f / sqrtf(var + eps));
}

// (mean, 1/sqrt(var + eps)) of one (sample, group) from its chunk partials, folded by one wave
// (every lane returns the result).
__device__ __forceinline__ float2 fold_group_stats(const float2* __restrict__ partial, int64_t bg, int splits,
                                                   int64_t group_size, float eps, int lane) {
  float s = 0.0f, ss = 0.0f;
  for (int i = lane; i < splits; i += 64) {
    const float2 p = partial[bg * splits + i];
    s += p.x;
    ss += p.y;
  }
  s = wave_sum(s);
  ss = wave_sum(ss);
  return gn_stats(s, ss, (float)group_size, eps);
}

// Normalised value of one element in the reference's per-dtype form, with the optional SiLU
// applied to the narrowed normalised value (the unfused op sequence narrows in between).
// P is the parameter (and computation) dtype: fp16 parameters take the fp16 path's form; fp32
// parameters over fp16 data are the "upcast" pattern group_norm(x.float(), w32, b32).half(),
// i.e. the fp32 path's form narrowed once.
// Statistics of the groups [0, ng) starting at (sample, group) bg0, one group per wave at a
// time, into st[k]; a wave takes groups k and k + 4 together so that both loads of partials are
// in flight before either reduction (splits <= 64: one partial per lane).  The same sums, in the
// same order, as fold_group_stats.
template <int NWAVES = 4>
__device__ __forceinline__ void fold_groups(const float2* __restrict__ partial, int64_t bg0, int ng, int splits,
                                            int64_t group_size, float eps, int wave, int lane, float2* st) {
  const float n = (float)group_size;
  for (int k0 = wave; k0 < ng; k0 += 2 * NWAVES) {
    const int k1 = k0 + NWAVES;
    float2 p0 = make_float2(0.0f, 0.0f), p1 = make_float2(0.0f, 0.0f);
    if (lane < splits) {
      p0 = partial[(bg0 + k0) * splits + lane];
      if (k1 < ng) p1 = partial[(bg0 + k1) * splits + lane];
    }
    float s0 = 0.0f, ss0 = 0.0f, s1 = 0.0f, ss1 = 0.0f;
    s0 += p0.x;
    ss0 += p0.y;
    s1 += p1.x;
    ss1 += p1.y;
    s0 = wave_sum(s0);
    ss0 = wave_sum(ss0);
    s1 = wave_sum(s1);
    ss1 = wave_sum(ss1);
    if (lane == 0) {
      st[k0] = gn_stats(s0, ss0, n, eps);
      if (k1 < ng) st[k1] = gn_stats(s1, ss1, n, eps);
    }
  }
}

template <typename T, typename P>
__device__ __forceinline__ float gn_value(float v, float mean, float inv, float gm, float bt, int fuse_silu) {
  float out;
  if constexpr (sizeof(P) == 2) {
    // affine_float32_to_half_bits(scale = gamma*inv, shift = beta - mean*gamma*inv)
    // (tensor.cpp:18768-18781).
    const float scale = gm * inv;
    const float shift = bt - mean * gm * inv;
    out = v * scale + shift;
  } else {
    // (x - mean) * inv * gamma + beta (tensor.cpp:18834-18837).
    out = (v - mean) * inv * gm + bt;
  }
  if (fuse_silu) out = apply_unary<T>(MTHIP_UNARY_SILU, Elem<T>::round_trip(out));
  return out;
}

template <typename T, typename P, bool VECT>
__global__ __launch_bounds__(256) void group_norm_apply_kernel(const T* __restrict__ x, const P* __restrict__ gamma,
                                                               const P* __restrict__ beta, T* __restrict__ y,
                                                               const float2* __restrict__ partial, int64_t C,
                                                               int64_t groups, int64_t inner, int64_t group_size,
                                                               int64_t chunk, int splits, float eps, int fuse_silu) {
  __shared__ float2 st_s;
  const int64_t bg = blockIdx.y;
  const int split = blockIdx.x;
  if (threadIdx.x < 64) {
    const float2 st = fold_group_stats(partial, bg, splits, group_size, eps, threadIdx.x);
    if (threadIdx.x == 0) st_s = st;
  }
  __syncthreads();
  const float mean = st_s.x, inv = st_s.y;
  const int64_t g = (uint32_t)bg % (uint32_t)groups;
  const int64_t gc = (uint32_t)C / (uint32_t)groups;
  const int64_t begin = (int64_t)split * chunk;
  const int64_t end = min(begin + chunk, group_size);
  const T* xb = x + bg * group_size;
  T* yb = y + bg * group_size;
  if constexpr (VECT) {
    // inner % V == 0, so a vector never straddles two channels.
    constexpr int V = Vec16<T>::N;
    for (int64_t i = begin + (int64_t)threadIdx.x * V; i < end; i += 256 * V) {
      const int64_t c = g * gc + (uint32_t)i / (uint32_t)inner;
      const float gm = gamma ? Elem<P>::load(gamma, c) : 1.0f;
      const float bt = beta ? Elem<P>::load(beta, c) : 0.0f;
      float f[V];
      Vec16<T>::load(xb + i, f);
      if constexpr (sizeof(T) == 2) {
        if (fuse_silu) {
          // Narrow the normalised value once and apply the fp16 SiLU to its bits: the same
          // halves as narrowing, widening, SiLU and narrowing again, with one conversion.
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t lo = silu_half(f2h_fast(gn_value<T, P>(f[2 * j], mean, inv, gm, bt, 0)));
            const uint32_t hi = silu_half(f2h_fast(gn_value<T, P>(f[2 * j + 1], mean, inv, gm, bt, 0)));
            w[j] = lo | (hi << 16);
          }
          *reinterpret_cast<uint4*>(yb + i) = make_uint4(w[0], w[1], w[2], w[3]);
          continue;
        }
      }
#pragma unroll
      for (int j = 0; j < V; ++j) f[j] = gn_value<T, P>(f[j], mean, inv, gm, bt, fuse_silu);
      Vec16<T>::store(yb + i, f);
    }
  } else {
    for (int64_t i = begin + threadIdx.x; i < end; i += 256) {
      const int64_t c = g * gc + (uint32_t)i / (uint32_t)inner;
      const float gm = gamma ? Elem<P>::load(gamma, c) : 1.0f;
      const float bt = beta ? Elem<P>::load(beta, c) : 0.0f;
      Elem<T>::store(yb, i, gn_value<T, P>(Elem<T>::load(xb, i), mean, inv, gm, bt, fuse_silu));
    }
  }
}

// GroupNorm in one pass over x for batches with many (sample, group) pairs (>= 2 per CU): a
// 1024-thread workgroup holds one whole group in registers, so x is read once (the two-kernel
// path reads it twice).  Values are bit-identical to group_norm_stats_kernel +
// group_norm_apply_kernel<T, P, true>: the four 256-thread parts of the workgroup take chunks
// p, p + 4, ... and replay the stats kernel's per-thread vectors (IPC vectors of V elements per
// chunk, summed in order), wave butterflies and four-wave combine, and wave 0 folds the chunk
// partials as fold_group_stats does.  Needs NCHW, whole 16-byte vectors, at most 4 * CPT chunks
// and chunk == IPC * 256 * V (all but possibly the last chunk full).  Four parts rather than two
// halve each thread's serial reduce-and-store work between its loads and the next group's
// (64x batch fp16: 200 -> 158 us); more than 10 fp16 vectors per thread would go to scratch.
template <typename T, typename P, int CPT, int IPC>
__global__ __launch_bounds__(1024) void group_norm_single_kernel(const T* __restrict__ x, const P* __restrict__ gamma,
                                                                const P* __restrict__ beta, T* __restrict__ y,
                                                                int64_t C, int64_t groups, int64_t inner,
                                                                int64_t group_size, int64_t chunk, int splits,
                                                                float eps, int fuse_silu, FastDiv div_inner) {
  constexpr int V = Vec16<T>::N;
  constexpr int NPART = 4;
  __shared__ float red_s[NPART * CPT][4], red_ss[NPART * CPT][4];
  __shared__ float2 st_s;
  const int64_t bg = blockIdx.x;
  const int t = threadIdx.x & 255, part = threadIdx.x >> 8, wave = (threadIdx.x >> 6) & 3, lane = threadIdx.x & 63;
  const T* xb = x + bg * group_size;
  T* yb = y + bg * group_size;
  uint4 d[CPT][IPC];
  // phase 1: chunk k = 4 * kk + part of this thread's part; the stats kernel's thread t
#pragma unroll
  for (int kk = 0; kk < CPT; ++kk) {
    const int k = NPART * kk + part;
    const int64_t begin = (int64_t)k * chunk, end = min(begin + chunk, group_size);
    float s = 0.0f, ss = 0.0f;
#pragma unroll
    for (int it = 0; it < IPC; ++it) {
      const int64_t i = begin + (int64_t)(t + it * 256) * V;
      d[kk][it] = make_uint4(0u, 0u, 0u, 0u);
      if (k < splits && i < end) {
        d[kk][it] = *reinterpret_cast<const uint4*>(xb + i);
        float f[V];
        Vec16<T>::unpack(d[kk][it], f);
#pragma unroll
        for (int j = 0; j < V; ++j) {
          s += f[j];
          ss += f[j] * f[j];
        }
      }
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    if (lane == 0 && k < splits) {
      red_s[k][wave] = s;
      red_ss[k][wave] = ss;
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    // the chunk partials (stats kernel: red[0] + red[1] + red[2] + red[3]), folded as
    // fold_group_stats folds them (splits <= 64: one per lane)
    float s = 0.0f, ss = 0.0f;
    if (lane < splits) {
      s += red_s[lane][0] + red_s[lane][1] + red_s[lane][2] + red_s[lane][3];
      ss += red_ss[lane][0] + red_ss[lane][1] + red_ss[lane][2] + red_ss[lane][3];
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    if (lane == 0) st_s = gn_stats(s, ss, (float)group_size, eps);
  }
  __syncthreads();
  const float mean = st_s.x, inv = st_s.y;
  const int64_t g = (uint32_t)bg % (uint32_t)groups;
  const int64_t gc = (uint32_t)C / (uint32_t)groups;
  // phase 2: group_norm_apply_kernel<T, P, true>'s arithmetic on the held vectors (the fused
  // SiLU chosen outside the loop, which keeps each loop body small enough to unroll: the held
  // vectors must stay in registers)
  auto apply = [&](auto silu_c) {
    constexpr bool SILU = decltype(silu_c)::value;
#pragma unroll
    for (int kk = 0; kk < CPT; ++kk) {
      const int k = NPART * kk + part;
      const int64_t begin = (int64_t)k * chunk, end = min(begin + chunk, group_size);
#pragma unroll
      for (int it = 0; it < IPC; ++it) {
        const int64_t i = begin + (int64_t)(t + it * 256) * V;
        if (k < splits && i < end) {
          const int64_t c = g * gc + div_inner.div((uint32_t)i);
          const float gm = gamma ? Elem<P>::load(gamma, c) : 1.0f;
          const float bt = beta ? Elem<P>::load(beta, c) : 0.0f;
          float f[V];
          Vec16<T>::unpack(d[kk][it], f);
          if constexpr (SILU && sizeof(T) == 2) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t lo = silu_half(f2h_fast(gn_value<T, P>(f[2 * j], mean, inv, gm, bt, 0)));
              const uint32_t hi = silu_half(f2h_fast(gn_value<T, P>(f[2 * j + 1], mean, inv, gm, bt, 0)));
              w[j] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(yb + i) = make_uint4(w[0], w[1], w[2], w[3]);
          } else {
#pragma unroll
            for (int j = 0; j < V; ++j) f[j] = gn_value<T, P>(f[j], mean, inv, gm, bt, SILU ? 1 : 0);
            Vec16<T>::store(yb + i, f);
          }
        }
      }
    }
  };
  if (fuse_silu)
    apply(std::true_type{});
  else
    apply(std::false_type{});
}

// Same values written channels-last: y[b][p][0..Cp) with channels C..Cp-1 zero, the layout the
// implicit-GEMM conv stages its input in.  A workgroup transposes a 64-channel x 64-pixel tile
// through LDS: reads walk pixels of one channel, writes walk channels of one pixel.
template <typename T, typename P>
__global__ __launch_bounds__(256) void group_norm_apply_nhwc_kernel(const T* __restrict__ x,
                                                                    const P* __restrict__ gamma,
                                                                    const P* __restrict__ beta, T* __restrict__ y,
                                                                    const float2* __restrict__ partial, int64_t C,
                                                                    int64_t Cp, int64_t groups, int64_t HW,
                                                                    int splits, float eps, int fuse_silu, int vec_io) {
  constexpr int TP = 64 + 2;  // LDS row pitch (elements)
  constexpr int V = Vec16<T>::N;
  __shared__ T tile[64 * TP];
  __shared__ float2 st_s[64];
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int t = threadIdx.x;
  const uint32_t gc = (uint32_t)C / (uint32_t)groups;
  const int64_t g_first = (uint32_t)c0 / gc;
  const int cl = t >> 2, pl0 = (t & 3) * 16;
  const int64_t c = c0 + cl;
  // The tile's input and affine parameters are requested first; the group statistics are
  // folded while they arrive.
  float f[16];
  float gm = 1.0f, bt = 0.0f;
  if (c < C) {
    if (gamma) gm = Elem<P>::load(gamma, c);
    if (beta) bt = Elem<P>::load(beta, c);
    const T* xr = x + (b * C + c) * HW + p0 + pl0;
    if (vec_io && p0 + pl0 + 16 <= HW) {
#pragma unroll
      for (int j = 0; j < 16; j += V) {
        float part[V];
        Vec16<T>::load(xr + j, part);
#pragma unroll
        for (int k = 0; k < V; ++k) f[j + k] = part[k];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) f[j] = p0 + pl0 + j < HW ? Elem<T>::load(xr, j) : 0.0f;
    }
  }
  {
    // statistics of the (at most 64) groups this tile's channels belong to, one wave each
    const int64_t c_last = (c0 + 64 < C ? c0 + 64 : C) - 1;
    const int ng = c0 < C ? (int)((uint32_t)c_last / gc - g_first + 1) : 0;
    fold_groups(partial, b * groups + g_first, ng, splits, (int64_t)gc * HW, eps, t >> 6, t & 63, st_s);
  }
  __syncthreads();
  {
    if (c < C) {
      const float2 st = st_s[(uint32_t)c / gc - g_first];
#pragma unroll
      for (int j = 0; j < 16; ++j) f[j] = gn_value<T, P>(f[j], st.x, st.y, gm, bt, fuse_silu);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) f[j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if constexpr (sizeof(T) == 2)
        tile[(pl0 + j) * TP + cl] = f2h_fast(f[j]);
      else
        tile[(pl0 + j) * TP + cl] = f[j];
    }
  }
  __syncthreads();
  {
    const int pl = t >> 2, cl0 = (t & 3) * 16;
    const int64_t p = p0 + pl;
    if (p < HW) {
      T* yr = y + (b * HW + p) * Cp + c0 + cl0;
      if (vec_io && c0 + cl0 + 16 <= Cp) {
#pragma unroll
        for (int j = 0; j < 16; j += V) {
          T part[V];
#pragma unroll
          for (int k = 0; k < V; ++k) part[k] = tile[pl * TP + cl0 + j + k];
          *reinterpret_cast<uint4*>(yr + j) = *reinterpret_cast<const uint4*>(part);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (c0 + cl0 + j < Cp) yr[j] = tile[pl * TP + cl0 + j];
      }
    }
  }
}

// fp16 SiLU of every half value (silu_half, the reference's fp16 SiLU bit for bit): the
// channels-last apply kernel looks the activation of each narrowed normalised value up by its
// bits, one gather where evaluating it costs ~20 vector instructions per element.  Filled once
// per device.
__device__ __align__(16) uint16_t g_silu_f16_table[65536];

__global__ void silu_f16_table_kernel(uint16_t* tab) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 65536) tab[i] = silu_half((uint16_t)i);
}

const uint16_t* silu_f16_table(int device, hipStream_t s) {
  static const uint16_t* ptr[64] = {nullptr};
  static std::mutex init_mutex;  // first use from several host threads fills the table once
  if (device < 0 || device >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(init_mutex);
  if (!ptr[device]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_silu_f16_table)) != hipSuccess) return nullptr;
    hipLaunchKernelGGL(silu_f16_table_kernel, dim3(256), dim3(256), 0, s, static_cast<uint16_t*>(p));
    if (hipGetLastError() != hipSuccess) return nullptr;
    // Under stream capture the fill is only recorded (it runs with each replay, ahead of the
    // kernel that reads the table), so the table counts as ready only after an eager fill.
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) return nullptr;
    if (st != hipStreamCaptureStatusNone) return static_cast<const uint16_t*>(p);
    ptr[device] = static_cast<const uint16_t*>(p);
  }
  return ptr[device];
}

// fp16 channels-last apply for 16-byte aligned rows (HW % 8 == 0, Cp % 8 == 0): a 64-channel x
// 64-pixel tile, thread t holding channels (2*(t%32), +1) of 8 consecutive pixels.  Both input
// rows are read with 16-byte loads, each normalised pixel pair is written to LDS as one 32-bit
// word of the pixel's channel row, and each output pixel row leaves as 16-byte stores of
// 16-byte LDS reads: 4 LDS instructions per thread where an element-wise transpose needs 32.
// The fused SiLU is a lookup of the narrowed normalised value (silu_f16_table).
// raw (nullable) also receives the input itself channels-last, [B][HW][Cp]: the operand of a
// 1x1 shortcut conv on the same (concatenated) input.
template <typename P, bool CAT, int TPX = 64>
__global__ __launch_bounds__(4 * TPX) void group_norm_apply_nhwc_f16_kernel(
    const GnSource<uint16_t> src, const P* __restrict__ gamma, const P* __restrict__ beta, uint16_t* __restrict__ y,
    uint16_t* __restrict__ raw, const float2* __restrict__ partial, int64_t C, int64_t Cp, int64_t groups, int64_t HW,
    int splits, float eps, const uint16_t* __restrict__ silu_tab) {
  constexpr int PW = 36;  // LDS words per pixel row: 64 channels + 8 pad (16-byte aligned rows)
  // TPX pixels x 64 channels per workgroup of 4 * TPX threads (TPX = 32 doubles the workgroups
  // of the small latents)
  __shared__ uint32_t tile[(CAT ? 2 : 1) * TPX * PW];
  uint32_t* const raw_tile = tile + TPX * PW;  // CAT only
  __shared__ float2 st_s[64];
  const int64_t b = blockIdx.z;
  const int64_t p0 = (int64_t)blockIdx.x * TPX, c0 = (int64_t)blockIdx.y * 64;
  const int t = threadIdx.x;
  const int cp = t & 31, po = t >> 5;  // channel pair, pixel octet
  const int64_t ca = c0 + 2 * cp;
  const int64_t pix = p0 + po * 8;
  const uint32_t gc = (uint32_t)C / (uint32_t)groups;
  const int64_t g_first = (uint32_t)c0 / gc;
  float fa[8], fb[8];
  float ga = 1.0f, ba = 0.0f, gb = 1.0f, bb = 0.0f;
  auto load_row = [&](int64_t c, float (&f)[8]) {
    if (c < C && pix < HW) {
      // HW % 8 == 0: an octet is either whole or past the end
      Vec16<uint16_t>::load((CAT ? src.channel(b, c) : src.x0 + (b * C + c) * HW) + pix, f);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = 0.0f;
    }
  };
  load_row(ca, fa);
  load_row(ca + 1, fb);
  if (ca < C) {
    if (gamma) ga = Elem<P>::load(gamma, ca);
    if (beta) ba = Elem<P>::load(beta, ca);
  }
  if (ca + 1 < C) {
    if (gamma) gb = Elem<P>::load(gamma, ca + 1);
    if (beta) bb = Elem<P>::load(beta, ca + 1);
  }
  {
    // statistics of the (at most 64) groups this tile's channels belong to, one wave each
    const int64_t c_last = (c0 + 64 < C ? c0 + 64 : C) - 1;
    const int ng = c0 < C ? (int)((uint32_t)c_last / gc - g_first + 1) : 0;
    fold_groups<TPX / 16>(partial, b * groups + g_first, ng, splits, (int64_t)gc * HW, eps, t >> 6, t & 63, st_s);
  }
  __syncthreads();
  {
    const float2 sa = ca < C ? st_s[(uint32_t)ca / gc - g_first] : make_float2(0.0f, 0.0f);
    const float2 sb = ca + 1 < C ? st_s[(uint32_t)(ca + 1) / gc - g_first] : make_float2(0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t ha = ca < C ? f2h_fast(gn_value<uint16_t, P>(fa[j], sa.x, sa.y, ga, ba, 0)) : 0u;
      uint32_t hb = ca + 1 < C ? f2h_fast(gn_value<uint16_t, P>(fb[j], sb.x, sb.y, gb, bb, 0)) : 0u;
      if (silu_tab) {
        // padding channels stay 0 (SiLU(0) = 0 anyway)
        ha = silu_tab[ha];
        hb = silu_tab[hb];
      }
      tile[(po * 8 + j) * PW + cp] = ha | (hb << 16);
      if (CAT && raw) raw_tile[(po * 8 + j) * PW + cp] = (uint32_t)f2h_fast(fa[j]) | ((uint32_t)f2h_fast(fb[j]) << 16);
    }
  }
  __syncthreads();
  {
    const int pl = t >> 2, q = (t & 3) * 8;  // pixel row, word offset (16 channels)
    const int64_t p = p0 + pl;
    const int64_t cq = c0 + 2 * q;
    if (p < HW) {
      uint16_t* yr = y + (b * HW + p) * Cp + cq;
      const uint4 lo = *reinterpret_cast<const uint4*>(&tile[pl * PW + q]);
      const uint4 hi = *reinterpret_cast<const uint4*>(&tile[pl * PW + q + 4]);
      if (cq + 8 <= Cp) *reinterpret_cast<uint4*>(yr) = lo;
      if (cq + 16 <= Cp) *reinterpret_cast<uint4*>(yr + 8) = hi;
      if (CAT && raw) {
        uint16_t* rr = raw + (b * HW + p) * Cp + cq;
        const uint4 rlo = *reinterpret_cast<const uint4*>(&raw_tile[pl * PW + q]);
        const uint4 rhi = *reinterpret_cast<const uint4*>(&raw_tile[pl * PW + q + 4]);
        if (cq + 8 <= Cp) *reinterpret_cast<uint4*>(rr) = rlo;
        if (cq + 16 <= Cp) *reinterpret_cast<uint4*>(rr + 8) = rhi;
      }
    }
  }
}

// ------------------------------------------------------------------------------ layer_norm
// One wave per row; the row lives in registers (up to 64*MAXV elements).
// P: parameter / computation dtype, as for group_norm (fp32 over fp16 data = the upcast pattern
// layer_norm(x.float(), w32, b32).half()).
template <typename T, typename P, int MAXV>
__global__ __launch_bounds__(256) void layer_norm_kernel(const T* __restrict__ x, const P* __restrict__ w,
                                                         const P* __restrict__ b, T* __restrict__ y, int64_t rows,
                                                         int64_t N, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * N;
  float v[MAXV];
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t i = lane + (int64_t)j * 64;
    v[j] = i < N ? Elem<T>::load(xr, i) : 0.0f;
    s += v[j];
  }
  const float n = (float)N;
  const float mean = wave_sum(s) / n;
  float var;
  if constexpr (sizeof(P) == 2) {
    // fp16: two-pass centred variance (tensor.cpp:17531-17545).
    float css = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int64_t i = lane + (int64_t)j * 64;
      const float c = v[j] - mean;
      css += i < N ? c * c : 0.0f;
    }
    var = fmaxf(0.0f, wave_sum(css) / n);
  } else {
    // fp32: one-pass sum of squares (tensor.cpp:17577-17587).
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) ss += v[j] * v[j];
    var = fmaxf(0.0f, wave_sum(ss) / n - mean * mean);
  }
  const float inv = 1.0f / sqrtf(var + eps);
  T* yr = y + row * N;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t i = lane + (int64_t)j * 64;
    if (i < N) {
      float o = (v[j] - mean) * inv;
      if (w) o = o * Elem<P>::load(w, i);
      if (b) o = o + Elem<P>::load(b, i);
      Elem<T>::store(yr, i, o);
    }
  }
}

// V consecutive parameters (V a multiple of the 16-byte vector width of P) as floats.
template <typename P, int V>
__device__ __forceinline__ void load_params(const P* p, float (&f)[V]) {
  constexpr int PV = Vec16<P>::N;
#pragma unroll
  for (int k = 0; k < V; k += PV) {
    float part[PV];
    Vec16<P>::load(p + k, part);
#pragma unroll
    for (int q = 0; q < PV; ++q) f[k + q] = part[q];
  }
}

// Rows whose length is a whole number of 16-byte chunks (every SD LayerNorm: 320..1280
// channels).  One wave per RPW rows; a row lives in registers as CPL 16-byte chunks per lane.  The affine
// parameters are loaded once per wave as 16-byte vectors, and all RPW rows are requested before
// the first is reduced, so their loads are in flight together.
template <typename T, typename P, int CPL, int RPW>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(const T* __restrict__ x, const P* __restrict__ w,
                                                             const P* __restrict__ b, T* __restrict__ y, int64_t rows,
                                                             int64_t N, float eps) {
  constexpr int V = Vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  if (row0 >= rows) return;
  const int chunks = (int)(N / V);
  if constexpr (sizeof(T) == 2 && sizeof(P) == 4) {
    // fp16 rows, fp32 parameters (the SD transformer's LayerNorms): the rows stay as raw
    // halves, every sum term, square and centring subtraction is one v_fma_mix_f32 on them
    // (the same roundings as widening first), and the outputs are narrowed pairwise with
    // f2h_rtz_pack; a row in which some lane met a value that covers not (NaN, infinity,
    // |value| >= 65520) is narrowed again with f2h_fast.
    uint4 hr[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        hr[r][j] = make_uint4(0u, 0u, 0u, 0u);
        if (row0 + r < rows && c < chunks) hr[r][j] = *reinterpret_cast<const uint4*>(x + (row0 + r) * N + c * V);
      }
    float wv[CPL][V], bv[CPL][V];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
#pragma unroll
      for (int k = 0; k < V; ++k) {
        wv[j][k] = 1.0f;
        bv[j][k] = 0.0f;
      }
      if (c < chunks) {
        if (w) load_params<P, V>(w + c * V, wv[j]);
        if (b) load_params<P, V>(b + c * V, bv[j]);
      }
    }
    const float n = (float)N;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      if (row0 + r >= rows) break;
      // fp32: one-pass sum of squares (tensor.cpp:17577-17587), terms in element order
      float s = 0.0f, ss = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const uint32_t wd[4] = {hr[r][j].x, hr[r][j].y, hr[r][j].z, hr[r][j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s = acc_add_half<false>(s, wd[q]);
          ss = acc_add_sq_half<false>(ss, wd[q]);
          s = acc_add_half<true>(s, wd[q]);
          ss = acc_add_sq_half<true>(ss, wd[q]);
        }
      }
      s = wave_sum(s);
      ss = wave_sum(ss);
      const float mean = s / n;
      const float var = fmaxf(0.0f, ss / n - mean * mean);
      const float inv = 1.0f / sqrtf(var + eps);
      T* yr = y + (row0 + r) * N;
      float o[CPL][V];
      float amax = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const uint32_t wd[4] = {hr[r][j].x, hr[r][j].y, hr[r][j].z, hr[r][j].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float t0 = acc_add_half<false>(-mean, wd[q]) * inv, t1 = acc_add_half<true>(-mean, wd[q]) * inv;
          if (w) {
            t0 = t0 * wv[j][2 * q];
            t1 = t1 * wv[j][2 * q + 1];
          }
          if (b) {
            t0 = t0 + bv[j][2 * q];
            t1 = t1 + bv[j][2 * q + 1];
          }
          o[j][2 * q] = t0;
          o[j][2 * q + 1] = t1;
          amax = abs_max_nan(abs_max_nan(amax, t0), t1);
        }
      }
      const bool redo = __builtin_amdgcn_ballot_w64(!(amax < 65520.0f)) != 0;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        if (c < chunks) {
          uint4 st;
          if (!redo) {
            st = make_uint4(f2h_rtz_pack(o[j][0], o[j][1]), f2h_rtz_pack(o[j][2], o[j][3]), f2h_rtz_pack(o[j][4], o[j][5]),
                            f2h_rtz_pack(o[j][6], o[j][7]));
            *reinterpret_cast<uint4*>(yr + c * V) = st;
          } else {
            Vec16<T>::store(yr + c * V, o[j]);
          }
        }
      }
    }
    return;
  }
  float v[RPW][CPL][V];
#pragma unroll
  for (int r = 0; r < RPW; ++r)
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (row0 + r < rows && c < chunks) {
        Vec16<T>::load(x + (row0 + r) * N + c * V, v[r][j]);
      } else {
#pragma unroll
        for (int k = 0; k < V; ++k) v[r][j][k] = 0.0f;
      }
    }
  float wv[CPL][V], bv[CPL][V];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      wv[j][k] = 1.0f;
      bv[j][k] = 0.0f;
    }
    if (c < chunks) {
      if (w) load_params<P, V>(w + c * V, wv[j]);
      if (b) load_params<P, V>(b + c * V, bv[j]);
    }
  }
  const float n = (float)N;
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    if (row0 + r >= rows) break;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int k = 0; k < V; ++k) s += v[r][j][k];
    float mean, var;
    if constexpr (sizeof(P) == 2) {
      // fp16: two-pass centred variance (tensor.cpp:17531-17545).
      mean = wave_sum(s) / n;
      float css = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
        if (lane + 64 * j < chunks)
#pragma unroll
          for (int k = 0; k < V; ++k) {
            const float c = v[r][j][k] - mean;
            css += c * c;
          }
      var = fmaxf(0.0f, wave_sum(css) / n);
    } else {
      // fp32: one-pass sum of squares (tensor.cpp:17577-17587); both sums reduce together.
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int k = 0; k < V; ++k) ss += v[r][j][k] * v[r][j][k];
      s = wave_sum(s);
      ss = wave_sum(ss);
      mean = s / n;
      var = fmaxf(0.0f, ss / n - mean * mean);
    }
    const float inv = 1.0f / sqrtf(var + eps);
    T* yr = y + (row0 + r) * N;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c < chunks) {
        float o[V];
#pragma unroll
        for (int k = 0; k < V; ++k) {
          float t = (v[r][j][k] - mean) * inv;
          if (w) t = t * wv[j][k];
          if (b) t = t + bv[j][k];
          o[k] = t;
        }
        Vec16<T>::store(yr + c * V, o);
      }
    }
  }
}

template <typename T, typename P>
__global__ __launch_bounds__(256) void layer_norm_long_kernel(const T* __restrict__ x, const P* __restrict__ w,
                                                              const P* __restrict__ b, T* __restrict__ y, int64_t N,
                                                              float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * N;
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < N; i += 256) s += Elem<T>::load(xr, i);
  const float n = (float)N;
  const float mean = block_sum256(s, red) / n;
  float var;
  if constexpr (sizeof(P) == 2) {
    float css = 0.0f;
    for (int64_t i = threadIdx.x; i < N; i += 256) {
      const float c = Elem<T>::load(xr, i) - mean;
      css += c * c;
    }
    var = fmaxf(0.0f, block_sum256(css, red) / n);
  } else {
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < N; i += 256) {
      const float v = Elem<T>::load(xr, i);
      ss += v * v;
    }
    var = fmaxf(0.0f, block_sum256(ss, red) / n - mean * mean);
  }
  const float inv = 1.0f / sqrtf(var + eps);
  T* yr = y + row * N;
  for (int64_t i = threadIdx.x; i < N; i += 256) {
    float o = (Elem<T>::load(xr, i) - mean) * inv;
    if (w) o = o * Elem<P>::load(w, i);
    if (b) o = o + Elem<P>::load(b, i);
    Elem<T>::store(yr, i, o);
  }
}

// ------------------------------------------------------------------------------ softmax
// e^d for d = x - max <= 0.  Half-width storage takes the native 2^x of d log2(e): its error
// (about 1e-6 relative for every d that leaves a nonzero half) is far below a half ulp (5e-4),
// and it costs a multiply and one transcendental where expf's range reduction costs eight more
// operations per element, which made the 16-bit softmax VALU- rather than HBM-bound.  fp32
// storage keeps expf.
template <typename T>
__device__ __forceinline__ float softmax_exp(float d) {
  if constexpr (sizeof(T) == 2) return __builtin_amdgcn_exp2f(d * 1.44269504088896341f);
  return expf(d);
}

template <typename T, int MAXV>
__global__ __launch_bounds__(256) void softmax_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                      int64_t cols, int divide) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  float v[MAXV];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t i = lane + (int64_t)j * 64;
    v[j] = i < cols ? Elem<T>::load(xr, i) : -INFINITY;
    mx = fmaxf(mx, v[j]);
  }
  mx = wave_max(mx);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t i = lane + (int64_t)j * 64;
    v[j] = i < cols ? softmax_exp<T>(v[j] - mx) : 0.0f;
    s += v[j];
  }
  s = wave_sum(s);
  const float inv = 1.0f / s;
  T* yr = y + row * cols;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int64_t i = lane + (int64_t)j * 64;
    if (i < cols) Elem<T>::store(yr, i, divide ? v[j] / s : v[j] * inv);
  }
}

// Rows whose length is a whole number of 16-byte chunks, 16-byte aligned: one wave per row,
// each lane holding CPL chunks (lane + 64 j) in registers, so every load and store moves 16 bytes
// per lane.
template <typename T, int CPL>
__global__ __launch_bounds__(256) void softmax_vec_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows,
                                                          int64_t cols, int divide) {
  constexpr int V = Vec16<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int chunks = (int)(cols / V);
  const T* xr = x + row * cols;
  float v[CPL][V];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
      Vec16<T>::load(xr + (int64_t)c * V, v[j]);
    } else {
#pragma unroll
      for (int q = 0; q < V; ++q) v[j][q] = -INFINITY;
    }
#pragma unroll
    for (int q = 0; q < V; ++q) mx = fmaxf(mx, v[j][q]);
  }
  mx = wave_max(mx);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const bool in = lane + 64 * j < chunks;
#pragma unroll
    for (int q = 0; q < V; ++q) {
      v[j][q] = in ? softmax_exp<T>(v[j][q] - mx) : 0.0f;
      s += v[j][q];
    }
  }
  s = wave_sum(s);
  const float inv = 1.0f / s;
  T* yr = y + row * cols;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
#pragma unroll
      for (int q = 0; q < V; ++q) v[j][q] = divide ? v[j][q] / s : v[j][q] * inv;
      Vec16<T>::store(yr + (int64_t)c * V, v[j]);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_long_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t cols,
                                                           int divide) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float mx = -INFINITY;
  for (int64_t i = threadIdx.x; i < cols; i += 256) mx = fmaxf(mx, Elem<T>::load(xr, i));
  mx = wave_max(mx);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += 256) s += softmax_exp<T>(Elem<T>::load(xr, i) - mx);
  s = block_sum256(s, red);
  const float inv = 1.0f / s;
  T* yr = y + row * cols;
  for (int64_t i = threadIdx.x; i < cols; i += 256) {
    const float e = softmax_exp<T>(Elem<T>::load(xr, i) - mx);
    Elem<T>::store(yr, i, divide ? e / s : e * inv);
  }
}

// Halves of the one-launch GroupNorm's LDS tile: a whole group of up to 5 chunks per part, else
// a 64 KB share ([gc][HW / NSPLIT + 8] rows, checked by the launcher), so two workgroups of any
// instance fit one CU's LDS.
constexpr int gn1_tile_halves(int cpt) { return (cpt <= 5 ? 4 * cpt * 2048 : 32768) + 4096; }

// Channels-last GroupNorm (+ SiLU) of fp16 NCHW input in ONE launch, for groups of at most
// 4 * CPT stats chunks of <= 2048 elements (every SD group, the up-block concatenations up to
// 122880 elements included): NSPLIT 1024-thread workgroups per (sample, group), each covering
// HW / NSPLIT pixels of it.
//  phase 1: every workgroup reads the whole group (its chunks replayed as the stats kernel's
//           workgroups sum them: thread t of part p takes vector t of chunks p, p + 4, ...;
//           the same per-thread sums, wave butterflies and four-wave combine), keeping the
//           vectors of its own pixels in LDS as [channel][pixel] rows;
//  phase 2: wave 0 folds the chunk partials as fold_groups does, so the statistics are bit for
//           bit those of the two-kernel path, and the per-channel affine terms go to LDS;
//  phase 3: each thread forms `unit` consecutive channels of one pixel from the LDS rows
//           (normalised as group_norm_apply_nhwc_f16_kernel normalises, then the fp16 SiLU
//           evaluated on the narrowed value -- the values of silu_f16_table) and stores them
//           with one 4-, 8- or 16-byte store into y[b][p][g*gc ...]; raw (CAT) receives the
//           input channels-last the same way.
// Against stats + apply (two launches, a partials round trip through memory and a table
// gather per value) this takes one launch; the NSPLIT workgroups of a group run on one XCD and
// the XCD's workgroups take consecutive groups, so one L2 serves a group's repeated reads and
// each XCD writes whole runs of a pixel's channels.
template <typename P, int CPT, bool CAT>
__global__ __launch_bounds__(1024) void group_norm_nhwc_onepass_kernel(
    const GnSource<uint16_t> src, const P* __restrict__ gamma, const P* __restrict__ beta, uint16_t* __restrict__ y,
    uint16_t* __restrict__ raw, int C, int Cp, int groups, int HW, int group_size, int chunk, int splits, int nsplit,
    float eps, int fuse_silu, int unit, FastDiv div_hw, FastDiv div_units, int xcd_map) {
  constexpr int V = 8;
  constexpr int NPART = 4;
  constexpr int TILE = gn1_tile_halves(CPT);  // halves: this workgroup's [gc][px + 8] rows
  __shared__ __align__(16) uint16_t tile[TILE];
  __shared__ float red_s[NPART * CPT][4], red_ss[NPART * CPT][4];
  __shared__ float2 ch_s[256];  // per channel: (scale, shift) for fp16 parameters, (gamma, beta) for fp32
  __shared__ float2 st_s;
  const int n_wg = (int)gridDim.x;
  int w = (int)blockIdx.x;
  if (xcd_map) {
    // workgroup w runs on XCD w % 8: give each XCD a contiguous run of (group, part) pairs
    const int per = n_wg >> 3;
    w = (w & 7) * per + (w >> 3);
  }
  const int bg = w / nsplit, r = w - bg * nsplit;
  const int t = threadIdx.x & 255, part = threadIdx.x >> 8, wave = (threadIdx.x >> 6) & 3, lane = threadIdx.x & 63;
  const int gc = C / groups;
  const int px = HW / nsplit, p_lo = r * px;
  const int pitch = px + 8;  // halves per LDS channel row (16-byte multiple)
  const uint16_t* lo = src.x0 + (int64_t)bg * group_size;
  const uint16_t* hi = lo;
  int64_t cut64 = group_size;
  if constexpr (CAT) src.group(bg, lo, hi, cut64);
  const int cut = (int)cut64;
  // phase 1: all loads first (CPT vectors per thread in flight), then the sums
  uint4 d[CPT];
#pragma unroll
  for (int kk = 0; kk < CPT; ++kk) {
    const int k = NPART * kk + part;
    const int i = k * chunk + t * V;
    d[kk] = make_uint4(0u, 0u, 0u, 0u);
    if (k < splits && t * V < chunk && i < group_size) d[kk] = *reinterpret_cast<const uint4*>((i < cut ? lo : hi) + i);
  }
#pragma unroll
  for (int kk = 0; kk < CPT; ++kk) {
    const int k = NPART * kk + part;
    const int i = k * chunk + t * V;
    const bool have = k < splits && t * V < chunk && i < group_size;
    float s = 0.0f, ss = 0.0f;
    if (have) {
      // s += f, ss += f * f in element order, each add one v_fma_mix_f32 on the raw halves
      // (the same roundings: a half's square is exact in fp32)
      const uint32_t w[4] = {d[kk].x, d[kk].y, d[kk].z, d[kk].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s = acc_add_half<false>(s, w[j]);
        ss = acc_add_sq_half<false>(ss, w[j]);
        s = acc_add_half<true>(s, w[j]);
        ss = acc_add_sq_half<true>(ss, w[j]);
      }
      const int c = (int)div_hw.div((uint32_t)i), p = i - c * HW;
      if (p >= p_lo && p < p_lo + px) *reinterpret_cast<uint4*>(&tile[c * pitch + (p - p_lo)]) = d[kk];
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    if (lane == 0 && k < splits) {
      red_s[k][wave] = s;
      red_ss[k][wave] = ss;
    }
  }
  __syncthreads();
  // phase 2: the chunk partials folded as fold_groups folds them (splits <= 64: one per lane)
  if (threadIdx.x < 64) {
    float s = 0.0f, ss = 0.0f;
    if (lane < splits) {
      s += red_s[lane][0] + red_s[lane][1] + red_s[lane][2] + red_s[lane][3];
      ss += red_ss[lane][0] + red_ss[lane][1] + red_ss[lane][2] + red_ss[lane][3];
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    if (lane == 0) st_s = gn_stats(s, ss, (float)group_size, eps);
  }
  __syncthreads();
  const int g = bg % groups, b = bg / groups;
  if ((int)threadIdx.x < gc) {
    const int c = g * gc + (int)threadIdx.x;
    const float gm = gamma ? Elem<P>::load(gamma, c) : 1.0f;
    const float bt = beta ? Elem<P>::load(beta, c) : 0.0f;
    if constexpr (sizeof(P) == 2) {
      // gn_value's fp16-parameter form: scale = gamma*inv, shift = beta - mean*gamma*inv
      const float scale = gm * st_s.y;
      const float shift = bt - st_s.x * gm * st_s.y;
      ch_s[threadIdx.x] = make_float2(scale, shift);
    } else {
      ch_s[threadIdx.x] = make_float2(gm, bt);
    }
  }
  __syncthreads();
  const float mean = st_s.x, inv = st_s.y;
  // phase 3
  auto run = [&](auto unit_c, auto silu_c) {
    constexpr int U = decltype(unit_c)::value;
    constexpr bool SILU = decltype(silu_c)::value;
    const int upp = gc / U;  // store units per pixel
    const int n_units = px * upp;
    for (int q = threadIdx.x; q < n_units; q += 1024) {
      const int pl = (int)div_units.div((uint32_t)q), u = q - pl * upp;
      uint32_t hv[U], rv[U];
      float outs[U];
#pragma unroll
      for (int j = 0; j < U; ++j) {
        const int cl = u * U + j;
        const uint16_t h = tile[cl * pitch + pl];
        rv[j] = h;
        const float v = h2f_bits(h);
        const float2 cs = ch_s[cl];
        if constexpr (sizeof(P) == 2)
          outs[j] = v * cs.x + cs.y;
        else
          outs[j] = (v - mean) * inv * cs.x + cs.y;
      }
      // Pairs narrowed with f2h_rtz_* and the SiLU evaluated as silu_half evaluates it, under a
      // running maximum of |value| and silu_half's own test for its pinned inputs (0, |x| > 60,
      // inf, NaN): a wave in which some lane met one of those redoes the unit with f2h_fast and
      // silu_half.  Equal to them for every other input (tests/f2h_fast_model.c;
      // test_gpu_ops.py's exhaustive SiLU cases).
      float amax = 0.0f;
      bool rare = false;
#pragma unroll
      for (int j = 0; j < U; j += 2) {
        amax = abs_max_nan(abs_max_nan(amax, outs[j]), outs[j + 1]);
        const uint32_t hp = f2h_rtz_pack(outs[j], outs[j + 1]);
        if constexpr (SILU) {
#pragma clang fp contract(off)
          const auto hh = __builtin_bit_cast(_Float16 __attribute__((ext_vector_type(2))), hp);
          float r[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const float x = (float)hh[t];
            const float e = __builtin_amdgcn_exp2f(-x * 1.44269504088896341f);
            r[t] = x * __builtin_amdgcn_rcpf(1.0f + e);
          }
          amax = abs_max_nan(abs_max_nan(amax, r[0]), r[1]);
          const uint32_t sp = f2h_rtz_pack(r[0], r[1]);
          const uint32_t h0 = hp & 0xffffu, h1 = hp >> 16;
          hv[j] = h0 == 0xc173u ? 0xb15du : (sp & 0xffffu);
          hv[j + 1] = h1 == 0xc173u ? 0xb15du : (sp >> 16);
          rare |= (h0 & 0x7fffu) - 1u >= 0x5380u || (h1 & 0x7fffu) - 1u >= 0x5380u;
        } else {
          hv[j] = hp & 0xffffu;
          hv[j + 1] = hp >> 16;
        }
      }
      if (__builtin_amdgcn_ballot_w64(rare || !(amax < 65520.0f))) {
#pragma unroll
        for (int j = 0; j < U; ++j) {
          uint16_t o = f2h_fast(outs[j]);
          if constexpr (SILU) o = silu_half(o);
          hv[j] = o;
        }
      }
      const int64_t off = ((int64_t)b * HW + p_lo + pl) * Cp + g * gc + u * U;
      if constexpr (U == 2) {
        *reinterpret_cast<uint32_t*>(y + off) = hv[0] | (hv[1] << 16);
        if (CAT && raw) *reinterpret_cast<uint32_t*>(raw + off) = rv[0] | (rv[1] << 16);
      } else if constexpr (U == 4) {
        *reinterpret_cast<uint2*>(y + off) = make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
        if (CAT && raw) *reinterpret_cast<uint2*>(raw + off) = make_uint2(rv[0] | (rv[1] << 16), rv[2] | (rv[3] << 16));
      } else {
        *reinterpret_cast<uint4*>(y + off) = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16),
                                                       hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
        if (CAT && raw)
          *reinterpret_cast<uint4*>(raw + off) = make_uint4(rv[0] | (rv[1] << 16), rv[2] | (rv[3] << 16),
                                                           rv[4] | (rv[5] << 16), rv[6] | (rv[7] << 16));
      }
    }
  };
  if (unit == 8) {
    if (fuse_silu) run(std::integral_constant<int, 8>{}, std::true_type{});
    else run(std::integral_constant<int, 8>{}, std::false_type{});
  } else if (unit == 4) {
    if (fuse_silu) run(std::integral_constant<int, 4>{}, std::true_type{});
    else run(std::integral_constant<int, 4>{}, std::false_type{});
  } else {
    if (fuse_silu) run(std::integral_constant<int, 2>{}, std::true_type{});
    else run(std::integral_constant<int, 2>{}, std::false_type{});
  }
  // channels [C, Cp) of this workgroup's pixels are zero (written by the last group's workgroups)
  if (g == groups - 1 && Cp > C) {
    const int padc = Cp - C;
    for (int q = threadIdx.x; q < px * padc; q += 1024) {
      const int pl = q / padc, c = C + (q - pl * padc);
      const int64_t off = ((int64_t)b * HW + p_lo + pl) * Cp + c;
      y[off] = 0;
      if (CAT && raw) raw[off] = 0;
    }
  }
}

int gn_cu_count(int device) {
  static int cached[64] = {0};
  if (device < 0 || device >= 64) return 256;
  if (!cached[device]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n < 1) n = 256;
    cached[device] = n;
  }
  return cached[device];
}

bool gn_single_enabled() {
  const char* e = std::getenv("MTHIP_GN_SINGLE");
  return !(e && e[0] == '0');
}

// The one-launch channels-last GroupNorm (group_norm_nhwc_onepass_kernel) where it applies: fp16
// data with whole 16-byte vectors, an even channel count per group (<= 256), at most 60 stats
// chunks per group.  Returns -1 when it does not apply.  Workgroups per group: MTHIP_GN1_SPLIT,
// else 4, 2 or 1 -- the most that keep the grid within two workgroups per CU.  MTHIP_GN_ONEPASS=0
// turns it off (the two-kernel path then runs).
template <typename P>
int try_gn_onepass(int device, const GnSource<uint16_t>& src, const P* gamma, const P* beta, uint16_t* y,
                   uint16_t* raw, int64_t C, int64_t Cp, int64_t groups, int64_t HW, int64_t B, int64_t group_size,
                   int64_t chunk, int64_t splits, float eps, int fuse_silu, hipStream_t s) {
  if (const char* e = std::getenv("MTHIP_GN_ONEPASS"))
    if (e[0] == '0') return -1;
  const int64_t gc = C / groups;
  if (gc % 2 != 0 || gc > 256 || splits > 60 || chunk > 2048 || Cp % 8 != 0 || HW % 8 != 0) return -1;
  const int cpt = (int)ceil_div(splits, 4);
  const int cpt_inst = cpt <= 2 ? 2 : cpt <= 4 ? 4 : cpt <= 5 ? 5 : cpt <= 8 ? 8 : 15;
  const int tile_halves = gn1_tile_halves(cpt_inst);
  const int64_t n_groups = B * groups;
  const int cus = gn_cu_count(device);
  int nsplit = 1;
  for (int cand : {4, 2}) {
    if (n_groups * cand <= 2 * (int64_t)cus) {
      nsplit = cand;
      break;
    }
  }
  if (const char* e = std::getenv("MTHIP_GN1_SPLIT")) nsplit = std::max(1, std::atoi(e));
  while (nsplit > 1 && (HW % (8 * nsplit) != 0 || gc * (HW / nsplit + 8) > tile_halves)) nsplit /= 2;
  if (HW % (8 * nsplit) != 0 || gc * (HW / nsplit + 8) > tile_halves) return -1;
  const int64_t n_wg = n_groups * nsplit;
  if (n_wg > 2147483647) return -1;
  const int unit = gc % 8 == 0 ? 8 : gc % 4 == 0 ? 4 : 2;
  const int xcd_map = (n_wg % 8 == 0 && n_groups % 8 == 0) ? 1 : 0;
  const FastDiv div_hw((uint32_t)HW), div_units((uint32_t)(gc / unit));
  const bool cat = src.x1 != nullptr || raw != nullptr;
#define MTHIP_GN1(CPT, CATV)                                                                                     \
  hipLaunchKernelGGL((group_norm_nhwc_onepass_kernel<P, CPT, CATV>), dim3((unsigned)n_wg), dim3(1024), 0, s, src, \
                     gamma, beta, y, raw, (int)C, (int)Cp, (int)groups, (int)HW, (int)group_size, (int)chunk,   \
                     (int)splits, nsplit, eps, fuse_silu, unit, div_hw, div_units, xcd_map)
  if (cat) {
    if (cpt_inst == 2) MTHIP_GN1(2, true);
    else if (cpt_inst == 4) MTHIP_GN1(4, true);
    else if (cpt_inst == 5) MTHIP_GN1(5, true);
    else if (cpt_inst == 8) MTHIP_GN1(8, true);
    else MTHIP_GN1(15, true);
  } else {
    if (cpt_inst == 2) MTHIP_GN1(2, false);
    else if (cpt_inst == 4) MTHIP_GN1(4, false);
    else if (cpt_inst == 5) MTHIP_GN1(5, false);
    else if (cpt_inst == 8) MTHIP_GN1(8, false);
    else MTHIP_GN1(15, false);
  }
#undef MTHIP_GN1
  return check_launch("group_norm_nhwc_onepass_kernel");
}

// Stats (chunked partials), then the apply pass, which folds its group's partials: NCHW as x
// (y_nhwc == false) or channels-last with Cp channels.
// x1 (nullable): a second NCHW input of C - C0 channels concatenated after x's C0 channels
// (channels-last fp16 output only); raw (nullable, channels-last only) receives the input
// channels-last too.
// ws_given (nullable): caller-owned room for ws_capacity float2 partials, used instead of a
// block from the caching allocator (the no-allocation entry point passes its static scratch).
template <typename T, typename P>
int run_group_norm(int device, const void* x, const void* weight, const void* bias, void* y, int64_t B, int64_t C,
                   int64_t inner, int64_t groups, double eps, int fuse_silu, bool y_nhwc, int64_t Cp, hipStream_t s,
                   const void* x1 = nullptr, int64_t C0 = -1, void* raw = nullptr, float2* ws_given = nullptr,
                   int64_t ws_capacity = 0) {
  const int64_t group_size = (C / groups) * inner;
  if (C0 < 0) C0 = C;
  const GnSource<T> src{(const T*)x, (const T*)x1, C0, C - C0, C / groups, inner, groups};
  const int64_t n_groups = B * groups;
  if (n_groups == 0 || group_size == 0) return MTHIP_OK;
  MTHIP_REQUIRE(n_groups <= 65535, "mthip_group_norm: batch*groups must be <= 65535");
  // channel and in-group indices are divided in 32-bit arithmetic
  MTHIP_REQUIRE(group_size < (int64_t(1) << 31) && C < (int64_t(1) << 31) && inner < (int64_t(1) << 31),
                "mthip_group_norm: a group, the channel count and the spatial size must stay below 2^31 elements");
  constexpr int V = Vec16<T>::N;
  const bool vect = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) && inner % V == 0 &&
                    ((uintptr_t)x1 % 16 == 0);
  // Stats chunks of >= 2048 elements (4-8 KB per workgroup; the SD tensors give >= 4
  // workgroups per CU, all loads in flight at once), at most 64 per group: the apply kernels
  // fold a group's partials themselves.
  int64_t splits = std::max<int64_t>(1, std::min<int64_t>(ceil_div(group_size, 2048), 64));
  int64_t chunk = ceil_div(group_size, splits);
  if (vect) chunk = ceil_div(chunk, V) * V;
  splits = ceil_div(group_size, chunk);
  // Many (sample, group) pairs, NCHW in and out: one pass over x (group_norm_single_kernel),
  // bit-identical to the two kernels below and without their partials buffer.  MTHIP_GN_SINGLE=0
  // turns it off.
  if (!y_nhwc && vect && !x1 && !raw && n_groups >= 2 * (int64_t)gn_cu_count(device) && gn_single_enabled()) {
    // (up to 20 chunks, five per thread, e.g. a 10-channel 64x64 group; a chunk is one vector
    // per thread in fp16, two in fp32)
    constexpr int IPC = sizeof(T) == 2 ? 1 : 2;
    if (chunk == (int64_t)IPC * 256 * V && splits <= 20) {
      const int cpt = (int)ceil_div(splits, 4);
#define MTHIP_GN_SINGLE(CPT)                                                                                       \
  hipLaunchKernelGGL((group_norm_single_kernel<T, P, CPT, IPC>), dim3((unsigned)n_groups), dim3(1024), 0, s,      \
                     (const T*)x, (const P*)weight, (const P*)bias, (T*)y, C, groups, inner, group_size, chunk,  \
                     (int)splits, (float)eps, fuse_silu, FastDiv((uint32_t)inner))
      if (cpt <= 2)
        MTHIP_GN_SINGLE(2);
      else if (cpt <= 4)
        MTHIP_GN_SINGLE(4);
      else
        MTHIP_GN_SINGLE(5);
#undef MTHIP_GN_SINGLE
      return check_launch("group_norm_single_kernel");
    }
  }
  // The fp16 channels-last apply (the only one that reads two sources or writes `raw`).
  const bool nhwc_f16 = y_nhwc && sizeof(T) == 2 && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) &&
                        inner % V == 0 && Cp % V == 0 && ((uintptr_t)x1 % 16 == 0) && ((uintptr_t)raw % 16 == 0) &&
                        C0 % 2 == 0;
  if ((x1 || raw) && !nhwc_f16)
    return fail(MTHIP_ERR_UNSUPPORTED, "mthip_group_norm_nhwc_cat: needs fp16, 16-byte aligned rows and an even split");
  if constexpr (sizeof(T) == 2) {
    if (nhwc_f16) {
      const GnSource<uint16_t> src16{(const uint16_t*)x, (const uint16_t*)x1, C0, C - C0, C / groups, inner, groups};
      const int rc = try_gn_onepass<P>(device, src16, (const P*)weight, (const P*)bias, (uint16_t*)y, (uint16_t*)raw, C,
                                       Cp, groups, inner, B, group_size, chunk, splits, (float)eps, fuse_silu, s);
      if (rc >= 0) return rc;
    }
  }
  // The two-kernel path's per-chunk partial sums: a caching-allocator block, or the caller's scratch.
  void* ws = nullptr;
  float2* partial = ws_given;
  if (ws_given) {
    if (n_groups * splits > ws_capacity)
      return fail(MTHIP_ERR_UNSUPPORTED, "mthip_group_norm_noalloc: batch*groups*chunks = " +
                                             std::to_string(n_groups * splits) + " partial sums exceed the scratch of " +
                                             std::to_string(ws_capacity));
  } else {
    if (int rc = mthip_malloc(device, (size_t)(n_groups * splits) * sizeof(float2), &ws)) return rc;
    partial = static_cast<float2*>(ws);
  }
  dim3 grid((unsigned)splits, (unsigned)n_groups);
  const bool cat = x1 != nullptr;
  if (vect && cat)
    hipLaunchKernelGGL((group_norm_stats_kernel<T, true, true>), grid, dim3(256), 0, s, src, partial, group_size, chunk,
                       (int)splits);
  else if (vect)
    hipLaunchKernelGGL((group_norm_stats_kernel<T, true, false>), grid, dim3(256), 0, s, src, partial, group_size,
                       chunk, (int)splits);
  else
    hipLaunchKernelGGL((group_norm_stats_kernel<T, false, false>), grid, dim3(256), 0, s, src, partial, group_size,
                       chunk, (int)splits);
  int rc = check_launch("group_norm_stats_kernel");
  // The fp16 channels-last apply looks the fused SiLU up in a table (built on first use).
  const uint16_t* silu_tab = nullptr;
  if (rc == MTHIP_OK && nhwc_f16 && fuse_silu) {
    silu_tab = silu_f16_table(device, s);
    if (!silu_tab) rc = fail(MTHIP_ERR_HIP, "mthip_group_norm: silu table setup failed");
  }
  if (rc == MTHIP_OK) {
    if (y_nhwc) {
      dim3 g2((unsigned)ceil_div(inner, 64), (unsigned)ceil_div(Cp, 64), (unsigned)B);
      // 16-byte row access: pixel rows and channel rows start on 16-byte boundaries.
      const int vec_io = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) && inner % V == 0 && Cp % V == 0;
      const GnSource<uint16_t> src16{(const uint16_t*)x, (const uint16_t*)x1, C0, C - C0, C / groups, inner, groups};
      // 32-pixel tiles (128-thread workgroups) where 64-pixel tiles would leave fewer than two
      // workgroups per CU (the 32x32, 16x16 and 8x8 latents); MTHIP_GN_TPX=32/64 forces one
      int tpx = (int64_t)g2.x * g2.y * g2.z < 2 * (int64_t)gn_cu_count(device) ? 32 : 64;
      if (const char* f = std::getenv("MTHIP_GN_TPX")) tpx = std::atoi(f) == 32 ? 32 : 64;
      const dim3 g32((unsigned)ceil_div(inner, 32), g2.y, g2.z);
      if (nhwc_f16 && (cat || raw)) {
        if (tpx == 32)
          hipLaunchKernelGGL((group_norm_apply_nhwc_f16_kernel<P, true, 32>), g32, dim3(128), 0, s, src16,
                             (const P*)weight, (const P*)bias, (uint16_t*)y, (uint16_t*)raw, (const float2*)partial, C,
                             Cp, groups, inner, (int)splits, (float)eps, silu_tab);
        else
          hipLaunchKernelGGL((group_norm_apply_nhwc_f16_kernel<P, true>), g2, dim3(256), 0, s, src16, (const P*)weight,
                             (const P*)bias, (uint16_t*)y, (uint16_t*)raw, (const float2*)partial, C, Cp, groups,
                             inner, (int)splits, (float)eps, silu_tab);
      } else if (nhwc_f16) {
        if (tpx == 32)
          hipLaunchKernelGGL((group_norm_apply_nhwc_f16_kernel<P, false, 32>), g32, dim3(128), 0, s, src16,
                             (const P*)weight, (const P*)bias, (uint16_t*)y, (uint16_t*)nullptr,
                             (const float2*)partial, C, Cp, groups, inner, (int)splits, (float)eps, silu_tab);
        else
          hipLaunchKernelGGL((group_norm_apply_nhwc_f16_kernel<P, false>), g2, dim3(256), 0, s, src16, (const P*)weight,
                             (const P*)bias, (uint16_t*)y, (uint16_t*)nullptr, (const float2*)partial, C, Cp, groups,
                             inner, (int)splits, (float)eps, silu_tab);
      } else
        hipLaunchKernelGGL((group_norm_apply_nhwc_kernel<T, P>), g2, dim3(256), 0, s, (const T*)x, (const P*)weight,
                           (const P*)bias, (T*)y, (const float2*)partial, C, Cp, groups, inner, (int)splits,
                           (float)eps, fuse_silu, vec_io);
    } else if (vect) {
      hipLaunchKernelGGL((group_norm_apply_kernel<T, P, true>), grid, dim3(256), 0, s, (const T*)x, (const P*)weight,
                         (const P*)bias, (T*)y, (const float2*)partial, C, groups, inner, group_size, chunk,
                         (int)splits, (float)eps, fuse_silu);
    } else {
      hipLaunchKernelGGL((group_norm_apply_kernel<T, P, false>), grid, dim3(256), 0, s, (const T*)x, (const P*)weight,
                         (const P*)bias, (T*)y, (const float2*)partial, C, groups, inner, group_size, chunk,
                         (int)splits, (float)eps, fuse_silu);
    }
    rc = check_launch("group_norm_apply_kernel");
  }
  mthip_free(device, ws);
  return rc;
}

template <typename T, typename P>
int run_layer_norm(const void* x, const void* w, const void* b, void* y, int64_t rows, int64_t N, double eps,
                   hipStream_t s) {
  if (rows == 0 || N == 0) return MTHIP_OK;
  const unsigned grid4 = (unsigned)ceil_div(rows, 4);
  const float e = (float)eps;
  const T* xp = (const T*)x;
  const P* wp = (const P*)w;
  const P* bp = (const P*)b;
  T* yp = (T*)y;
  constexpr int V = Vec16<T>::N;
  const bool params_aligned = (uintptr_t)w % 16 == 0 && (uintptr_t)b % 16 == 0;
  if (N % V == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 && params_aligned && N <= 64 * V * 4) {
    const int64_t chunks = N / V;
    // two rows per wave once there are enough rows to keep >= 4 waves per SIMD
    const bool two = rows >= 8192;
    const unsigned g = (unsigned)ceil_div(rows, two ? 8 : 4);
#define MTHIP_LN_VEC(CPL)                                                                                           \
  do {                                                                                                             \
    if (two)                                                                                                       \
      hipLaunchKernelGGL((layer_norm_vec_kernel<T, P, CPL, 2>), dim3(g), dim3(256), 0, s, xp, wp, bp, yp, rows, N, e); \
    else                                                                                                           \
      hipLaunchKernelGGL((layer_norm_vec_kernel<T, P, CPL, 1>), dim3(g), dim3(256), 0, s, xp, wp, bp, yp, rows, N, e); \
  } while (0)
    if (chunks <= 64)
      MTHIP_LN_VEC(1);
    else if (chunks <= 128)
      MTHIP_LN_VEC(2);
    else if (chunks <= 192)
      MTHIP_LN_VEC(3);
    else
      MTHIP_LN_VEC(4);
#undef MTHIP_LN_VEC
    return check_launch("layer_norm_vec_kernel");
  }
  if (N <= 64 * 4)
    hipLaunchKernelGGL((layer_norm_kernel<T, P, 4>), dim3(grid4), dim3(256), 0, s, xp, wp, bp, yp, rows, N, e);
  else if (N <= 64 * 12)
    hipLaunchKernelGGL((layer_norm_kernel<T, P, 12>), dim3(grid4), dim3(256), 0, s, xp, wp, bp, yp, rows, N, e);
  else if (N <= 64 * 20)
    hipLaunchKernelGGL((layer_norm_kernel<T, P, 20>), dim3(grid4), dim3(256), 0, s, xp, wp, bp, yp, rows, N, e);
  else if (N <= 64 * 32)
    hipLaunchKernelGGL((layer_norm_kernel<T, P, 32>), dim3(grid4), dim3(256), 0, s, xp, wp, bp, yp, rows, N, e);
  else
    hipLaunchKernelGGL((layer_norm_long_kernel<T, P>), dim3((unsigned)rows), dim3(256), 0, s, xp, wp, bp, yp, N, e);
  return check_launch("layer_norm_kernel");
}

template <typename T>
int run_softmax(const void* x, void* y, int64_t rows, int64_t cols, int divide, hipStream_t s) {
  if (rows == 0 || cols == 0) return MTHIP_OK;
  const unsigned grid4 = (unsigned)ceil_div(rows, 4);
  constexpr int V = Vec16<T>::N;
  const int64_t chunks = cols / V;
  if (cols % V == 0 && (((uintptr_t)x | (uintptr_t)y) & 15) == 0 && chunks <= 64 * 8) {
    if (chunks <= 64)
      hipLaunchKernelGGL((softmax_vec_kernel<T, 1>), dim3(grid4), dim3(256), 0, s, (const T*)x, (T*)y, rows, cols, divide);
    else if (chunks <= 128)
      hipLaunchKernelGGL((softmax_vec_kernel<T, 2>), dim3(grid4), dim3(256), 0, s, (const T*)x, (T*)y, rows, cols, divide);
    else if (chunks <= 256)
      hipLaunchKernelGGL((softmax_vec_kernel<T, 4>), dim3(grid4), dim3(256), 0, s, (const T*)x, (T*)y, rows, cols, divide);
    else
      hipLaunchKernelGGL((softmax_vec_kernel<T, 8>), dim3(grid4), dim3(256), 0, s, (const T*)x, (T*)y, rows, cols, divide);
  } else if (cols <= 64 * 4)
    hipLaunchKernelGGL((softmax_kernel<T, 4>), dim3(grid4), dim3(256), 0, s, (const T*)x, (T*)y, rows, cols, divide);
  else if (cols <= 64 * 16)
    hipLaunchKernelGGL((softmax_kernel<T, 16>), dim3(grid4), dim3(256), 0, s, (const T*)x, (T*)y, rows, cols, divide);
  else if (cols <= 64 * 64)
    hipLaunchKernelGGL((softmax_kernel<T, 64>), dim3(grid4), dim3(256), 0, s, (const T*)x, (T*)y, rows, cols, divide);
  else
    hipLaunchKernelGGL(softmax_long_kernel<T>, dim3((unsigned)rows), dim3(256), 0, s, (const T*)x, (T*)y, cols, divide);
  return check_launch("softmax_kernel");
}

}  // namespace

const uint16_t* silu_f16_lookup(int device, hipStream_t s) { return silu_f16_table(device, s); }

}  // namespace mthip

using namespace mthip;

extern "C" {

// Data / parameter dtype pairs: (F16, F16), (F32, F32) and (F16, F32) -- the last one is the
// upcast pattern norm(x.float(), w32, b32).half().
static bool norm_dtypes_ok(int dtype, int param_dtype) {
  return (dtype == MTHIP_F16 || dtype == MTHIP_F32) && (param_dtype == dtype || (dtype == MTHIP_F16 && param_dtype == MTHIP_F32));
}

int mthip_group_norm(int device, int dtype, const void* x, const void* weight, const void* bias, void* y, int64_t B,
                     int64_t C, int64_t inner, int64_t groups, double eps, int fuse_silu, int param_dtype) {
  MTHIP_REQUIRE(norm_dtypes_ok(dtype, param_dtype), "mthip_group_norm: unsupported dtype / param_dtype pair");
  MTHIP_REQUIRE(groups > 0 && C % groups == 0, "mthip_group_norm: num_channels must be divisible by num_groups");
  MTHIP_REQUIRE(B >= 0 && inner >= 0, "mthip_group_norm: negative extent");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F32)
    return run_group_norm<float, float>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, false, C, s);
  if (param_dtype == MTHIP_F32)
    return run_group_norm<uint16_t, float>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, false, C, s);
  return run_group_norm<uint16_t, uint16_t>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, false, C, s);
}

// ---- the no-allocation entry point.  The statistics partials live in one file-scope device
// array per GPU (each GPU that loads the library holds its own copy for the life of the
// process); host code reaches it only through the per-device address hipGetSymbolAddress
// returns.  Every (group, chunk) partial is written by the statistics pass before the apply pass
// reads it, so nothing has to start at zero; concurrent calls on one GPU from different streams
// or threads share the array and race.
constexpr int64_t kGnScratchPartials = 131072;  // 1 MiB of float2
static __device__ __align__(256) float2 scratch[kGnScratchPartials];

static float2* gn_scratch_ptr(int device) {
  static float2* ptrs[64] = {nullptr};
  static std::mutex m;
  if (device < 0 || device >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(m);
  if (!ptrs[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
      set_error(std::string("mthip_group_norm_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
      return nullptr;
    }
    ptrs[device] = static_cast<float2*>(p);
  }
  return ptrs[device];
}

int mthip_group_norm_noalloc(int device, int dtype, const void* x, const void* weight, const void* bias, void* y,
                             int64_t B, int64_t C, int64_t inner, int64_t groups, double eps, int fuse_silu,
                             int param_dtype) {
  MTHIP_REQUIRE(norm_dtypes_ok(dtype, param_dtype), "mthip_group_norm_noalloc: unsupported dtype / param_dtype pair");
  MTHIP_REQUIRE(groups > 0 && C % groups == 0, "mthip_group_norm_noalloc: num_channels must be divisible by num_groups");
  MTHIP_REQUIRE(B >= 0 && inner >= 0, "mthip_group_norm_noalloc: negative extent");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;  // the symbol address below is the current device's
  float2* ws = gn_scratch_ptr(device);
  if (!ws) return MTHIP_ERR_HIP;
  if (dtype == MTHIP_F32)
    return run_group_norm<float, float>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, false, C, s,
                                        nullptr, -1, nullptr, ws, kGnScratchPartials);
  if (param_dtype == MTHIP_F32)
    return run_group_norm<uint16_t, float>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, false, C,
                                           s, nullptr, -1, nullptr, ws, kGnScratchPartials);
  return run_group_norm<uint16_t, uint16_t>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, false, C,
                                            s, nullptr, -1, nullptr, ws, kGnScratchPartials);
}

int mthip_group_norm_nhwc(int device, int dtype, const void* x, const void* weight, const void* bias, void* y_nhwc,
                          int64_t B, int64_t C, int64_t HW, int64_t groups, double eps, int fuse_silu,
                          int param_dtype) {
  MTHIP_REQUIRE(norm_dtypes_ok(dtype, param_dtype), "mthip_group_norm_nhwc: unsupported dtype / param_dtype pair");
  MTHIP_REQUIRE(groups > 0 && C % groups == 0, "mthip_group_norm_nhwc: num_channels must be divisible by num_groups");
  MTHIP_REQUIRE(B >= 0 && HW >= 0 && B <= 65535, "mthip_group_norm_nhwc: bad extents");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  const int64_t vec = dtype == MTHIP_F16 ? 8 : 4;
  const int64_t Cp = ceil_div(C, vec) * vec;
  if (dtype == MTHIP_F32)
    return run_group_norm<float, float>(device, x, weight, bias, y_nhwc, B, C, HW, groups, eps, fuse_silu, true, Cp, s);
  if (param_dtype == MTHIP_F32)
    return run_group_norm<uint16_t, float>(device, x, weight, bias, y_nhwc, B, C, HW, groups, eps, fuse_silu, true, Cp, s);
  return run_group_norm<uint16_t, uint16_t>(device, x, weight, bias, y_nhwc, B, C, HW, groups, eps, fuse_silu, true, Cp,
                                            s);
}

int mthip_group_norm_nhwc_cat(int device, int dtype, const void* x0, int64_t C0, const void* x1, int64_t C1,
                              const void* weight, const void* bias, void* y_nhwc, void* raw_nhwc, int64_t B,
                              int64_t HW, int64_t groups, double eps, int fuse_silu, int param_dtype) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 && norm_dtypes_ok(dtype, param_dtype),
                "mthip_group_norm_nhwc_cat: data must be F16 (parameters F16 or F32)");
  const int64_t C = C0 + C1;
  MTHIP_REQUIRE(C0 >= 0 && C1 >= 0 && groups > 0 && C % groups == 0,
                "mthip_group_norm_nhwc_cat: num_channels must be divisible by num_groups");
  MTHIP_REQUIRE(C1 == 0 || x1 != nullptr, "mthip_group_norm_nhwc_cat: second input missing");
  MTHIP_REQUIRE(B >= 0 && HW >= 0 && B <= 65535, "mthip_group_norm_nhwc_cat: bad extents");
  MTHIP_REQUIRE(C % 8 == 0 && C0 % 2 == 0 && HW % 8 == 0,
                "mthip_group_norm_nhwc_cat: channel counts and HW must allow 16-byte rows");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  const void* second = C1 > 0 ? x1 : nullptr;
  if (param_dtype == MTHIP_F32)
    return run_group_norm<uint16_t, float>(device, x0, weight, bias, y_nhwc, B, C, HW, groups, eps, fuse_silu, true, C,
                                           s, second, C0, raw_nhwc);
  return run_group_norm<uint16_t, uint16_t>(device, x0, weight, bias, y_nhwc, B, C, HW, groups, eps, fuse_silu, true,
                                            C, s, second, C0, raw_nhwc);
}

int mthip_layer_norm(int device, int dtype, const void* x, const void* weight, const void* bias, void* y, int64_t rows,
                     int64_t N, double eps, int param_dtype) {
  MTHIP_REQUIRE(norm_dtypes_ok(dtype, param_dtype), "mthip_layer_norm: unsupported dtype / param_dtype pair");
  MTHIP_REQUIRE(rows >= 0 && N >= 0, "mthip_layer_norm: negative extent");
  MTHIP_REQUIRE(rows <= 0x7fffffffLL * 4, "mthip_layer_norm: too many rows");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F32) return run_layer_norm<float, float>(x, weight, bias, y, rows, N, eps, s);
  if (param_dtype == MTHIP_F32) return run_layer_norm<uint16_t, float>(x, weight, bias, y, rows, N, eps, s);
  return run_layer_norm<uint16_t, uint16_t>(x, weight, bias, y, rows, N, eps, s);
}

int mthip_softmax_lastdim(int device, int dtype, const void* x, void* y, int64_t rows, int64_t cols, int divide) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_softmax_lastdim: dtype must be F16 or F32");
  MTHIP_REQUIRE(rows >= 0 && cols >= 0, "mthip_softmax_lastdim: negative extent");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16) return run_softmax<uint16_t>(x, y, rows, cols, divide, s);
  return run_softmax<float>(x, y, rows, cols, divide, s);
}

}  // extern "C"
