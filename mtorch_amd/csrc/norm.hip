// group_norm (+ fused SiLU), layer_norm and last-dim softmax: HBM-streaming kernels with
// wave64 shuffle reductions.
//
// group_norm splits every (sample, group) range into chunks so that thousands of workgroups
// stream at once (an SD group is 40,960 elements but there are only B*32 groups): a stats pass
// writes per-chunk (sum, sum of squares), and an apply pass folds the chunk partials of its
// group and normalises its own chunk (its re-read of the input is served mostly by the 256 MB
// last-level cache).  Statistics follow the reference's one-pass E[x^2] - mean^2 form
// (tensor.cpp:18765-18767, 18822-18824) with fp32 tree sums.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "activations.h"
#include "common.h"

namespace mthip {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
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
template <typename T>
__global__ __launch_bounds__(256) void group_norm_stats_kernel(const T* __restrict__ x, float2* __restrict__ partial,
                                                               int64_t group_size, int64_t chunk, int splits) {
  __shared__ float red[8];
  const int64_t bg = blockIdx.y;
  const int split = blockIdx.x;
  const int64_t begin = (int64_t)split * chunk;
  const int64_t end = min(begin + chunk, group_size);
  const T* base = x + bg * group_size;
  float s = 0.0f, ss = 0.0f;
  for (int64_t i = begin + threadIdx.x; i < end; i += 256) {
    const float v = Elem<T>::load(base, i);
    s += v;
    ss += v * v;
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

template <typename T>
__global__ __launch_bounds__(256) void group_norm_apply_kernel(const T* __restrict__ x, const T* __restrict__ gamma,
                                                               const T* __restrict__ beta, T* __restrict__ y,
                                                               const float2* __restrict__ partial, int64_t C,
                                                               int64_t groups, int64_t inner, int64_t group_size,
                                                               int64_t chunk, int splits, float eps, int fuse_silu) {
  __shared__ float stats[2];
  const int64_t bg = blockIdx.y;
  const int split = blockIdx.x;
  if (threadIdx.x < 64) {
    float s = 0.0f, ss = 0.0f;
    for (int i = threadIdx.x; i < splits; i += 64) {
      const float2 p = partial[bg * splits + i];
      s += p.x;
      ss += p.y;
    }
    s = wave_sum(s);
    ss = wave_sum(ss);
    if (threadIdx.x == 0) {
      const float n = (float)group_size;
      const float mean = s / n;
      const float var = fmaxf(0.0f, ss / n - mean * mean);
      stats[0] = mean;
      stats[1] = 1.0f / sqrtf(var + eps);
    }
  }
  __syncthreads();
  const float mean = stats[0], inv = stats[1];
  const int64_t g = bg % groups;
  const int64_t gc = C / groups;
  const int64_t begin = (int64_t)split * chunk;
  const int64_t end = min(begin + chunk, group_size);
  const T* xb = x + bg * group_size;
  T* yb = y + bg * group_size;
  for (int64_t i = begin + threadIdx.x; i < end; i += 256) {
    const int64_t c = g * gc + i / inner;
    const float gm = gamma ? Elem<T>::load(gamma, c) : 1.0f;
    const float bt = beta ? Elem<T>::load(beta, c) : 0.0f;
    const float v = Elem<T>::load(xb, i);
    float out;
    if constexpr (sizeof(T) == 2) {
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
    Elem<T>::store(yb, i, out);
  }
}

// ------------------------------------------------------------------------------ layer_norm
// One wave per row; the row lives in registers (up to 64*MAXV elements).
template <typename T, int MAXV>
__global__ __launch_bounds__(256) void layer_norm_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                         const T* __restrict__ b, T* __restrict__ y, int64_t rows,
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
  if constexpr (sizeof(T) == 2) {
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
      if (w) o = o * Elem<T>::load(w, i);
      if (b) o = o + Elem<T>::load(b, i);
      Elem<T>::store(yr, i, o);
    }
  }
}

// Rows too long for registers: one workgroup per row, three passes over the row.
template <typename T>
__global__ __launch_bounds__(256) void layer_norm_long_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                              const T* __restrict__ b, T* __restrict__ y, int64_t N,
                                                              float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * N;
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < N; i += 256) s += Elem<T>::load(xr, i);
  const float n = (float)N;
  const float mean = block_sum256(s, red) / n;
  float var;
  if constexpr (sizeof(T) == 2) {
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
    if (w) o = o * Elem<T>::load(w, i);
    if (b) o = o + Elem<T>::load(b, i);
    Elem<T>::store(yr, i, o);
  }
}

// ------------------------------------------------------------------------------ softmax
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
    v[j] = i < cols ? expf(v[j] - mx) : 0.0f;
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
  for (int64_t i = threadIdx.x; i < cols; i += 256) s += expf(Elem<T>::load(xr, i) - mx);
  s = block_sum256(s, red);
  const float inv = 1.0f / s;
  T* yr = y + row * cols;
  for (int64_t i = threadIdx.x; i < cols; i += 256) {
    const float e = expf(Elem<T>::load(xr, i) - mx);
    Elem<T>::store(yr, i, divide ? e / s : e * inv);
  }
}

template <typename T>
int run_group_norm(int device, const void* x, const void* weight, const void* bias, void* y, int64_t B, int64_t C,
                   int64_t inner, int64_t groups, double eps, int fuse_silu, hipStream_t s) {
  const int64_t group_size = (C / groups) * inner;
  const int64_t n_groups = B * groups;
  if (n_groups == 0 || group_size == 0) return MTHIP_OK;
  MTHIP_REQUIRE(n_groups <= 65535, "mthip_group_norm: batch*groups must be <= 65535");
  // Aim for ~4096 workgroups in total, each streaming at least 2048 elements.
  int64_t splits = std::max<int64_t>(1, std::min<int64_t>(ceil_div(4096, n_groups), ceil_div(group_size, 2048)));
  splits = std::min<int64_t>(splits, 1024);
  const int64_t chunk = ceil_div(group_size, splits);
  splits = ceil_div(group_size, chunk);
  void* partial = nullptr;
  if (int rc = mthip_malloc(device, (size_t)(n_groups * splits) * sizeof(float2), &partial)) return rc;
  dim3 grid((unsigned)splits, (unsigned)n_groups);
  hipLaunchKernelGGL(group_norm_stats_kernel<T>, grid, dim3(256), 0, s, (const T*)x, (float2*)partial, group_size,
                     chunk, (int)splits);
  int rc = check_launch("group_norm_stats_kernel");
  if (rc == MTHIP_OK) {
    hipLaunchKernelGGL(group_norm_apply_kernel<T>, grid, dim3(256), 0, s, (const T*)x, (const T*)weight,
                       (const T*)bias, (T*)y, (const float2*)partial, C, groups, inner, group_size, chunk, (int)splits,
                       (float)eps, fuse_silu);
    rc = check_launch("group_norm_apply_kernel");
  }
  mthip_free(device, partial);
  return rc;
}

template <typename T>
int run_layer_norm(const void* x, const void* w, const void* b, void* y, int64_t rows, int64_t N, double eps,
                   hipStream_t s) {
  if (rows == 0 || N == 0) return MTHIP_OK;
  const unsigned grid4 = (unsigned)ceil_div(rows, 4);
  const float e = (float)eps;
  if (N <= 64 * 4)
    hipLaunchKernelGGL((layer_norm_kernel<T, 4>), dim3(grid4), dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b, (T*)y, rows, N, e);
  else if (N <= 64 * 12)
    hipLaunchKernelGGL((layer_norm_kernel<T, 12>), dim3(grid4), dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b, (T*)y, rows, N, e);
  else if (N <= 64 * 20)
    hipLaunchKernelGGL((layer_norm_kernel<T, 20>), dim3(grid4), dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b, (T*)y, rows, N, e);
  else if (N <= 64 * 32)
    hipLaunchKernelGGL((layer_norm_kernel<T, 32>), dim3(grid4), dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b, (T*)y, rows, N, e);
  else
    hipLaunchKernelGGL(layer_norm_long_kernel<T>, dim3((unsigned)rows), dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b, (T*)y, N, e);
  return check_launch("layer_norm_kernel");
}

template <typename T>
int run_softmax(const void* x, void* y, int64_t rows, int64_t cols, int divide, hipStream_t s) {
  if (rows == 0 || cols == 0) return MTHIP_OK;
  const unsigned grid4 = (unsigned)ceil_div(rows, 4);
  if (cols <= 64 * 4)
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
}  // namespace mthip

using namespace mthip;

extern "C" {

int mthip_group_norm(int device, int dtype, const void* x, const void* weight, const void* bias, void* y, int64_t B,
                     int64_t C, int64_t inner, int64_t groups, double eps, int fuse_silu) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_group_norm: dtype must be F16 or F32");
  MTHIP_REQUIRE(groups > 0 && C % groups == 0, "mthip_group_norm: num_channels must be divisible by num_groups");
  MTHIP_REQUIRE(B >= 0 && inner >= 0, "mthip_group_norm: negative extent");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16) return run_group_norm<uint16_t>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, s);
  return run_group_norm<float>(device, x, weight, bias, y, B, C, inner, groups, eps, fuse_silu, s);
}

int mthip_layer_norm(int device, int dtype, const void* x, const void* weight, const void* bias, void* y, int64_t rows,
                     int64_t N, double eps) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_layer_norm: dtype must be F16 or F32");
  MTHIP_REQUIRE(rows >= 0 && N >= 0, "mthip_layer_norm: negative extent");
  MTHIP_REQUIRE(rows <= 0x7fffffffLL * 4, "mthip_layer_norm: too many rows");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16) return run_layer_norm<uint16_t>(x, weight, bias, y, rows, N, eps, s);
  return run_layer_norm<float>(x, weight, bias, y, rows, N, eps, s);
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
