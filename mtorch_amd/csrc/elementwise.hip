// HBM-streaming elementwise kernels: casts, fills, strided copies, broadcast binary ops,
// activations, GEGLU gating, concatenation and nearest upsampling.
//
// Contiguous inputs run through grid-stride loops that move 16 bytes per lane per step;
// strided and broadcast inputs go through a rank-collapsed index walk.  Every narrowing to
// fp16 follows mtorch's half-away-from-zero rule (f2h_bits, or its branch-free equivalent
// f2h_fast in the vectorised paths).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "activations.h"
#include "common.h"

namespace mthip {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxRank = 8;

// Enough workgroups to cover every CU several times over; grid-stride loops do the rest.
inline unsigned grid_for(int64_t work_items, int per_thread = 1) {
  int64_t blocks = ceil_div(std::max<int64_t>(work_items, 1), (int64_t)kThreads * per_thread);
  return (unsigned)std::min<int64_t>(blocks, 256 * 32);
}

// Streaming kernels (same-shape elementwise ops over 16-byte chunks): U chunks per thread in
// flight and at most two 256-thread workgroups per CU -- the shape at which a plain copy of a
// 640 MB read+write stream ran fastest on MI355X (6.1 TB/s with non-temporal accesses, 5.8
// without; four or more workgroups per CU, or one chunk per thread, stayed at 4.6-5.4 TB/s).
// Buffers above kStreamNTBytes are read and written non-temporally (not kept in the caches):
// their data would not fit the caches anyway, while the smaller intermediates of a model step
// are read back by the next kernel from L2 or the Infinity Cache.
constexpr int kStreamU = 4;
constexpr int64_t kStreamNTBytes = int64_t(64) << 20;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 ld16(const uint4* p) {
  if constexpr (NT) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *p;
  }
}

template <bool NT>
__device__ __forceinline__ void st16(uint4* p, const uint4 v) {
  if constexpr (NT) {
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
  } else {
    *p = v;
  }
}

int cu_count_dev(int device) {
  static int cached[64] = {0};
  if (device < 0 || device >= 64) return 256;
  if (cached[device] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n < 1) n = 256;
    cached[device] = n;
  }
  return cached[device];
}

inline unsigned stream_grid(int device, int64_t nvec) {
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(nvec, (int64_t)kThreads * kStreamU),
                                                          2 * (int64_t)cu_count_dev(device)));
}

struct Shape {
  int rank;
  int64_t sizes[kMaxRank];
  int64_t a_strides[kMaxRank];
  int64_t b_strides[kMaxRank];
};

// Merge adjacent dims whose strides are contiguous with respect to each other in every
// operand, and drop size-1 dims.  Returns the collapsed rank (0 means a single element).
int collapse(int rank, const int64_t* sizes, const int64_t* const* strides, int n_ops,
             int64_t* out_sizes, int64_t* const* out_strides) {
  int r = 0;
  for (int d = 0; d < rank; ++d) {
    if (sizes[d] == 1) continue;
    if (r > 0) {
      bool merge = true;
      for (int o = 0; o < n_ops; ++o) {
        if (out_strides[o][r - 1] != strides[o][d] * sizes[d]) merge = false;
      }
      if (merge) {
        out_sizes[r - 1] *= sizes[d];
        for (int o = 0; o < n_ops; ++o) out_strides[o][r - 1] = strides[o][d];
        continue;
      }
    }
    out_sizes[r] = sizes[d];
    for (int o = 0; o < n_ops; ++o) out_strides[o][r] = strides[o][d];
    ++r;
  }
  return r;
}

// ------------------------------------------------------------------------------ casts
// Element readers/writers by dtype code for the cast kernel (values widened to double, the
// way storage_get_unchecked does; narrowed the way storage_set_unchecked does).
__device__ __forceinline__ double read_as_double(int dtype, const void* p, int64_t i) {
  switch (dtype) {
    case MTHIP_F16: return (double)h2f_exact(((const uint16_t*)p)[i]);
    case MTHIP_F32: return (double)((const float*)p)[i];
    case MTHIP_F64: return ((const double*)p)[i];
    case MTHIP_I32: return (double)((const int32_t*)p)[i];
    case MTHIP_I64: return (double)((const int64_t*)p)[i];
    default: return ((const uint8_t*)p)[i] ? 1.0 : 0.0;
  }
}

__device__ __forceinline__ void write_from_double(int dtype, void* p, int64_t i, double v) {
  switch (dtype) {
    case MTHIP_F16: ((uint16_t*)p)[i] = f2h_bits((float)v); break;
    case MTHIP_F32: ((float*)p)[i] = (float)v; break;
    case MTHIP_F64: ((double*)p)[i] = v; break;
    case MTHIP_I32: ((int32_t*)p)[i] = (int32_t)v; break;
    case MTHIP_I64: ((int64_t*)p)[i] = (int64_t)v; break;
    default: ((uint8_t*)p)[i] = v == 0.0 ? 0 : 1; break;
  }
}

// fp32 -> fp16, 8 elements per lane per step (two 16-byte loads, one 16-byte store).
__global__ void cast_f32_f16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t nvec = n / 8;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    const float4 a = reinterpret_cast<const float4*>(src)[2 * v];
    const float4 b = reinterpret_cast<const float4*>(src)[2 * v + 1];
    uint4 out;
    out.x = (uint32_t)f2h_fast(a.x) | ((uint32_t)f2h_fast(a.y) << 16);
    out.y = (uint32_t)f2h_fast(a.z) | ((uint32_t)f2h_fast(a.w) << 16);
    out.z = (uint32_t)f2h_fast(b.x) | ((uint32_t)f2h_fast(b.y) << 16);
    out.w = (uint32_t)f2h_fast(b.z) | ((uint32_t)f2h_fast(b.w) << 16);
    reinterpret_cast<uint4*>(dst)[v] = out;
  }
  for (int64_t i = nvec * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = f2h_bits(src[i]);
}

__global__ void cast_f16_f32_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t nvec = n / 8;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    const uint4 in = reinterpret_cast<const uint4*>(src)[v];
    float4 a, b;
    a.x = h2f_exact((uint16_t)(in.x & 0xffff));
    a.y = h2f_exact((uint16_t)(in.x >> 16));
    a.z = h2f_exact((uint16_t)(in.y & 0xffff));
    a.w = h2f_exact((uint16_t)(in.y >> 16));
    b.x = h2f_exact((uint16_t)(in.z & 0xffff));
    b.y = h2f_exact((uint16_t)(in.z >> 16));
    b.z = h2f_exact((uint16_t)(in.w & 0xffff));
    b.w = h2f_exact((uint16_t)(in.w >> 16));
    reinterpret_cast<float4*>(dst)[2 * v] = a;
    reinterpret_cast<float4*>(dst)[2 * v + 1] = b;
  }
  for (int64_t i = nvec * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = h2f_exact(src[i]);
}

// Dense casts convert element by element with static_cast (cast_dense_numeric_to_half /
// cast_dense_half_to_numeric, tensor.cpp:2633-2657): fp32<->fp16 never widens to double, so
// NaN payloads pass through untouched; the other pairs go through double exactly.
__global__ void cast_generic_kernel(int src_dtype, const void* src, int dst_dtype, void* dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    if (src_dtype == MTHIP_F32 && dst_dtype == MTHIP_F16)
      ((uint16_t*)dst)[i] = f2h_bits(((const float*)src)[i]);
    else if (src_dtype == MTHIP_F16 && dst_dtype == MTHIP_F32)
      ((float*)dst)[i] = h2f_exact(((const uint16_t*)src)[i]);
    else
      write_from_double(dst_dtype, dst, i, read_as_double(src_dtype, src, i));
  }
}

// ------------------------------------------------------------------------------ copies
template <typename T>
__global__ void copy_strided_kernel(const T* __restrict__ src, T* __restrict__ dst, Shape s, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, off = 0;
    for (int d = s.rank - 1; d >= 0; --d) {
      const int64_t idx = rem % s.sizes[d];
      rem /= s.sizes[d];
      off += idx * s.a_strides[d];
    }
    dst[i] = src[off];
  }
}

// dst viewed through b_strides <- src viewed through a_strides (both in element units).
template <typename T>
__global__ void copy_strided_to_kernel(const T* __restrict__ src, T* __restrict__ dst, Shape s, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, so = 0, dof = 0;
    for (int d = s.rank - 1; d >= 0; --d) {
      const int64_t idx = rem % s.sizes[d];
      rem /= s.sizes[d];
      so += idx * s.a_strides[d];
      dof += idx * s.b_strides[d];
    }
    dst[dof] = src[so];
  }
}

// 2-D tiled transpose through LDS for views whose source is unit-stride along the second-last
// collapsed dim (head split/merge [B,L,H,D] <-> [B,H,L,D], NCHW <-> NHWC):
//   dst[b][r][c] (contiguous, c fastest) = src[b*sb + r + c*sc].
// Reads walk r across lanes and writes walk c across lanes, so both are coalesced.
template <typename T>
__global__ void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t R, int64_t C, int64_t sb,
                                 int64_t sc) {
  __shared__ T tile[32][33];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.x * 32, c0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8 threads
  for (int j = ty; j < 32; j += 8) {
    const int64_t r = r0 + tx, c = c0 + j;
    if (r < R && c < C) tile[j][tx] = src[b * sb + r + c * sc];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int64_t c = c0 + tx, r = r0 + j;
    if (r < R && c < C) dst[(b * R + r) * C + c] = tile[tx][j];
  }
}

template <typename T>
__global__ void fill_kernel(T* __restrict__ dst, int64_t n, T value) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = value;
}

// ------------------------------------------------------------------------------ binary
__device__ __forceinline__ float apply_bin(int op, float a, float b) {
  switch (op) {
    case MTHIP_BIN_ADD: return a + b;
    case MTHIP_BIN_MUL: return a * b;
    case MTHIP_BIN_SUB: return a - b;
    default: return a / b;
  }
}

template <typename T>
__global__ void binary_contig_kernel(int op, const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ out,
                                     int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    Elem<T>::store(out, i, apply_bin(op, Elem<T>::load(a, i), Elem<T>::load(b, i)));
}

// Same-shape binary op over 16-byte chunks (8 halves or 4 floats), streamed.
template <typename T, bool NT, int U>
__global__ __launch_bounds__(256) void binary_contig_vec_kernel(int op, const uint4* __restrict__ a,
                                                                const uint4* __restrict__ b, uint4* __restrict__ out,
                                                                int64_t nvec) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < nvec; i0 += stride * U) {
    uint4 x[U], y[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * stride < nvec) {
        x[u] = ld16<NT>(a + i0 + u * stride);
        y[u] = ld16<NT>(b + i0 + u * stride);
      }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (i0 + u * stride >= nvec) break;
      const uint32_t xs[4] = {x[u].x, x[u].y, x[u].z, x[u].w}, ys[4] = {y[u].x, y[u].y, y[u].z, y[u].w};
      uint32_t r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (sizeof(T) == 2) {
          const float lo = apply_bin(op, h2f_bits((uint16_t)(xs[j] & 0xffff)), h2f_bits((uint16_t)(ys[j] & 0xffff)));
          const float hi = apply_bin(op, h2f_bits((uint16_t)(xs[j] >> 16)), h2f_bits((uint16_t)(ys[j] >> 16)));
          r[j] = (uint32_t)f2h_fast(lo) | ((uint32_t)f2h_fast(hi) << 16);
        } else {
          r[j] = __float_as_uint(apply_bin(op, __uint_as_float(xs[j]), __uint_as_float(ys[j])));
        }
      }
      st16<NT>(out + i0 + u * stride, make_uint4(r[0], r[1], r[2], r[3]));
    }
  }
}

template <typename T>
__global__ void binary_strided_kernel(int op, const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ out,
                                      Shape s, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, oa = 0, ob = 0;
    for (int d = s.rank - 1; d >= 0; --d) {
      const int64_t idx = rem % s.sizes[d];
      rem /= s.sizes[d];
      oa += idx * s.a_strides[d];
      ob += idx * s.b_strides[d];
    }
    Elem<T>::store(out, i, apply_bin(op, Elem<T>::load(a, oa), Elem<T>::load(b, ob)));
  }
}

// out[i] = mask[i] ? fill : x[i] over a strided (broadcast) mask and input, as raw element bits
// (masked_fill, tensor.cpp:13497-13610: the fill value is narrowed once on the host).
template <typename U>
__global__ void masked_fill_kernel(const U* __restrict__ x, const uint8_t* __restrict__ mask, U fill, U* __restrict__ out,
                                   Shape s, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, ox = 0, om = 0;
    for (int d = s.rank - 1; d >= 0; --d) {
      const int64_t idx = rem % s.sizes[d];
      rem /= s.sizes[d];
      ox += idx * s.a_strides[d];
      om += idx * s.b_strides[d];
    }
    out[i] = mask[om] ? fill : x[ox];
  }
}

// dst viewed through strides (a_strides) <- value bits.
template <typename U>
__global__ void fill_strided_kernel(U* __restrict__ dst, U value, Shape s, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t rem = i, o = 0;
    for (int d = s.rank - 1; d >= 0; --d) {
      const int64_t idx = rem % s.sizes[d];
      rem /= s.sizes[d];
      o += idx * s.a_strides[d];
    }
    dst[o] = value;
  }
}

// bool not (logical_not, tensor.cpp:14616): any nonzero byte is true.
__global__ void logical_not_kernel(const uint8_t* __restrict__ x, uint8_t* __restrict__ y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = x[i] ? 0 : 1;
}

// Tensor-scalar ops run in double and are narrowed once, as the reference's double path does.
template <typename T>
__global__ void binary_scalar_kernel(int op, const T* __restrict__ x, double scalar, int scalar_first,
                                     T* __restrict__ out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const double v = (double)Elem<T>::load(x, i);
    const double l = scalar_first ? scalar : v, r = scalar_first ? v : scalar;
    double res;
    switch (op) {
      case MTHIP_BIN_ADD: res = l + r; break;
      case MTHIP_BIN_MUL: res = l * r; break;
      case MTHIP_BIN_SUB: res = l - r; break;
      default: res = l / r; break;
    }
    Elem<T>::store(out, i, (float)res);
  }
}

// ------------------------------------------------------------------------------ unary
template <typename T>
__global__ void unary_kernel(int op, const T* __restrict__ x, T* __restrict__ y, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    Elem<T>::store(y, i, apply_unary<T>(op, Elem<T>::load(x, i)));
}

// 16-byte chunks per lane (8 halves or 4 floats) over 16-byte aligned buffers, the op fixed at
// compile time.  With `tab` (fp16 erf-gelu, whose evaluation needs a double-precision erf) each
// half is looked up by its bits instead.
template <typename T, int OP, bool NT, int U>
__global__ __launch_bounds__(256) void unary_vec_kernel(const uint4* __restrict__ x, uint4* __restrict__ y,
                                                        int64_t nvec, const uint16_t* __restrict__ tab) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < nvec; i0 += stride * U) {
  uint4 rr[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (i0 + u * stride < nvec) rr[u] = ld16<NT>(x + i0 + u * stride);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + u * stride;
    if (i >= nvec) break;
    const uint4 r = rr[u];
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (sizeof(T) == 2) {
        uint32_t lo = w[j] & 0xffffu, hi = w[j] >> 16;
        if (tab) {
          lo = tab[lo];
          hi = tab[hi];
        } else if constexpr (OP == MTHIP_UNARY_SILU) {
          lo = silu_half((uint16_t)lo);
          hi = silu_half((uint16_t)hi);
        } else {
          lo = f2h_fast(apply_unary<T>(OP, h2f_bits((uint16_t)lo)));
          hi = f2h_fast(apply_unary<T>(OP, h2f_bits((uint16_t)hi)));
        }
        w[j] = lo | (hi << 16);
      } else {
        w[j] = __float_as_uint(apply_unary<T>(OP, __uint_as_float(w[j])));
      }
    }
    st16<NT>(y + i, make_uint4(w[0], w[1], w[2], w[3]));
  }
  }
}

// fp16 SiLU / erf-GELU over large buffers: one workgroup per CU copies the op's 64 K-entry
// result table (128 KB, exactly what evaluating the op gives for each half) into LDS, then
// streams 16-byte chunks, four per thread in flight, each half looked up in LDS: about four
// vector instructions per element where evaluating SiLU costs ~30 (two of them quarter-rate
// transcendentals) and the GELU table gathers from L2.
// TH threads: 256 for buffers that stream from HBM (see kStreamU), 1024 below that, where
// filling the table with more waves, and more waves per CU, matter more.
template <bool NT, int TH>
__global__ __launch_bounds__(TH) void unary_lut_f16_kernel(const uint4* __restrict__ x, uint4* __restrict__ y,
                                                           int64_t nvec, const uint4* __restrict__ tab) {
  __shared__ uint4 lut[65536 * 2 / 16];
  for (int i = threadIdx.x; i < 65536 * 2 / 16; i += TH) lut[i] = tab[i];
  __syncthreads();
  const uint16_t* L = reinterpret_cast<const uint16_t*>(lut);
  const int64_t stride = (int64_t)gridDim.x * TH;
  for (int64_t i0 = (int64_t)blockIdx.x * TH + threadIdx.x; i0 < nvec; i0 += stride * kStreamU) {
    uint4 r[kStreamU];
#pragma unroll
    for (int u = 0; u < kStreamU; ++u)
      if (i0 + u * stride < nvec) r[u] = ld16<NT>(x + i0 + u * stride);
#pragma unroll
    for (int u = 0; u < kStreamU; ++u) {
      if (i0 + u * stride >= nvec) break;
      uint32_t w[4] = {r[u].x, r[u].y, r[u].z, r[u].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = (uint32_t)L[w[j] & 0xffffu] | ((uint32_t)L[w[j] >> 16] << 16);
      st16<NT>(y + i0 + u * stride, make_uint4(w[0], w[1], w[2], w[3]));
    }
  }
}

// Chunks from which the LDS-table kernel pays for its 128 KB table fill per CU.
constexpr int64_t kLutMinVec = 1 << 18;

template <typename T, bool NT, int U>
void launch_unary_vec_nt(int device, int op, const void* x, void* y, int64_t nvec, const uint16_t* tab,
                         hipStream_t s) {
  const dim3 grid(U > 1 ? stream_grid(device, nvec) : grid_for(nvec, 2)), block(kThreads);
  const uint4* xv = (const uint4*)x;
  uint4* yv = (uint4*)y;
  switch (op) {
#define MTHIP_UNARY_CASE(K) \
    case K: hipLaunchKernelGGL((unary_vec_kernel<T, K, NT, U>), grid, block, 0, s, xv, yv, nvec, tab); break;
    MTHIP_UNARY_CASE(MTHIP_UNARY_SILU)
    MTHIP_UNARY_CASE(MTHIP_UNARY_GELU)
    MTHIP_UNARY_CASE(MTHIP_UNARY_GELU_TANH)
    MTHIP_UNARY_CASE(MTHIP_UNARY_EXP)
    MTHIP_UNARY_CASE(MTHIP_UNARY_SIN)
    MTHIP_UNARY_CASE(MTHIP_UNARY_COS)
    MTHIP_UNARY_CASE(MTHIP_UNARY_NEG)
    MTHIP_UNARY_CASE(MTHIP_UNARY_SIGMOID)
    default: MTHIP_UNARY_CASE(MTHIP_UNARY_RELU)
#undef MTHIP_UNARY_CASE
  }
}

// Large fp32 buffers of the cheap ops stream (see kStreamU); the evaluated fp16 forms, the erf
// and tanh GELUs and the double-precision exp/sin/cos keep one chunk per thread with more waves
// per CU, which hides their vector work better.
template <typename T>
void launch_unary_vec(int device, int op, const void* x, void* y, int64_t nvec, const uint16_t* tab, hipStream_t s) {
  const bool big = 2 * nvec * 16 > kStreamNTBytes;
  const bool cheap = sizeof(T) == 4 && (op == MTHIP_UNARY_SILU || op == MTHIP_UNARY_NEG || op == MTHIP_UNARY_RELU);
  if (big && cheap)
    launch_unary_vec_nt<T, true, kStreamU>(device, op, x, y, nvec, tab, s);
  else if (big)
    launch_unary_vec_nt<T, true, 1>(device, op, x, y, nvec, tab, s);
  else
    launch_unary_vec_nt<T, false, 1>(device, op, x, y, nvec, tab, s);
}

template <typename T>
__global__ void geglu_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t rows, int64_t D) {
  const int64_t n = rows * D;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / D, d = i - r * D;
    const float val = Elem<T>::load(x, r * 2 * D + d);
    const float gate = Elem<T>::load(x, r * 2 * D + D + d);
    const float g = Elem<T>::round_trip(apply_unary<T>(MTHIP_UNARY_GELU, gate));
    Elem<T>::store(y, i, val * g);
  }
}

// ------------------------------------------------------------------------------ cat / upsample
template <typename T>
__global__ void copy_2d_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t outer, int64_t inner,
                               int64_t dst_row_stride) {
  const int64_t n = outer * inner;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t o = i / inner, j = i - o * inner;
    dst[o * dst_row_stride + j] = src[i];
  }
}

template <typename T>
__global__ void upsample_nearest_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t planes, int64_t H,
                                        int64_t W, int64_t sh, int64_t sw) {
  const int64_t OH = H * sh, OW = W * sw;
  const int64_t n = planes * OH * OW;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t ox = i % OW;
    const int64_t t = i / OW;
    const int64_t oy = t % OH;
    const int64_t p = t / OH;
    y[i] = x[(p * H + oy / sh) * W + ox / sw];
  }
}

// 2x2 nearest upsampling with W % 4 == 0: a thread reads 4 consecutive inputs of one row and
// writes the 8 outputs of each of the two output rows they cover (16-byte stores for fp16, two
// for fp32).  Chunk index -> (plane row, chunk) by one 32-bit division (FastDiv).
template <typename T>
__global__ __launch_bounds__(256) void upsample2x_vec_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                             uint32_t rows, uint32_t W, FastDiv div_cw) {
  const uint32_t cw = div_cw.d;  // chunks per input row
  const uint32_t n = rows * cw;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const uint32_t r = div_cw.div(i), c = i - r * cw;  // input row (plane * H + iy), chunk
    const T* src = x + (size_t)r * W + 4 * c;
    T* dst = y + (size_t)r * 4 * W + 8 * c;  // output row 2 * (plane * H + iy) = plane * 2H + 2iy
    if constexpr (sizeof(T) == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(src);
      const uint32_t a = v.x & 0xffffu, b = v.x >> 16, cc = v.y & 0xffffu, d = v.y >> 16;
      const uint4 o = make_uint4(a | (a << 16), b | (b << 16), cc | (cc << 16), d | (d << 16));
      *reinterpret_cast<uint4*>(dst) = o;
      *reinterpret_cast<uint4*>(dst + 2 * W) = o;
    } else {
      const uint4 v = *reinterpret_cast<const uint4*>(src);
      const uint4 o0 = make_uint4(v.x, v.x, v.y, v.y), o1 = make_uint4(v.z, v.z, v.w, v.w);
      *reinterpret_cast<uint4*>(dst) = o0;
      *reinterpret_cast<uint4*>(dst + 4) = o1;
      *reinterpret_cast<uint4*>(dst + 2 * W) = o0;
      *reinterpret_cast<uint4*>(dst + 2 * W + 4) = o1;
    }
  }
}

int elem_size(int dtype) {
  switch (dtype) {
    case MTHIP_F16: return 2;
    case MTHIP_F32: return 4;
    case MTHIP_F64: return 8;
    case MTHIP_I32: return 4;
    case MTHIP_I64: return 8;
    case MTHIP_BOOL: return 1;
    default: return 0;
  }
}

// The SD timestep embedding narrowed to fp16: out[b][j] = half(cos(t[b] f[j])) for j < half and
// half(sin(t[b] f[j - half])) after it -- the broadcast product, cos, sin, cat and cast each
// computed as their own kernels compute them (fp32 product, the double-precision sin/cos of
// apply_unary<float>, f2h_fast), in one launch.
__global__ void timestep_embedding_f16_kernel(const float* __restrict__ t, const float* __restrict__ f,
                                              uint16_t* __restrict__ out, int64_t B, int64_t half) {
  const int64_t n = B * 2 * half;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t b = i / (2 * half), j = i - b * 2 * half;
    const bool second = j >= half;
    const float x = t[b] * f[second ? j - half : j];
    out[i] = f2h_fast(apply_unary<float>(second ? MTHIP_UNARY_SIN : MTHIP_UNARY_COS, x));
  }
}

}  // namespace
}  // namespace mthip

using namespace mthip;

extern "C" {

int mthip_timestep_embedding_f16(int device, const void* t, const void* freqs, void* out, int64_t B, int64_t half) {
  MTHIP_REQUIRE(B >= 0 && half > 0 && B * 2 * half < (int64_t(1) << 40), "mthip_timestep_embedding_f16: bad extents");
  if (B == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  hipLaunchKernelGGL(timestep_embedding_f16_kernel, dim3(grid_for(B * 2 * half)), dim3(kThreads), 0, s,
                     (const float*)t, (const float*)freqs, (uint16_t*)out, B, half);
  return check_launch("timestep_embedding_f16_kernel");
}

int mthip_cast(int device, int src_dtype, const void* src, int dst_dtype, void* dst, int64_t n) {
  MTHIP_REQUIRE(elem_size(src_dtype) && elem_size(dst_dtype), "mthip_cast: unknown dtype");
  MTHIP_REQUIRE(n >= 0, "mthip_cast: negative element count");
  if (n == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  const bool aligned = ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0);
  if (src_dtype == dst_dtype) {
    MTHIP_CHECK_HIP(hipMemcpyAsync(dst, src, (size_t)n * elem_size(src_dtype), hipMemcpyDeviceToDevice, s));
    return MTHIP_OK;
  }
  if (src_dtype == MTHIP_F32 && dst_dtype == MTHIP_F16 && aligned) {
    hipLaunchKernelGGL(cast_f32_f16_kernel, dim3(grid_for(n, 8)), dim3(kThreads), 0, s, (const float*)src, (uint16_t*)dst, n);
  } else if (src_dtype == MTHIP_F16 && dst_dtype == MTHIP_F32 && aligned) {
    hipLaunchKernelGGL(cast_f16_f32_kernel, dim3(grid_for(n, 8)), dim3(kThreads), 0, s, (const uint16_t*)src, (float*)dst, n);
  } else {
    hipLaunchKernelGGL(cast_generic_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s, src_dtype, src, dst_dtype, dst, n);
  }
  return check_launch("mthip_cast");
}

int mthip_copy_strided(int device, int dtype, const void* src, int rank, const int64_t* sizes,
                       const int64_t* src_strides, void* dst) {
  const int es = elem_size(dtype);
  MTHIP_REQUIRE(es != 0, "mthip_copy_strided: unknown dtype");
  MTHIP_REQUIRE(rank >= 0 && rank <= kMaxRank, "mthip_copy_strided: rank must be <= 8");
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) {
    MTHIP_REQUIRE(sizes[d] >= 0, "mthip_copy_strided: negative size");
    n *= sizes[d];
  }
  if (n == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  // Destination strides are contiguous; collapse dims jointly with the source strides.
  int64_t dst_strides[kMaxRank];
  {
    int64_t acc = 1;
    for (int d = rank - 1; d >= 0; --d) {
      dst_strides[d] = acc;
      acc *= sizes[d];
    }
  }
  Shape sh{};
  int64_t* outs[2] = {sh.a_strides, sh.b_strides};
  const int64_t* ins[2] = {src_strides, dst_strides};
  sh.rank = collapse(rank, sizes, ins, 2, sh.sizes, outs);
  if (sh.rank == 0 || (sh.rank == 1 && sh.a_strides[0] == 1)) {
    MTHIP_CHECK_HIP(hipMemcpyAsync(dst, src, (size_t)n * es, hipMemcpyDeviceToDevice, s));
    return MTHIP_OK;
  }
  // Source unit-stride along the second-last collapsed dim: tiled transpose through LDS.
  if (sh.rank >= 2 && sh.rank <= 3 && sh.a_strides[sh.rank - 2] == 1 && (es == 2 || es == 4)) {
    const int64_t R = sh.sizes[sh.rank - 2], C = sh.sizes[sh.rank - 1];
    const int64_t batch = sh.rank == 3 ? sh.sizes[0] : 1;
    const int64_t sb = sh.rank == 3 ? sh.a_strides[0] : 0;
    const int64_t sc = sh.a_strides[sh.rank - 1];
    dim3 grid((unsigned)ceil_div(R, 32), (unsigned)ceil_div(C, 32), (unsigned)batch);
    if (batch <= 65535 && ceil_div(C, 32) <= 65535) {
      if (es == 2)
        hipLaunchKernelGGL(transpose_kernel<uint16_t>, grid, dim3(256), 0, s, (const uint16_t*)src, (uint16_t*)dst, R, C, sb, sc);
      else
        hipLaunchKernelGGL(transpose_kernel<uint32_t>, grid, dim3(256), 0, s, (const uint32_t*)src, (uint32_t*)dst, R, C, sb, sc);
      return check_launch("mthip_copy_strided(transpose)");
    }
  }
  switch (es) {
    case 1: hipLaunchKernelGGL(copy_strided_kernel<uint8_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint8_t*)src, (uint8_t*)dst, sh, n); break;
    case 2: hipLaunchKernelGGL(copy_strided_kernel<uint16_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint16_t*)src, (uint16_t*)dst, sh, n); break;
    case 4: hipLaunchKernelGGL(copy_strided_kernel<uint32_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint32_t*)src, (uint32_t*)dst, sh, n); break;
    default: hipLaunchKernelGGL(copy_strided_kernel<uint64_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint64_t*)src, (uint64_t*)dst, sh, n); break;
  }
  return check_launch("mthip_copy_strided");
}

int mthip_copy_strided_to(int device, int dtype, const void* src, const int64_t* src_strides, int rank,
                          const int64_t* sizes, void* dst, const int64_t* dst_strides) {
  const int es = elem_size(dtype);
  MTHIP_REQUIRE(es != 0, "mthip_copy_strided_to: unknown dtype");
  MTHIP_REQUIRE(rank >= 0 && rank <= kMaxRank, "mthip_copy_strided_to: rank must be <= 8");
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) {
    MTHIP_REQUIRE(sizes[d] >= 0, "mthip_copy_strided_to: negative size");
    n *= sizes[d];
  }
  if (n == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  Shape sh{};
  int64_t* outs[2] = {sh.a_strides, sh.b_strides};
  const int64_t* ins[2] = {src_strides, dst_strides};
  sh.rank = collapse(rank, sizes, ins, 2, sh.sizes, outs);
  if (sh.rank == 0) sh.rank = 1, sh.sizes[0] = 1, sh.a_strides[0] = 0, sh.b_strides[0] = 0;
  const unsigned g = grid_for(n);
  switch (es) {
    case 1: hipLaunchKernelGGL(copy_strided_to_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, s, (const uint8_t*)src, (uint8_t*)dst, sh, n); break;
    case 2: hipLaunchKernelGGL(copy_strided_to_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, (const uint16_t*)src, (uint16_t*)dst, sh, n); break;
    case 4: hipLaunchKernelGGL(copy_strided_to_kernel<uint32_t>, dim3(g), dim3(kThreads), 0, s, (const uint32_t*)src, (uint32_t*)dst, sh, n); break;
    default: hipLaunchKernelGGL(copy_strided_to_kernel<uint64_t>, dim3(g), dim3(kThreads), 0, s, (const uint64_t*)src, (uint64_t*)dst, sh, n); break;
  }
  return check_launch("mthip_copy_strided_to");
}

// The storage bits of `value` written as `dtype` (F16: float_to_half_bits((float)value),
// tensor.cpp:276-315, restated on the host for one value; F32 through (float); BOOL as value != 0).
static uint64_t host_fill_bits(int dtype, double value) {
  switch (dtype) {
    case MTHIP_F16: {
      const float f = (float)value;
      uint32_t bits;
      std::memcpy(&bits, &f, 4);
      const uint32_t sign = (bits >> 16) & 0x8000u, raw = (bits >> 23) & 0xffu;
      const uint32_t man = bits & 0x7fffffu;
      if (raw == 0xffu) return sign | 0x7c00u | (man ? ((man >> 13) ? (man >> 13) : 0x200u) : 0u);
      const int32_t e = (int32_t)raw - 112;
      if (e <= 0) return e < -10 ? sign : (sign | ((((man | 0x800000u) >> (1 - e)) + 0x1000u) >> 13));
      const uint32_t r = ((uint32_t)e << 10) + ((man + 0x1000u) >> 13);
      return sign | (r >= 0x7c00u ? 0x7c00u : r);
    }
    case MTHIP_F32: {
      const float f = (float)value;
      uint32_t bits;
      std::memcpy(&bits, &f, 4);
      return bits;
    }
    case MTHIP_F64: {
      uint64_t bits;
      std::memcpy(&bits, &value, 8);
      return bits;
    }
    case MTHIP_I32: return (uint32_t)(int32_t)value;
    case MTHIP_I64: return (uint64_t)(int64_t)value;
    default: return value != 0.0 ? 1u : 0u;
  }
}

int mthip_fill(int device, int dtype, void* dst, int64_t n, double value) {
  const int es = elem_size(dtype);
  MTHIP_REQUIRE(es != 0, "mthip_fill: unknown dtype");
  if (n <= 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  const unsigned g = grid_for(n);
  const uint64_t bits = host_fill_bits(dtype, value);
  switch (es) {
    case 1: hipLaunchKernelGGL(fill_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, s, (uint8_t*)dst, n, (uint8_t)bits); break;
    case 2: hipLaunchKernelGGL(fill_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, (uint16_t*)dst, n, (uint16_t)bits); break;
    case 4: hipLaunchKernelGGL(fill_kernel<uint32_t>, dim3(g), dim3(kThreads), 0, s, (uint32_t*)dst, n, (uint32_t)bits); break;
    default: hipLaunchKernelGGL(fill_kernel<uint64_t>, dim3(g), dim3(kThreads), 0, s, (uint64_t*)dst, n, bits); break;
  }
  return check_launch("mthip_fill");
}

int mthip_fill_strided(int device, int dtype, void* dst, int rank, const int64_t* sizes, const int64_t* strides,
                       double value) {
  const int es = elem_size(dtype);
  MTHIP_REQUIRE(es != 0, "mthip_fill_strided: unknown dtype");
  MTHIP_REQUIRE(rank >= 0 && rank <= kMaxRank, "mthip_fill_strided: rank must be <= 8");
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= sizes[d];
  if (n == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  Shape sh{};
  int64_t unused[kMaxRank];
  int64_t* outs[2] = {sh.a_strides, unused};
  const int64_t* ins[2] = {strides, strides};
  sh.rank = collapse(rank, sizes, ins, 2, sh.sizes, outs);
  if (sh.rank == 0) sh.rank = 1, sh.sizes[0] = 1, sh.a_strides[0] = 0;
  const unsigned g = grid_for(n);
  const uint64_t bits = host_fill_bits(dtype, value);
  switch (es) {
    case 1: hipLaunchKernelGGL(fill_strided_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, s, (uint8_t*)dst, (uint8_t)bits, sh, n); break;
    case 2: hipLaunchKernelGGL(fill_strided_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, (uint16_t*)dst, (uint16_t)bits, sh, n); break;
    case 4: hipLaunchKernelGGL(fill_strided_kernel<uint32_t>, dim3(g), dim3(kThreads), 0, s, (uint32_t*)dst, (uint32_t)bits, sh, n); break;
    default: hipLaunchKernelGGL(fill_strided_kernel<uint64_t>, dim3(g), dim3(kThreads), 0, s, (uint64_t*)dst, bits, sh, n); break;
  }
  return check_launch("mthip_fill_strided");
}

int mthip_masked_fill(int device, int dtype, const void* x, const int64_t* x_strides, const void* mask,
                      const int64_t* mask_strides, double value, void* out, int rank, const int64_t* out_sizes) {
  const int es = elem_size(dtype);
  MTHIP_REQUIRE(es != 0, "mthip_masked_fill: unknown dtype");
  MTHIP_REQUIRE(rank >= 0 && rank <= kMaxRank, "mthip_masked_fill: rank must be <= 8");
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= out_sizes[d];
  if (n == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  int64_t out_strides[kMaxRank];
  {
    int64_t acc = 1;
    for (int d = rank - 1; d >= 0; --d) {
      out_strides[d] = acc;
      acc *= out_sizes[d];
    }
  }
  Shape sh{};
  int64_t o_str[kMaxRank];
  int64_t* outs[3] = {sh.a_strides, sh.b_strides, o_str};
  const int64_t* ins[3] = {x_strides, mask_strides, out_strides};
  sh.rank = collapse(rank, out_sizes, ins, 3, sh.sizes, outs);
  if (sh.rank == 0) sh.rank = 1, sh.sizes[0] = 1, sh.a_strides[0] = 0, sh.b_strides[0] = 0;
  const unsigned g = grid_for(n);
  const uint64_t bits = host_fill_bits(dtype, value);
  const uint8_t* m = static_cast<const uint8_t*>(mask);
  switch (es) {
    case 1: hipLaunchKernelGGL(masked_fill_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, s, (const uint8_t*)x, m, (uint8_t)bits, (uint8_t*)out, sh, n); break;
    case 2: hipLaunchKernelGGL(masked_fill_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, (const uint16_t*)x, m, (uint16_t)bits, (uint16_t*)out, sh, n); break;
    case 4: hipLaunchKernelGGL(masked_fill_kernel<uint32_t>, dim3(g), dim3(kThreads), 0, s, (const uint32_t*)x, m, (uint32_t)bits, (uint32_t*)out, sh, n); break;
    default: hipLaunchKernelGGL(masked_fill_kernel<uint64_t>, dim3(g), dim3(kThreads), 0, s, (const uint64_t*)x, m, bits, (uint64_t*)out, sh, n); break;
  }
  return check_launch("mthip_masked_fill");
}

int mthip_logical_not(int device, const void* x, void* y, int64_t n) {
  if (n <= 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  hipLaunchKernelGGL(logical_not_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint8_t*)x, (uint8_t*)y, n);
  return check_launch("mthip_logical_not");
}

int mthip_cat(int device, int dtype, int count, const void* const* inputs, const int64_t* dim_sizes, int rank,
              const int64_t* out_sizes, int dim, void* out) {
  const int es = elem_size(dtype);
  MTHIP_REQUIRE(es != 0, "mthip_cat: unknown dtype");
  MTHIP_REQUIRE(rank >= 1 && dim >= 0 && dim < rank, "mthip_cat: bad dim");
  int64_t outer = 1, inner = 1, total = 0;
  for (int d = 0; d < dim; ++d) outer *= out_sizes[d];
  for (int d = dim + 1; d < rank; ++d) inner *= out_sizes[d];
  for (int i = 0; i < count; ++i) total += dim_sizes[i];
  MTHIP_REQUIRE(total == out_sizes[dim], "mthip_cat: input extents do not sum to the output extent");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  int64_t offset = 0;
  for (int i = 0; i < count; ++i) {
    const int64_t in_inner = dim_sizes[i] * inner;
    const int64_t n = outer * in_inner;
    if (n > 0) {
      char* dst = (char*)out + offset * inner * es;
      const unsigned g = grid_for(n);
      switch (es) {
        case 1: hipLaunchKernelGGL(copy_2d_kernel<uint8_t>, dim3(g), dim3(kThreads), 0, s, (const uint8_t*)inputs[i], (uint8_t*)dst, outer, in_inner, total * inner); break;
        case 2: hipLaunchKernelGGL(copy_2d_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, (const uint16_t*)inputs[i], (uint16_t*)dst, outer, in_inner, total * inner); break;
        case 4: hipLaunchKernelGGL(copy_2d_kernel<uint32_t>, dim3(g), dim3(kThreads), 0, s, (const uint32_t*)inputs[i], (uint32_t*)dst, outer, in_inner, total * inner); break;
        default: hipLaunchKernelGGL(copy_2d_kernel<uint64_t>, dim3(g), dim3(kThreads), 0, s, (const uint64_t*)inputs[i], (uint64_t*)dst, outer, in_inner, total * inner); break;
      }
      if (int rc = check_launch("mthip_cat")) return rc;
    }
    offset += dim_sizes[i];
  }
  return MTHIP_OK;
}

int mthip_upsample_nearest2d(int device, int dtype, const void* x, void* y, int64_t planes, int64_t H, int64_t W,
                             int64_t scale_h, int64_t scale_w) {
  const int es = elem_size(dtype);
  MTHIP_REQUIRE(es == 2 || es == 4, "mthip_upsample_nearest2d: dtype must be F16 or F32");
  MTHIP_REQUIRE(scale_h >= 1 && scale_w >= 1, "mthip_upsample_nearest2d: scale must be >= 1");
  const int64_t n = planes * H * scale_h * W * scale_w;
  if (n == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  const int64_t rows = planes * H;
  if (scale_h == 2 && scale_w == 2 && W % 4 == 0 && rows * W < (int64_t(1) << 31) && ((uintptr_t)x & 15) == 0 &&
      ((uintptr_t)y & 15) == 0) {
    // the decoder's 2x upsampling: vectorised rows
    const FastDiv div_cw((uint32_t)(W / 4));
    const unsigned g = grid_for(rows * (W / 4));
    if (es == 2)
      hipLaunchKernelGGL(upsample2x_vec_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, (const uint16_t*)x,
                         (uint16_t*)y, (uint32_t)rows, (uint32_t)W, div_cw);
    else
      hipLaunchKernelGGL(upsample2x_vec_kernel<uint32_t>, dim3(g), dim3(kThreads), 0, s, (const uint32_t*)x,
                         (uint32_t*)y, (uint32_t)rows, (uint32_t)W, div_cw);
    return check_launch("mthip_upsample_nearest2d");
  }
  if (es == 2)
    hipLaunchKernelGGL(upsample_nearest_kernel<uint16_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint16_t*)x, (uint16_t*)y, planes, H, W, scale_h, scale_w);
  else
    hipLaunchKernelGGL(upsample_nearest_kernel<uint32_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint32_t*)x, (uint32_t*)y, planes, H, W, scale_h, scale_w);
  return check_launch("mthip_upsample_nearest2d");
}

int mthip_binary(int device, int op, int dtype, const void* a, const int64_t* a_strides, const void* b,
                 const int64_t* b_strides, void* out, int rank, const int64_t* out_sizes) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_binary: dtype must be F16 or F32");
  MTHIP_REQUIRE(op >= MTHIP_BIN_ADD && op <= MTHIP_BIN_DIV, "mthip_binary: unknown op");
  MTHIP_REQUIRE(rank >= 0 && rank <= kMaxRank, "mthip_binary: rank must be <= 8");
  int64_t n = 1;
  for (int d = 0; d < rank; ++d) n *= out_sizes[d];
  if (n == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  int64_t out_strides[kMaxRank];
  {
    int64_t acc = 1;
    for (int d = rank - 1; d >= 0; --d) {
      out_strides[d] = acc;
      acc *= out_sizes[d];
    }
  }
  Shape sh{};
  int64_t o_str[kMaxRank];
  int64_t* outs[3] = {sh.a_strides, sh.b_strides, o_str};
  const int64_t* ins[3] = {a_strides, b_strides, out_strides};
  sh.rank = collapse(rank, out_sizes, ins, 3, sh.sizes, outs);
  const bool contig = sh.rank <= 1 && (sh.rank == 0 || (sh.a_strides[0] == 1 && sh.b_strides[0] == 1));
  const unsigned g = grid_for(n);
  const int esz = dtype == MTHIP_F16 ? 2 : 4;
  if (contig && (n * esz) % 16 == 0 && (((uintptr_t)a | (uintptr_t)b | (uintptr_t)out) & 15) == 0) {
    const int64_t nvec = n * esz / 16;
    const uint4 *av = (const uint4*)a, *bv = (const uint4*)b;
    uint4* ov = (uint4*)out;
    // Large fp32 buffers stream (see kStreamU); the narrowing in fp16 ops keeps one chunk per
    // thread, more waves per CU and cached accesses (64x batch: 202 us against 212 us non-temporal
    // and 263 us streamed).
    if (3 * n * esz > kStreamNTBytes && dtype == MTHIP_F32)
      hipLaunchKernelGGL((binary_contig_vec_kernel<float, true, kStreamU>), dim3(stream_grid(device, nvec)),
                         dim3(kThreads), 0, s, op, av, bv, ov, nvec);
    else if (dtype == MTHIP_F32)
      hipLaunchKernelGGL((binary_contig_vec_kernel<float, false, 1>), dim3(grid_for(nvec)), dim3(kThreads), 0, s, op,
                         av, bv, ov, nvec);
    else
      hipLaunchKernelGGL((binary_contig_vec_kernel<uint16_t, false, 1>), dim3(grid_for(nvec)), dim3(kThreads), 0, s,
                         op, av, bv, ov, nvec);
  } else if (contig) {
    if (dtype == MTHIP_F16)
      hipLaunchKernelGGL(binary_contig_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, op, (const uint16_t*)a, (const uint16_t*)b, (uint16_t*)out, n);
    else
      hipLaunchKernelGGL(binary_contig_kernel<float>, dim3(g), dim3(kThreads), 0, s, op, (const float*)a, (const float*)b, (float*)out, n);
  } else {
    if (sh.rank == 0) sh.rank = 1, sh.sizes[0] = 1, sh.a_strides[0] = 0, sh.b_strides[0] = 0;
    if (dtype == MTHIP_F16)
      hipLaunchKernelGGL(binary_strided_kernel<uint16_t>, dim3(g), dim3(kThreads), 0, s, op, (const uint16_t*)a, (const uint16_t*)b, (uint16_t*)out, sh, n);
    else
      hipLaunchKernelGGL(binary_strided_kernel<float>, dim3(g), dim3(kThreads), 0, s, op, (const float*)a, (const float*)b, (float*)out, sh, n);
  }
  return check_launch("mthip_binary");
}

int mthip_binary_scalar(int device, int op, int dtype, const void* x, double scalar, int scalar_first, void* out,
                        int64_t n) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_binary_scalar: dtype must be F16 or F32");
  MTHIP_REQUIRE(op >= MTHIP_BIN_ADD && op <= MTHIP_BIN_DIV, "mthip_binary_scalar: unknown op");
  if (n <= 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16)
    hipLaunchKernelGGL(binary_scalar_kernel<uint16_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, op, (const uint16_t*)x, scalar, scalar_first, (uint16_t*)out, n);
  else
    hipLaunchKernelGGL(binary_scalar_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, s, op, (const float*)x, scalar, scalar_first, (float*)out, n);
  return check_launch("mthip_binary_scalar");
}

int mthip_unary(int device, int op, int dtype, const void* x, void* y, int64_t n) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_unary: dtype must be F16 or F32");
  MTHIP_REQUIRE(op >= MTHIP_UNARY_SILU && op <= MTHIP_UNARY_RELU, "mthip_unary: unknown op");
  if (n <= 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  const int esz = dtype == MTHIP_F16 ? 2 : 4;
  int64_t done = 0;
  if ((((uintptr_t)x | (uintptr_t)y) & 15) == 0 && n * esz >= 16) {
    const int64_t nvec = n * esz / 16;
    const bool lut = dtype == MTHIP_F16 && (op == MTHIP_UNARY_SILU || op == MTHIP_UNARY_GELU) && nvec >= kLutMinVec;
    if (lut) {
      const uint16_t* tab = op == MTHIP_UNARY_GELU ? gelu_f16_lookup(device, s) : silu_f16_lookup(device, s);
      if (!tab) return fail(MTHIP_ERR_HIP, "mthip_unary: table setup failed");
      // one workgroup per CU (the table fills the LDS)
      if (2 * nvec * 16 > kStreamNTBytes)
        hipLaunchKernelGGL((unary_lut_f16_kernel<true, 256>), dim3((unsigned)std::min<int64_t>(cu_count_dev(device),
                                                                                              ceil_div(nvec, 256))),
                           dim3(256), 0, s, (const uint4*)x, (uint4*)y, nvec, (const uint4*)tab);
      else
        hipLaunchKernelGGL((unary_lut_f16_kernel<false, 1024>), dim3((unsigned)std::min<int64_t>(cu_count_dev(device),
                                                                                                 ceil_div(nvec, 1024))),
                           dim3(1024), 0, s, (const uint4*)x, (uint4*)y, nvec, (const uint4*)tab);
    } else if (dtype == MTHIP_F16)
      launch_unary_vec<uint16_t>(device, op, x, y, nvec, op == MTHIP_UNARY_GELU ? gelu_f16_lookup(device, s) : nullptr,
                                 s);
    else
      launch_unary_vec<float>(device, op, x, y, nvec, nullptr, s);
    done = nvec * 16 / esz;
  }
  if (done < n) {
    const int64_t rest = n - done;
    if (dtype == MTHIP_F16)
      hipLaunchKernelGGL(unary_kernel<uint16_t>, dim3(grid_for(rest)), dim3(kThreads), 0, s, op,
                         (const uint16_t*)x + done, (uint16_t*)y + done, rest);
    else
      hipLaunchKernelGGL(unary_kernel<float>, dim3(grid_for(rest)), dim3(kThreads), 0, s, op,
                         (const float*)x + done, (float*)y + done, rest);
  }
  return check_launch("mthip_unary");
}

int mthip_geglu(int device, int dtype, const void* x, void* y, int64_t rows, int64_t D) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_geglu: dtype must be F16 or F32");
  const int64_t n = rows * D;
  if (n <= 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16)
    hipLaunchKernelGGL(geglu_kernel<uint16_t>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const uint16_t*)x, (uint16_t*)y, rows, D);
  else
    hipLaunchKernelGGL(geglu_kernel<float>, dim3(grid_for(n)), dim3(kThreads), 0, s, (const float*)x, (float*)y, rows, D);
  return check_launch("mthip_geglu");
}

}  // extern "C"
