// MFMA GEMM core for gfx950, shared by linear/matmul/addmm (gemm.hip) and the implicit-GEMM
// conv2d (conv.hip).
//
//   C[m, n] = sum_k A[m, k] * B[n, k]      (A and B staged k-contiguous in LDS)
//
// One workgroup = 4 wave64s computing a BM x BN tile; each wave owns a (BM/WGM) x (BN/WGN)
// sub-tile made of 32x32 MFMA fragments.  fp16 uses v_mfma_f32_32x32x16_f16 (fp32
// accumulate), fp32 uses v_mfma_f32_32x32x2f32.  K advances in BK-wide tiles through two LDS
// buffers: the global loads of tile k+1 are issued before the MFMAs of tile k and written to
// the other buffer afterwards, so one barrier per tile suffices.
//
// The B operand has three sources (MODE): a k-contiguous [N, K] matrix (linear weights, x.W^T),
// an n-contiguous [K, N] matrix (matmul; transposed while staging), or an implicit im2col of an
// NHWC activation (conv2d).  The epilogue (EPI) applies the op-specific tail and narrows with
// mtorch's fp16 rounding.
#pragma once

#include <hip/hip_runtime.h>

#include "activations.h"
#include "common.h"

namespace mthip {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

enum { MODE_NT = 0, MODE_NN = 1, MODE_CONV = 2 };
enum { EPI_LINEAR = 0, EPI_GEMM = 1, EPI_CONV = 2 };

template <typename T>
struct Mfma;

template <>
struct Mfma<uint16_t> {
  static constexpr int KI = 16;  // k consumed per MFMA
  static constexpr int VEC = 8;  // elements per 16-byte global chunk
  static constexpr int PAD = 8;  // LDS row padding (elements) against bank conflicts
  static __device__ __forceinline__ floatx16 fma(const uint16_t* a_row, const uint16_t* b_row, int kk, int lane,
                                                 floatx16 acc) {
    const halfx8 a = *reinterpret_cast<const halfx8*>(a_row + kk + (lane >> 5) * 8);
    const halfx8 b = *reinterpret_cast<const halfx8*>(b_row + kk + (lane >> 5) * 8);
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int KI = 2;
  static constexpr int VEC = 4;
  static constexpr int PAD = 4;
  static __device__ __forceinline__ floatx16 fma(const float* a_row, const float* b_row, int kk, int lane,
                                                 floatx16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a_row[kk + (lane >> 5)], b_row[kk + (lane >> 5)], acc, 0, 0, 0);
  }
};

struct GemmArgs {
  int64_t M, N, K;
  const void* a;
  int64_t lda, stride_a;
  const void* b;
  int64_t ldb, stride_b;
  void* c;
  int64_t ldc, stride_c;
  // EPI_LINEAR / EPI_CONV
  const void* bias;
  int act;
  const void* residual;
  int64_t ld_res;
  // EPI_GEMM
  float alpha, beta;
  const void* c_in;
  int64_t c_in_rs, c_in_cs, stride_c_in;
  // MODE_CONV: B[n = output pixel, k = (ky, kx, c)] gathered from x_nhwc[img, iy, ix, Cp]
  int64_t H, W, Cp, OH, OW, KW, sh, sw, ph, pw, dh, dw;
  int vec_ok;  // every A/B chunk may be read as one aligned 16-byte load
};

// Loads one VEC-element chunk of a row-major operand (k contiguous) with bounds on rows and k.
template <typename T>
__device__ __forceinline__ uint4 load_chunk_k(const T* base, int64_t row, int64_t rows, int64_t ld, int64_t k,
                                              int64_t K, bool vec_ok) {
  constexpr int VEC = Mfma<T>::VEC;
  uint4 r = make_uint4(0, 0, 0, 0);
  if (row >= rows) return r;
  const T* p = base + row * ld + k;
  if (vec_ok && k + VEC <= K) return *reinterpret_cast<const uint4*>(p);
  T tmp[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) tmp[j] = (k + j < K) ? p[j] : T(0);
  __builtin_memcpy(&r, tmp, 16);
  return r;
}

template <typename T, int BM, int BN, int BK, int WGM, int MODE, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs args) {
  constexpr int VEC = Mfma<T>::VEC, LDK = BK + Mfma<T>::PAD;
  constexpr int WGN = 4 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  static_assert(FM >= 1 && FN >= 1 && WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
  constexpr int CH_PER_ROW = BK / VEC;
  constexpr int A_CH = BM * CH_PER_ROW / 256;
  constexpr int B_CH = BN * CH_PER_ROW / 256;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");
  constexpr int NB_CH_ROW = BN / VEC;  // MODE_NN: chunks along n per k row
  constexpr int B_CH_NN = BK * NB_CH_ROW / 256;

  __shared__ __align__(16) T As[2][BM * LDK];
  __shared__ __align__(16) T Bs[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int64_t bz = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const T* A = reinterpret_cast<const T*>(args.a) + bz * args.stride_a;
  const T* Bm = reinterpret_cast<const T*>(args.b) + bz * args.stride_b;
  const bool vec_ok = args.vec_ok != 0;

  // MODE_CONV: each thread's B chunks cover fixed output pixels; decompose them once.
  int64_t conv_img[B_CH], conv_iy0[B_CH], conv_ix0[B_CH];
  if constexpr (MODE == MODE_CONV) {
    const int64_t OHW = args.OH * args.OW;
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + i * 256;
      const int64_t p = n0 + c / CH_PER_ROW;
      const int64_t img = p / OHW, pix = p - img * OHW;
      const int64_t oy = pix / args.OW, ox = pix - oy * args.OW;
      conv_img[i] = p < args.N ? img : -1;
      conv_iy0[i] = oy * args.sh - args.ph;
      conv_ix0[i] = ox * args.sw - args.pw;
    }
  }

  uint4 ra[A_CH];
  uint4 rb[MODE == MODE_NN ? B_CH_NN : B_CH];

  auto load_tiles = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * 256;
      ra[i] = load_chunk_k<T>(A, m0 + c / CH_PER_ROW, args.M, args.lda, k0 + (c % CH_PER_ROW) * VEC, args.K, vec_ok);
    }
    if constexpr (MODE == MODE_NT) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + i * 256;
        rb[i] = load_chunk_k<T>(Bm, n0 + c / CH_PER_ROW, args.N, args.ldb, k0 + (c % CH_PER_ROW) * VEC, args.K, vec_ok);
      }
    } else if constexpr (MODE == MODE_NN) {
#pragma unroll
      for (int i = 0; i < B_CH_NN; ++i) {
        const int c = tid + i * 256;
        const int64_t k = k0 + c / NB_CH_ROW, n = n0 + (c % NB_CH_ROW) * VEC;
        uint4 r = make_uint4(0, 0, 0, 0);
        if (k < args.K) {
          const T* p = Bm + k * args.ldb + n;
          if (vec_ok && n + VEC <= args.N) {
            r = *reinterpret_cast<const uint4*>(p);
          } else {
            T tmp[VEC];
#pragma unroll
            for (int j = 0; j < VEC; ++j) tmp[j] = (n + j < args.N) ? p[j] : T(0);
            __builtin_memcpy(&r, tmp, 16);
          }
        }
        rb[i] = r;
      }
    } else {
      const T* X = reinterpret_cast<const T*>(args.b);
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + i * 256;
        const int64_t k = k0 + (c % CH_PER_ROW) * VEC;
        uint4 r = make_uint4(0, 0, 0, 0);
        if (conv_img[i] >= 0 && k < args.K) {
          const int64_t tap = k / args.Cp, ch = k - tap * args.Cp;
          const int64_t ky = tap / args.KW, kx = tap - ky * args.KW;
          const int64_t iy = conv_iy0[i] + ky * args.dh, ix = conv_ix0[i] + kx * args.dw;
          if (iy >= 0 && iy < args.H && ix >= 0 && ix < args.W)
            r = *reinterpret_cast<const uint4*>(X + ((conv_img[i] * args.H + iy) * args.W + ix) * args.Cp + ch);
        }
        rb[i] = r;
      }
    }
  };

  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<uint4*>(&As[buf][(c / CH_PER_ROW) * LDK + (c % CH_PER_ROW) * VEC]) = ra[i];
    }
    if constexpr (MODE == MODE_NN) {
#pragma unroll
      for (int i = 0; i < B_CH_NN; ++i) {
        const int c = tid + i * 256;
        const int kr = c / NB_CH_ROW, nc = (c % NB_CH_ROW) * VEC;
        T tmp[VEC];
        __builtin_memcpy(tmp, &rb[i], 16);
#pragma unroll
        for (int j = 0; j < VEC; ++j) Bs[buf][(nc + j) * LDK + kr] = tmp[j];
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int c = tid + i * 256;
        *reinterpret_cast<uint4*>(&Bs[buf][(c / CH_PER_ROW) * LDK + (c % CH_PER_ROW) * VEC]) = rb[i];
      }
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int64_t nk = ceil_div(args.K, BK);
  load_tiles(0);
  store_tiles(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = (int)(kt & 1);
    if (kt + 1 < nk) load_tiles((kt + 1) * BK);
    const T* a_base = &As[cur][(wm * WM + (lane & 31)) * LDK];
    const T* b_base = &Bs[cur][(wn * WN + (lane & 31)) * LDK];
#pragma unroll
    for (int kk = 0; kk < BK; kk += Mfma<T>::KI) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = Mfma<T>::fma(a_base + i * 32 * LDK, b_base + j * 32 * LDK, kk, lane, acc[i][j]);
    }
    if (kt + 1 < nk) store_tiles(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue.  Fragment (i, j) register r of lane l holds
  //      row = wm*WM + i*32 + 8*(r/4) + 4*(l/32) + r%4,   col = wn*WN + j*32 + l%32.
  T* Cp_ = reinterpret_cast<T*>(args.c);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn * WN + j * 32 + (lane & 31);
      if (col >= args.N) continue;
      // Per-column state for the conv epilogue (NCHW address of output pixel `col`).
      int64_t conv_base = 0;
      if constexpr (EPI == EPI_CONV) {
        const int64_t OHW = args.OH * args.OW;
        const int64_t img = col / OHW, pix = col - img * OHW;
        conv_base = img * args.M * OHW + pix;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= args.M) continue;
        float v = acc[i][j][r];
        if constexpr (EPI == EPI_LINEAR) {
          if (args.bias) v += Elem<T>::load(reinterpret_cast<const T*>(args.bias), col);
          v = Elem<T>::round_trip(v);
          if (args.act) v = Elem<T>::round_trip(apply_act<T>(args.act, v));
          if (args.residual) v += Elem<T>::load(reinterpret_cast<const T*>(args.residual), row * args.ld_res + col);
          Elem<T>::store(Cp_, row * args.ldc + col, v);
        } else if constexpr (EPI == EPI_GEMM) {
          v *= args.alpha;
          if (args.c_in) {
            const float base = Elem<T>::round_trip(
                args.beta * Elem<T>::load(reinterpret_cast<const T*>(args.c_in),
                                          bz * args.stride_c_in + row * args.c_in_rs + col * args.c_in_cs));
            v = base + v;
          }
          Elem<T>::store(Cp_, bz * args.stride_c + row * args.ldc + col, v);
        } else {
          const int64_t OHW = args.OH * args.OW;
          if (args.bias) v += Elem<T>::load(reinterpret_cast<const T*>(args.bias), row);
          const int64_t addr = conv_base + row * OHW;
          if (args.residual) {
            v = Elem<T>::round_trip(v);
            v += Elem<T>::load(reinterpret_cast<const T*>(args.residual), addr);
          }
          Elem<T>::store(Cp_, addr, v);
        }
      }
    }
  }
}

}  // namespace mthip
