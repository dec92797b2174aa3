// MFMA GEMM core for gfx950, shared by linear/matmul/addmm (gemm.hip) and the implicit-GEMM
// conv2d (conv.hip).
//
//   C[m, n] = sum_k A[m, k] * B[n, k]      (both operands staged k-contiguous in LDS)
//
// A workgroup is 4 wave64s computing a BM x BN tile; each wave owns a (BM/WGM) x (BN/WGN)
// sub-tile made of 32x32 MFMA fragments.  fp16 uses v_mfma_f32_32x32x16_f16 (fp32 accumulate),
// fp32 uses v_mfma_f32_32x32x2f32.  The MFMA is issued as D = B-fragment x A-fragment, i.e. it
// computes C^T: a lane's accumulator then holds one row m of C and, per group of four
// registers, four consecutive columns n -- the memory-contiguous direction of every output
// here -- so results leave in 8/16-byte stores.
//
// K advances in BK-wide tiles through two LDS buffers fed by two register stages: the global
// loads of tile k+2 are issued before the MFMAs of tile k, tile k+1 (requested one tile
// earlier) is written to the other LDS buffer after them, and one barrier per tile suffices.
// Loads are range-checked buffer loads from precomputed per-thread offsets; the implicit
// im2col of the conv mode derives the (ky, kx, channel) of a tile once per tile (uniform
// across the workgroup) when the padded channel count is a multiple of BK.
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
  static constexpr int BK = 64;
  // acc += rowfrag(p) x colfrag(q): p supplies the MFMA's A (output rows i), q its B (cols j).
  static __device__ __forceinline__ floatx16 fma(const uint16_t* p, const uint16_t* q, int kk, int lane, floatx16 acc) {
    const halfx8 a = *reinterpret_cast<const halfx8*>(p + kk + (lane >> 5) * 8);
    const halfx8 b = *reinterpret_cast<const halfx8*>(q + kk + (lane >> 5) * 8);
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int KI = 2;
  static constexpr int VEC = 4;
  static constexpr int PAD = 4;
  static constexpr int BK = 32;
  static __device__ __forceinline__ floatx16 fma(const float* p, const float* q, int kk, int lane, floatx16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(p[kk + (lane >> 5)], q[kk + (lane >> 5)], acc, 0, 0, 0);
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
  // Extent (bytes) of the A and B buffers as seen from one batch's base; buffer loads beyond
  // it return zeros.  Must stay below 2^31.
  int64_t a_bytes, b_bytes;
};

// Narrowed store of 4 consecutive outputs (8 bytes fp16 / 16 bytes fp32) when aligned.
template <typename T>
__device__ __forceinline__ void store4(T* p, const float v[4], bool vec) {
  if (vec) {
    if constexpr (sizeof(T) == 2) {
      uint2 u;
      u.x = (uint32_t)f2h_fast(v[0]) | ((uint32_t)f2h_fast(v[1]) << 16);
      u.y = (uint32_t)f2h_fast(v[2]) | ((uint32_t)f2h_fast(v[3]) << 16);
      *reinterpret_cast<uint2*>(p) = u;
    } else {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) Elem<T>::store(p, j, v[j]);
  }
}

template <typename T, int BM, int BN, int WGM, int MODE, int EPI, bool CONV_FAST>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmArgs args) {
  constexpr int BK = Mfma<T>::BK;
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
  static_assert(MODE != MODE_NN || B_CH_NN >= 1, "tile too small for the NN loader");

  __shared__ __align__(16) T As[2][BM * LDK];
  __shared__ __align__(16) T Bs[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int64_t bz = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int kc = (tid % CH_PER_ROW) * VEC;  // k offset of this thread's chunks within a tile

  // ---- per-thread loader state ------------------------------------------------------
  // Every global read is a buffer load whose byte offset is either the chunk's address or
  // kOOB: the buffer's range check returns zeros for the latter, so rows past M/N, chunks past
  // K and the conv's padding taps need no branches (a branch here makes the compiler wait for
  // every outstanding load before the LDS stores, serialising the prefetch).
  constexpr uint32_t kOOB = 0x80000000u;
  constexpr int ES = (int)sizeof(T);
  const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<const T*>(args.a) + bz * args.stride_a), (short)0, (int)args.a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<const T*>(args.b) + (MODE == MODE_CONV ? 0 : bz * args.stride_b)), (short)0,
      (int)args.b_bytes, 0x00020000);
  uint32_t a_off[A_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int64_t row = m0 + (tid + i * 256) / CH_PER_ROW;
    a_off[i] = row < args.M ? (uint32_t)((row * args.lda + kc) * ES) : kOOB;
  }
  uint32_t b_off[MODE == MODE_NN ? 1 : B_CH];
  int conv_iy[MODE == MODE_CONV ? B_CH : 1], conv_ix[MODE == MODE_CONV ? B_CH : 1];
  if constexpr (MODE == MODE_NT) {
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int64_t row = n0 + (tid + i * 256) / CH_PER_ROW;
      b_off[i] = row < args.N ? (uint32_t)((row * args.ldb + kc) * ES) : kOOB;
    }
  } else if constexpr (MODE == MODE_CONV) {
    const int64_t OHW = args.OH * args.OW;
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int64_t p = n0 + (tid + i * 256) / CH_PER_ROW;
      const bool ok = p < args.N;
      const int64_t pp = ok ? p : 0;
      const int64_t img = pp / OHW, pix = pp - img * OHW;
      const int oy = (int)(pix / args.OW), ox = (int)(pix - (pix / args.OW) * args.OW);
      // rows past N get an origin no tap can reach, so every tap tests out of bounds
      conv_iy[i] = ok ? oy * (int)args.sh - (int)args.ph : -(1 << 28);
      conv_ix[i] = ox * (int)args.sw - (int)args.pw;
      // element offset of x_nhwc[img, iy0, ix0, kc] (iy0/ix0 may lie in the padding; only
      // in-bounds taps are ever turned into a real offset)
      b_off[i] = (uint32_t)((((img * args.H) * args.W) * args.Cp) + kc);
    }
  }

  constexpr int NRB = MODE == MODE_NN ? B_CH_NN : B_CH;
  // Two register stages: tile k+2 is requested while tile k is multiplied, so every global
  // load has two tiles of MFMA work (plus a barrier) to arrive.
  uint4 ra0[A_CH], rb0[NRB], ra1[A_CH], rb1[NRB];

  auto bload = [&](const __amdgpu_buffer_rsrc_t& r, uint32_t off) -> uint4 {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
  };

  auto load_tiles = [&](int64_t k0, uint4(&ra)[A_CH], uint4(&rb)[NRB]) {
    const bool kin = k0 + kc < args.K;  // K % VEC == 0: a chunk is entirely in or out
    const uint32_t kb = (uint32_t)(k0 * ES);
#pragma unroll
    for (int i = 0; i < A_CH; ++i) ra[i] = bload(a_rsrc, (kin && a_off[i] != kOOB) ? a_off[i] + kb : kOOB);
    if constexpr (MODE == MODE_NT) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) rb[i] = bload(b_rsrc, (kin && b_off[i] != kOOB) ? b_off[i] + kb : kOOB);
    } else if constexpr (MODE == MODE_NN) {
#pragma unroll
      for (int i = 0; i < B_CH_NN; ++i) {
        const int c = tid + i * 256;
        const int64_t k = k0 + c / NB_CH_ROW, n = n0 + (c % NB_CH_ROW) * VEC;
        const bool ok = k < args.K && n < args.N;  // N % VEC == 0: chunks are whole
        rb[i] = bload(b_rsrc, ok ? (uint32_t)((k * args.ldb + n) * ES) : kOOB);
      }
    } else {
      // Implicit im2col: k = (ky*KW + kx)*Cp + ch.  With Cp % BK == 0 a tile never straddles
      // two taps, so (ky, kx, ch0) are uniform across the workgroup for the whole tile.
      const int W = (int)args.W, H = (int)args.H, Cp = (int)args.Cp, KW = (int)args.KW;
      int tap, ch;
      if constexpr (CONV_FAST) {
        tap = (int)k0 / Cp;
        ch = (int)k0 - tap * Cp;  // + kc, already folded into b_off
      } else {
        const int k = (int)k0 + kc;
        tap = k / Cp;
        ch = k - tap * Cp - kc;
      }
      const int ky = tap / KW, kx = tap - (tap / KW) * KW;
      const int dy = ky * (int)args.dh, dx = kx * (int)args.dw;
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int iy = conv_iy[i] + dy, ix = conv_ix[i] + dx;
        const bool ok = kin && iy >= 0 && iy < H && ix >= 0 && ix < W;
        const uint32_t off = (b_off[i] + (uint32_t)((iy * W + ix) * Cp + ch)) * (uint32_t)ES;
        rb[i] = bload(b_rsrc, ok ? off : kOOB);
      }
    }
  };

  auto store_tiles = [&](int buf, const uint4(&ra)[A_CH], const uint4(&rb)[NRB]) {
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
  auto compute = [&](int buf) {
    const T* a_base = &As[buf][(wm * WM + (lane & 31)) * LDK];
    const T* b_base = &Bs[buf][(wn * WN + (lane & 31)) * LDK];
#pragma unroll
    for (int kk = 0; kk < BK; kk += Mfma<T>::KI) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = Mfma<T>::fma(b_base + j * 32 * LDK, a_base + i * 32 * LDK, kk, lane, acc[i][j]);
    }
  };
  load_tiles(0, ra0, rb0);
  if (nk > 1) load_tiles(BK, ra1, rb1);
  store_tiles(0, ra0, rb0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; kt += 2) {
    // even tile kt in buffer 0; tile kt+1 is landing in stage 1
    if (kt + 2 < nk) load_tiles((kt + 2) * BK, ra0, rb0);
    compute(0);
    if (kt + 1 < nk) store_tiles(1, ra1, rb1);
    __syncthreads();
    if (kt + 1 >= nk) break;
    // odd tile kt+1 in buffer 1; tile kt+2 is landing in stage 0
    if (kt + 3 < nk) load_tiles((kt + 3) * BK, ra1, rb1);
    compute(1);
    if (kt + 2 < nk) store_tiles(0, ra0, rb0);
    __syncthreads();
  }

  // ---- epilogue.  Fragment (i, j), register r of lane l holds C[row][col] with
  //      row = m0 + wm*WM + i*32 + l%32,
  //      col = n0 + wn*WN + j*32 + 8*(r/4) + 4*(l/32) + r%4     (4 consecutive cols per r/4).
  // Values are narrowed once, except where a fused activation or residual needs the narrowed
  // intermediate the unfused op sequence would have produced.
  T* Cptr = reinterpret_cast<T*>(args.c);
  const int M = (int)args.M, N = (int)args.N;
  const int lane_col = 4 * (lane >> 5);
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int row = (int)m0 + wm * WM + i * 32 + (lane & 31);
    if (row >= M) continue;
    if constexpr (EPI == EPI_LINEAR) {
      const T* bias = reinterpret_cast<const T*>(args.bias);
      const T* res = args.residual ? reinterpret_cast<const T*>(args.residual) + (int64_t)row * args.ld_res : nullptr;
      T* crow = Cptr + (int64_t)row * args.ldc;
      const bool plain = args.act == 0 && res == nullptr;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col0 = (int)n0 + wn * WN + j * 32 + 8 * g + lane_col;
          if (col0 >= N) continue;
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = acc[i][j][4 * g + t];
          if (col0 + 4 <= N) {
            if (bias) {
#pragma unroll
              for (int t = 0; t < 4; ++t) v[t] += Elem<T>::load(bias, col0 + t);
            }
            if (!plain) {
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                float x = Elem<T>::round_trip(v[t]);
                if (args.act) x = apply_act<T>(args.act, x);
                if (res) x = Elem<T>::round_trip(x) + Elem<T>::load(res, col0 + t);
                v[t] = x;
              }
            }
            store4<T>(crow + col0, v, ((uintptr_t)(crow + col0) & (4 * sizeof(T) - 1)) == 0);
          } else {
            for (int t = 0; t < 4 && col0 + t < N; ++t) {
              float x = v[t];
              if (bias) x += Elem<T>::load(bias, col0 + t);
              if (!plain) {
                x = Elem<T>::round_trip(x);
                if (args.act) x = apply_act<T>(args.act, x);
                if (res) x = Elem<T>::round_trip(x) + Elem<T>::load(res, col0 + t);
              }
              Elem<T>::store(crow, col0 + t, x);
            }
          }
        }
      }
    } else if constexpr (EPI == EPI_GEMM) {
      const T* cin = reinterpret_cast<const T*>(args.c_in);
      T* crow = Cptr + bz * args.stride_c + (int64_t)row * args.ldc;
      const T* cinrow = cin ? cin + bz * args.stride_c_in + (int64_t)row * args.c_in_rs : nullptr;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col0 = (int)n0 + wn * WN + j * 32 + 8 * g + lane_col;
          if (col0 >= N) continue;
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float x = acc[i][j][4 * g + t] * args.alpha;
            if (cinrow && col0 + t < N)
              x = Elem<T>::round_trip(args.beta * Elem<T>::load(cinrow, (int64_t)(col0 + t) * args.c_in_cs)) + x;
            v[t] = x;
          }
          if (col0 + 4 <= N) {
            store4<T>(crow + col0, v, ((uintptr_t)(crow + col0) & (4 * sizeof(T) - 1)) == 0);
          } else {
            for (int t = 0; t < 4 && col0 + t < N; ++t) Elem<T>::store(crow, col0 + t, v[t]);
          }
        }
      }
    } else {
      // conv: row = output channel, col = output pixel (image-major); NCHW store.
      const int OHW = (int)(args.OH * args.OW);
      const T* bias = reinterpret_cast<const T*>(args.bias);
      const T* res = reinterpret_cast<const T*>(args.residual);
      const float bv = bias ? Elem<T>::load(bias, row) : 0.0f;
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        // A fragment's 32 pixels lie in one image when OHW is a multiple of 32 (every SD
        // level); one division per fragment then addresses all of them.
        const int frag0 = (int)n0 + wn * WN + j * 32;
        if (frag0 >= N) continue;
        if (OHW % 32 == 0) {
          const int img = frag0 / OHW;
          const int64_t base = ((int64_t)img * M + row) * OHW + (frag0 - img * OHW) + lane_col;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            if (frag0 + 8 * g + lane_col >= N) continue;
            float v[4];
            const int64_t addr = base + 8 * g;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              float x = acc[i][j][4 * g + t] + bv;
              if (res) x = Elem<T>::round_trip(x) + Elem<T>::load(res, addr + t);
              v[t] = x;
            }
            store4<T>(Cptr + addr, v, ((uintptr_t)(Cptr + addr) & (4 * sizeof(T) - 1)) == 0);
          }
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            for (int t = 0; t < 4; ++t) {
              const int c = frag0 + 8 * g + lane_col + t;
              if (c >= N) break;
              const int im = c / OHW, px = c - im * OHW;
              const int64_t addr = ((int64_t)im * M + row) * OHW + px;
              float x = acc[i][j][4 * g + t] + bv;
              if (res) x = Elem<T>::round_trip(x) + Elem<T>::load(res, addr);
              Elem<T>::store(Cptr, addr, x);
            }
          }
        }
      }
    }
  }
}

}  // namespace mthip
