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
// Work decomposition.  The problem is cut into units = (batch, K slice, output tile).  The
// grid is persistent (about one wave of resident workgroups); workgroup w takes units w,
// w + G, w + 2G, ...  and treats its units' K tiles as one flat stream: the global loads of
// step s+2 are issued while step s is multiplied, also across unit boundaries, so a unit's
// first tiles arrive while the previous unit is still computing and storing.  (SD shapes have
// K = 320..2560, i.e. 5..40 K tiles per unit: without this the load latency at each unit's
// start dominates.)  Units are numbered so that each XCD (workgroups are dealt to the 8 XCDs
// round-robin) walks a contiguous run of output tiles, which share A rows in its L2.
//
// K advances in BK-wide tiles through two LDS buffers fed by two register stages; one barrier
// per step suffices.  Loads are range-checked buffer loads from precomputed per-thread
// offsets.  The implicit im2col of the conv mode, when the padded channel count is a multiple
// of BK (a tile never straddles two filter taps) and the filter has <= 32 taps, keeps per
// output pixel the offset of tap (0, 0) and a bitmask of the taps inside the image (both set
// once per unit) and steps the tile's (tap, ky, kx, channel) with counters, so a chunk costs a
// bit test and one add per tile.
//
// When the output tiles alone cannot fill the chip and K is long (the 1280-channel convs at
// 8x8 and 16x16), K is split into slices whose fp32 partial tiles go to a workspace;
// gemm_splitk_reduce_kernel then sums the slices in a fixed order and applies the epilogue.
//
// The B operand has three sources (MODE): a k-contiguous [N, K] matrix (linear weights, x.W^T),
// an n-contiguous [K, N] matrix (matmul; transposed while staging), or an implicit im2col of an
// NHWC activation (conv2d).  The epilogue (EPI) applies the op-specific tail and narrows with
// mtorch's fp16 rounding.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "activations.h"
#include "common.h"

namespace mthip {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

enum { MODE_NT = 0, MODE_NN = 1, MODE_CONV = 2 };
enum { EPI_LINEAR = 0, EPI_GEMM = 1, EPI_CONV = 2, EPI_GEGLU = 3 };

template <typename T>
struct Mfma;

template <>
struct Mfma<uint16_t> {
  static constexpr int KI = 16;  // k consumed per MFMA
  static constexpr int VEC = 8;  // elements per 16-byte global chunk
  static constexpr int PAD = 8;  // LDS row padding (elements) against bank conflicts
  static constexpr int BK = 64;
  typedef halfx8 Frag;
  // This lane's operand fragment of a 32-row LDS block at k offset kk.
  static __device__ __forceinline__ Frag load(const uint16_t* p, int kk, int lane) {
    return *reinterpret_cast<const halfx8*>(p + kk + (lane >> 5) * 8);
  }
  // acc += a x b, a supplying the MFMA's A (output rows), b its B (output cols).
  static __device__ __forceinline__ floatx16 mma(const Frag& a, const Frag& b, floatx16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int KI = 2;
  static constexpr int VEC = 4;
  static constexpr int PAD = 4;
  static constexpr int BK = 32;
  typedef float Frag;
  static __device__ __forceinline__ Frag load(const float* p, int kk, int lane) { return p[kk + (lane >> 5)]; }
  static __device__ __forceinline__ floatx16 mma(const Frag& a, const Frag& b, floatx16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
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
  int64_t KH_;  // filter height (CONV_FAST tap masks)
  // Extent (bytes) of the A and B buffers as seen from one batch's base; buffer loads beyond
  // it return zeros.  Must stay below 2^31.
  int64_t a_bytes, b_bytes;
  // Work decomposition, filled by the launcher (gemm.hip).
  int64_t tiles_m, tiles_n;  // output tiles per batch
  int64_t ksplit;            // K slices per output tile (1: no split)
  int64_t kt_per_split;      // K tiles per slice (the last slice may hold fewer)
  int64_t units;             // batch * ksplit * tiles_m * tiles_n
  float* partial;            // ksplit > 1: fp32 slices [ksplit][M][ld_partial]
  int64_t ld_partial;        // N rounded up to a multiple of 4
  // Divisors of the index arithmetic (units, pixels and N stay below 2^31).
  FastDiv div_tiles_n, div_tiles_m, div_ksplit, div_ohw, div_ow;
  int xcd_remap;  // 1: number units XCD-contiguously (see decode_unit)
  int m_fast;     // 1: consecutive units walk the M tiles of one N tile (else the N tiles of one M tile)
  // EPI_GEGLU: gelu of every fp16 value (65536 entries, mtorch's fp16 gelu bit for bit)
  const uint16_t* gelu_tab;
  // EPI_CONV: per-(image, output channel) addend chan_add[img * chan_add_ld + row] (an SD
  // ResNet block's time embedding), added after the bias and before the residual
  const void* chan_add;
  int64_t chan_add_ld;
};

// v as the unfused op sequence reads it back after storing it in T, for the general epilogue
// paths (partial tiles, the split-K reduction, fp32); the straight-line fp16 tile epilogues use
// epi_chain_h with f2h_nonnan instead.
template <typename T>
__device__ __forceinline__ float epi_round(float v) {
  if constexpr (sizeof(T) == 2) {
    return h2f_bits(f2h_generic(v));
  } else {
    return v;
  }
}

// Stores the first nv (1..4) of 4 consecutive outputs, narrowed once each; one 8-byte (fp16)
// or 16-byte (fp32) store when all four are valid and aligned.
template <typename T>
__device__ __forceinline__ void store_cols(T* p, const float (&v)[4], int nv) {
  if constexpr (sizeof(T) == 2) {
    uint32_t h[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) h[t] = f2h_generic(v[t]);
    if (nv == 4 && ((uintptr_t)p & 7) == 0) {
      *reinterpret_cast<uint2*>(p) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (t < nv) p[t] = (uint16_t)h[t];
    }
  } else {
    if (nv == 4 && ((uintptr_t)p & 15) == 0) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (t < nv) p[t] = v[t];
    }
  }
}

// Reads the first nv (1..4) of 4 consecutive elements as floats (0 past nv); one 8-byte (fp16)
// or 16-byte (fp32) load when all four are valid and aligned.
template <typename T>
__device__ __forceinline__ void load_cols(const T* p, float (&o)[4], int nv) {
  if constexpr (sizeof(T) == 2) {
    if (nv == 4 && ((uintptr_t)p & 7) == 0) {
      const uint2 u = *reinterpret_cast<const uint2*>(p);
      o[0] = h2f_bits((uint16_t)(u.x & 0xffffu));
      o[1] = h2f_bits((uint16_t)(u.x >> 16));
      o[2] = h2f_bits((uint16_t)(u.y & 0xffffu));
      o[3] = h2f_bits((uint16_t)(u.y >> 16));
      return;
    }
  } else {
    if (nv == 4 && ((uintptr_t)p & 15) == 0) {
      const float4 u = *reinterpret_cast<const float4*>(p);
      o[0] = u.x;
      o[1] = u.y;
      o[2] = u.z;
      o[3] = u.w;
      return;
    }
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = t < nv ? Elem<T>::load(p, t) : 0.0f;
}

// Four consecutive stored elements, read with one 8-byte (fp16) or 16-byte (fp32) load and kept
// packed until used.
template <typename T>
struct Raw4;
template <>
struct Raw4<uint16_t> {
  uint2 u;
  __device__ __forceinline__ float at(int t) const {
    const uint32_t w = t < 2 ? u.x : u.y;
    return h2f_bits((uint16_t)((t & 1) ? (w >> 16) : (w & 0xffffu)));
  }
};
template <>
struct Raw4<float> {
  float4 u;
  __device__ __forceinline__ float at(int t) const { return t == 0 ? u.x : t == 1 ? u.y : t == 2 ? u.z : u.w; }
};
// p must be aligned to the load (8 bytes for fp16, 16 for fp32).
template <typename T>
__device__ __forceinline__ Raw4<T> load_raw4(const T* p) {
  Raw4<T> r;
  if constexpr (sizeof(T) == 2) {
    r.u = *reinterpret_cast<const uint2*>(p);
  } else {
    r.u = *reinterpret_cast<const float4*>(p);
  }
  return r;
}

// The epilogue arithmetic on operands already read: b is the per-column bias (EPI_LINEAR) or
// the row's bias in every slot (EPI_CONV, 0 without a bias), av the channel addend (EPI_CONV),
// r the residual.  Values are narrowed once, except where a fused activation or residual needs
// the narrowed intermediate that the unfused op sequence would have produced.
// gtab: the fp16 gelu of every half value (ACT_GELU on fp16 only; unused otherwise): the
// activation of the narrowed linear output is looked up by its bits -- the table holds exactly
// what evaluating it gives -- instead of a double-precision erf per element.
template <typename T, int EPI, int ACT>
__device__ __forceinline__ void epi_math(float (&v)[4], const float (&b)[4], bool has_b, float av, bool has_av,
                                         const float (&r)[4], bool has_r, const uint16_t* gtab = nullptr) {
  if constexpr (EPI == EPI_LINEAR) {
    if (has_b) {
#pragma unroll
      for (int t = 0; t < 4; ++t) v[t] += b[t];
    }
    if constexpr (ACT == MTHIP_ACT_GELU && sizeof(T) == 2) {
      uint32_t g[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) g[t] = gtab[f2h_generic(v[t])];  // every gather before the first use
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float x = h2f_bits(g[t]);
        if (has_r) x += r[t];
        v[t] = x;
      }
    } else if (ACT != MTHIP_ACT_NONE || has_r) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float x = epi_round<T>(v[t]);
        if constexpr (ACT != MTHIP_ACT_NONE) x = apply_act<T>(ACT, x);
        if (has_r) x = epi_round<T>(x) + r[t];
        v[t] = x;
      }
    }
  } else if constexpr (EPI == EPI_CONV) {
    // conv + bias, then (+ chan_add), then (+ residual), each add narrowed as the unfused op
    // sequence narrows it
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float x = v[t] + b[t];
      if (has_av) x = epi_round<T>(x) + av;
      if (has_r) x = epi_round<T>(x) + r[t];
      v[t] = x;
    }
  }
}

// fp16 narrowings of the straight-line epilogues.  NarrowFast is exact for every non-NaN value
// (f2h_nonnan, ~10 VALU operations) and records whether a NaN went through it; a wave that met
// one computes its values again with NarrowExact (f2h_generic: NaN payloads as mtorch keeps
// them).
struct NarrowFast {
  bool nan = false;
  __device__ __forceinline__ uint32_t operator()(float x) {
    nan |= x != x;
    return f2h_nonnan(x);
  }
};
struct NarrowExact {
  __device__ __forceinline__ uint32_t operator()(float x) const { return f2h_generic(x); }
};

// One fp16 output of EPI_LINEAR / EPI_CONV from its fp32 dot product x: + b (the bias, or -0.0,
// which leaves every value as it is), then the activation (LINEAR) or the channel addend
// (CONV, HA), then the residual (HR), each narrowed where the unfused op sequence stores it.
template <int EPI, int ACT, bool HA, bool HR, typename N>
__device__ __forceinline__ uint32_t epi_chain_h(float x, float b, float av, float r, const uint16_t* gtab, N& narrow) {
  x += b;
  if constexpr (EPI == EPI_LINEAR && ACT == MTHIP_ACT_GELU) {
    const uint32_t g = gtab[narrow(x)];
    if constexpr (!HR) return g;
    x = h2f_bits((uint16_t)g) + r;
  } else if constexpr (EPI == EPI_LINEAR && ACT != MTHIP_ACT_NONE) {
    x = apply_act<uint16_t>(ACT, h2f_bits((uint16_t)narrow(x)));
    if constexpr (HR) x = h2f_bits((uint16_t)narrow(x)) + r;
  } else {
    if constexpr (HA) x = h2f_bits((uint16_t)narrow(x)) + av;
    if constexpr (HR) x = h2f_bits((uint16_t)narrow(x)) + r;
  }
  return narrow(x);
}

// Epilogue for C[row][col0 .. col0+3] of batch bz (row < M checked by the caller; columns
// past N are skipped).  v holds the fp32 dot products.  Values are narrowed once, except where
// a fused activation or residual needs the narrowed intermediate that the unfused op sequence
// would have produced.  ACT (EPI_LINEAR only) is the fused activation, fixed at compile time.
template <typename T, int EPI, int ACT>
__device__ __forceinline__ void emit4(const GemmArgs& args, int64_t bz, int row, int col0, float (&v)[4]) {
  const int N = (int)args.N;
  if (col0 >= N) return;
  const int nv = N - col0 < 4 ? N - col0 : 4;  // valid columns (1..4)
  T* Cptr = reinterpret_cast<T*>(args.c);
  if constexpr (EPI == EPI_LINEAR) {
    const T* bias = reinterpret_cast<const T*>(args.bias);
    const T* res = args.residual ? reinterpret_cast<const T*>(args.residual) + (int64_t)row * args.ld_res : nullptr;
    float b[4] = {0.0f, 0.0f, 0.0f, 0.0f}, r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (bias) load_cols<T>(bias + col0, b, nv);
    if (res) load_cols<T>(res + col0, r, nv);
    epi_math<T, EPI, ACT>(v, b, bias != nullptr, 0.0f, false, r, res != nullptr, args.gelu_tab);
    store_cols<T>(Cptr + (int64_t)row * args.ldc + col0, v, nv);
  } else if constexpr (EPI == EPI_GEMM) {
    const T* cin = reinterpret_cast<const T*>(args.c_in);
    const T* cinrow = cin ? cin + bz * args.stride_c_in + (int64_t)row * args.c_in_rs : nullptr;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float x = v[t] * args.alpha;
      if (cinrow && t < nv)
        x = epi_round<T>(args.beta * Elem<T>::load(cinrow, (int64_t)(col0 + t) * args.c_in_cs)) + x;
      v[t] = x;
    }
    store_cols<T>(Cptr + bz * args.stride_c + (int64_t)row * args.ldc + col0, v, nv);
  } else {
    // conv: row = output channel, col = output pixel (image-major); NCHW store.
    const int M = (int)args.M;
    const int OHW = (int)(args.OH * args.OW);
    const T* bias = reinterpret_cast<const T*>(args.bias);
    const T* res = reinterpret_cast<const T*>(args.residual);
    const T* cadd = reinterpret_cast<const T*>(args.chan_add);
    const float bv = bias ? Elem<T>::load(bias, row) : 0.0f;
    if (OHW % 4 == 0) {
      // col0 is a multiple of 4, so the 4 pixels lie in one image and are contiguous.
      const int img = (int)args.div_ohw.div((uint32_t)col0);
      const int64_t addr = ((int64_t)img * M + row) * OHW + (col0 - img * OHW);
      const float av = cadd ? Elem<T>::load(cadd, img * args.chan_add_ld + row) : 0.0f;
      const float b[4] = {bv, bv, bv, bv};
      float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (res) load_cols<T>(res + addr, r, nv);
      epi_math<T, EPI, ACT>(v, b, true, av, cadd != nullptr, r, res != nullptr);
      store_cols<T>(Cptr + addr, v, nv);
    } else {
      for (int t = 0; t < nv; ++t) {
        const int c = col0 + t;
        const int im = (int)args.div_ohw.div((uint32_t)c), px = c - im * OHW;
        const int64_t addr = ((int64_t)im * M + row) * OHW + px;
        float x = v[t] + bv;
        if (cadd) x = epi_round<T>(x) + Elem<T>::load(cadd, im * args.chan_add_ld + row);
        if (res) x = epi_round<T>(x) + Elem<T>::load(res, addr);
        Elem<T>::store(Cptr, addr, x);
      }
    }
  }
}

// One unit of work: an output tile of one batch over one K slice.
struct GemmUnit {
  int64_t m0, n0, bz;
  int64_t split;  // K slice index
  int64_t kt0;    // first K tile
  int64_t nkt;    // K tiles in this slice (>= 1)
};

template <int BM, int BN>
__device__ __forceinline__ GemmUnit decode_unit(const GemmArgs& args, uint32_t u, uint32_t nk_total) {
  // XCD-contiguous numbering: workgroups w = x (mod 8) run on XCD x and take units u = x (mod 8)
  // (the grid size is a multiple of 8).  Remapping q = (u % 8) * (U / 8) + u / 8 hands XCD x the
  // contiguous range [x*U/8, (x+1)*U/8) of tiles; the U % 8 tail keeps q = u (a bijection).
  // Within the range the smaller tile dimension varies fastest (m_fast when M has fewer tiles),
  // so an XCD holds a band of the large operand and all of the small one in its L2, and a
  // conv's neighbouring pixel tiles, which share 3x3 halo rows, run on the same XCD.
  const uint32_t U = (uint32_t)args.units, U8 = U / 8;
  const uint32_t q = (args.xcd_remap && u < 8 * U8) ? (u % 8) * U8 + u / 8 : u;
  uint32_t tm, tn, t2;
  if (args.m_fast) {
    const uint32_t t1 = args.div_tiles_m.div(q);
    tm = q - t1 * args.div_tiles_m.d;
    t2 = args.div_tiles_n.div(t1);
    tn = t1 - t2 * args.div_tiles_n.d;
  } else {
    const uint32_t t1 = args.div_tiles_n.div(q);
    tn = q - t1 * args.div_tiles_n.d;
    t2 = args.div_tiles_m.div(t1);
    tm = t1 - t2 * args.div_tiles_m.d;
  }
  const uint32_t bz = args.div_ksplit.div(t2);
  GemmUnit un;
  un.split = t2 - bz * args.div_ksplit.d;
  un.bz = bz;
  un.m0 = (int64_t)tm * BM;
  un.n0 = (int64_t)tn * BN;
  un.kt0 = un.split * args.kt_per_split;
  const int64_t left = (int64_t)nk_total - un.kt0;
  un.nkt = left < args.kt_per_split ? left : args.kt_per_split;
  if (un.nkt < 1) un.nkt = 1;  // K == 0: one all-zero step, so the unit still gets its epilogue
  return un;
}

// Whether a unit's EPI_LINEAR / EPI_CONV epilogue can take the straight-line path: every column
// of the tile exists, bias and residual rows are aligned to 4-element loads and (conv) the tile's
// pixels lie in one image.  The test is uniform across the workgroup.
template <typename T, int EPI, int BN>
__device__ __forceinline__ bool epi_tile_fast(const GemmArgs& args, const GemmUnit& un) {
  constexpr uintptr_t kAlign = sizeof(T) == 2 ? 7 : 15;
  if (un.n0 + BN > args.N) return false;
  if constexpr (EPI == EPI_LINEAR) {
    if (args.bias && ((uintptr_t)args.bias & kAlign)) return false;
    if (args.residual && (((uintptr_t)args.residual & kAlign) || (args.ld_res & 3))) return false;
    return true;
  } else if constexpr (EPI == EPI_CONV) {
    const int64_t OHW = args.OH * args.OW;
    if (OHW % 4) return false;
    if (args.div_ohw.div((uint32_t)un.n0) != args.div_ohw.div((uint32_t)(un.n0 + BN - 1))) return false;
    if (args.residual && ((uintptr_t)args.residual & kAlign)) return false;
    return true;
  } else {
    return false;
  }
}

// Epilogue of one unit.  Fragment (i, j), register r of lane l holds
//   C[row][col], row = m0 + wm*WM + i*32 + l%32,
//   col = n0 + wn*WN + j*32 + 8*(r/4) + 4*(l/32) + r%4     (4 consecutive cols per r/4),
// with (wm, wn) the wave's position in the workgroup's WGM x (4/WGM) grid of wave tiles.
//
// Every read of an epilogue is issued before its first use.  A load's result is waited for
// where it is used and the wait counter drains in issue order, behind the next unit's operand
// loads already in flight: reads interleaved with their uses would each pay that wait, reads
// issued together share one.
template <typename T, int BM, int BN, int WGM, int EPI, int ACT, int FM, int FN>
__device__ __forceinline__ void gemm_finish_unit(const GemmArgs& args, const GemmUnit& un, floatx16 (&acc)[FM][FN],
                                                 int lane, int wm, int wn) {
  constexpr int WGN = 4 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  static_assert(FM == WM / 32 && FN == WN / 32, "fragment grid");
  const int lane_col = 4 * (lane >> 5);
  const int M = (int)args.M;
  if constexpr (EPI == EPI_GEGLU) {
    // B rows come interleaved in 32-row blocks (values, then the matching gates), and each
    // wave owns 64 columns = fragment 0 (values) + fragment 1 (gates) of 32 output columns:
    // out[row][col] = value * gelu(gate), each factor narrowed as the unfused
    // linear -> chunk -> gelu -> mul sequence narrows it.  N is a multiple of 64 (the launcher
    // requires 32 output columns per block), so a wave's 64 columns exist whole or not at all.
    static_assert(FN == 2 && WN == 64, "GEGLU epilogue pairs two 32-column fragments");
    const T* bias = reinterpret_cast<const T*>(args.bias);
    T* Cp = reinterpret_cast<T*>(args.c);
    const int Nout = (int)args.N / 2;
    const int n0 = (int)un.n0 + wn * WN;  // the wave's first (permuted) column
    if (n0 >= (int)args.N) return;
    const bool has_b = bias != nullptr;
    float bval[4][4], bgate[4][4];
    if (has_b && ((uintptr_t)bias & (sizeof(T) == 2 ? 7 : 15)) == 0) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int pc = n0 + 8 * g + lane_col;  // permuted column of the value
        const Raw4<T> bv = load_raw4<T>(bias + pc), bg = load_raw4<T>(bias + pc + 32);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          bval[g][t] = bv.at(t);
          bgate[g][t] = bg.at(t);
        }
      }
    } else if (has_b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int pc = n0 + 8 * g + lane_col;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          bval[g][t] = Elem<T>::load(bias, pc + t);
          bgate[g][t] = Elem<T>::load(bias, pc + 32 + t);
        }
      }
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int t = 0; t < 4; ++t) bval[g][t] = bgate[g][t] = -0.0f;  // adding -0.0 leaves every value as it is
    }
    if constexpr (sizeof(T) == 2) {
      // out = value * gelu(gate): the gate narrowed and looked up, the value narrowed, their
      // product narrowed; every gather of a row before the first use
      uint2 out[FM][4];
      // Every narrowing with f2h_rtz_* (the gate pairwise before its two table gathers, the
      // value's narrowed pair multiplied by the gelu halves inside v_fma_mix_f32), under a
      // running maximum of |value|; a wave that met a NaN, an infinity or |value| >= 65520
      // redoes its outputs with f2h_nonnan, and with f2h_generic if one was NaN.
      float amax = 0.0f;
      auto npair = [&](float a, float b) {
        amax = abs_max_nan(abs_max_nan(amax, a), b);
        return f2h_rtz_pack(a, b);
      };
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        uint32_t gh[4][4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const uint32_t p = npair(acc[i][1][4 * g + 2 * q] + bgate[g][2 * q], acc[i][1][4 * g + 2 * q + 1] + bgate[g][2 * q + 1]);
            gh[g][2 * q] = args.gelu_tab[p & 0xffffu];
            gh[g][2 * q + 1] = args.gelu_tab[p >> 16];
          }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t v01 = npair(acc[i][0][4 * g] + bval[g][0], acc[i][0][4 * g + 1] + bval[g][1]);
          const uint32_t v23 = npair(acc[i][0][4 * g + 2] + bval[g][2], acc[i][0][4 * g + 3] + bval[g][3]);
          out[i][g] = make_uint2(npair(mul_halves<false, false>(v01, gh[g][0]), mul_halves<true, false>(v01, gh[g][1])),
                                 npair(mul_halves<false, false>(v23, gh[g][2]), mul_halves<true, false>(v23, gh[g][3])));
        }
      }
      auto chain = [&](auto& narrow) {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          uint32_t gh[4][4];
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int t = 0; t < 4; ++t) gh[g][t] = args.gelu_tab[narrow(acc[i][1][4 * g + t] + bgate[g][t])];
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            uint32_t h[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
              h[t] = narrow(h2f_bits((uint16_t)narrow(acc[i][0][4 * g + t] + bval[g][t])) * h2f_bits((uint16_t)gh[g][t]));
            out[i][g] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
          }
        }
      };
      if (__builtin_amdgcn_ballot_w64(!(amax < 65520.0f))) {
        NarrowFast fast;
        chain(fast);
        if (__builtin_amdgcn_ballot_w64(fast.nan)) {
          NarrowExact exact;
          chain(exact);
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = (int)un.m0 + wm * WM + i * 32 + (lane & 31);
        if (row >= M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col0 = n0 / 2 + 8 * g + lane_col;
          uint16_t* p = reinterpret_cast<uint16_t*>(Cp) + (int64_t)row * args.ldc + col0;
          const uint32_t hv[4] = {out[i][g].x & 0xffffu, out[i][g].x >> 16, out[i][g].y & 0xffffu, out[i][g].y >> 16};
          if (col0 + 4 <= Nout && ((uintptr_t)p & 7) == 0) {
            *reinterpret_cast<uint2*>(p) = out[i][g];
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (col0 + t < Nout) p[t] = (uint16_t)hv[t];
          }
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = (int)un.m0 + wm * WM + i * 32 + (lane & 31);
      float gl[4][4];
      {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float gate = acc[i][1][4 * g + t];
            if (has_b) gate += bgate[g][t];
            gl[g][t] = gelu_ref_f32(gate);
          }
      }
      if (row < M) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col0 = n0 / 2 + 8 * g + lane_col;
          if (col0 < Nout) {
            float v[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              float val = acc[i][0][4 * g + t];
              if (has_b) val += bval[g][t];
              v[t] = val * gl[g][t];
            }
            store_cols<T>(Cp + (int64_t)row * args.ldc + col0, v, Nout - col0 < 4 ? Nout - col0 : 4);
          }
        }
      }
    }
    return;
  }
  if (args.ksplit > 1) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = (int)un.m0 + wm * WM + i * 32 + (lane & 31);
      if (row < M) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int col0 = (int)un.n0 + wn * WN + j * 32 + 8 * g + lane_col;
            if (col0 < (int)args.N)
              *reinterpret_cast<float4*>(args.partial + (un.split * args.M + row) * args.ld_partial + col0) =
                  make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          }
      }
    }
    return;
  }
  if constexpr ((EPI == EPI_LINEAR || EPI == EPI_CONV) && sizeof(T) == 2) {
    if (epi_tile_fast<T, EPI, BN>(args, un)) {
      // fp16, every column of the tile present: all values computed into registers (a lane holds
      // 4 consecutive columns per (i, j, g)), then one 8-byte store each.
      const uint16_t* bias = reinterpret_cast<const uint16_t*>(args.bias);
      const uint16_t* res = reinterpret_cast<const uint16_t*>(args.residual);
      const uint16_t* cadd = reinterpret_cast<const uint16_t*>(args.chan_add);
      uint16_t* Cptr = reinterpret_cast<uint16_t*>(args.c);
      const int col_base = (int)un.n0 + wn * WN + lane_col;  // + j*32 + 8*g
      int rows[FM], rrows[FM];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        rows[i] = (int)un.m0 + wm * WM + i * 32 + (lane & 31);
        rrows[i] = rows[i] < M ? rows[i] : M - 1;
      }
      const int OHW = (int)(args.OH * args.OW);
      const int img = EPI == EPI_CONV ? (int)args.div_ohw.div((uint32_t)un.n0) : 0;
      const int pix_base = col_base - img * OHW;
      // output element offset of (i, j, g)
      auto out_off = [&](int i, int j, int g) -> int64_t {
        if constexpr (EPI == EPI_CONV) return ((int64_t)img * M + rows[i]) * OHW + pix_base + j * 32 + 8 * g;
        return (int64_t)rows[i] * args.ldc + col_base + j * 32 + 8 * g;
      };
      // bias: per column (LINEAR) or per row (CONV); fp16 -0 without one
      Raw4<uint16_t> bz[EPI == EPI_LINEAR ? FN : 1][4];
      float bv[FM], av[FM];
      if constexpr (EPI == EPI_LINEAR) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            bz[j][g].u = bias ? load_raw4<uint16_t>(bias + col_base + j * 32 + 8 * g).u : make_uint2(0x80008000u, 0x80008000u);
      } else {
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          bv[i] = bias ? h2f_bits(bias[rrows[i]]) : -0.0f;
          av[i] = cadd ? h2f_bits(cadd[img * args.chan_add_ld + rrows[i]]) : 0.0f;
        }
      }
      auto run = [&](auto ha_c, auto hr_c) {
        constexpr bool HA = decltype(ha_c)::value, HR = decltype(hr_c)::value;
        Raw4<uint16_t> rz[FM][FN][4];
        if constexpr (HR) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int64_t o = EPI == EPI_CONV ? ((int64_t)img * M + rrows[i]) * OHW + pix_base + j * 32 + 8 * g
                                                  : (int64_t)rrows[i] * args.ld_res + col_base + j * 32 + 8 * g;
                rz[i][j][g] = load_raw4<uint16_t>(res + o);
              }
        }
        uint2 out[FM][FN][4];
        auto chain = [&](auto& narrow) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                uint32_t h[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                  float b, a = 0.0f, r = 0.0f;
                  if constexpr (EPI == EPI_LINEAR) {
                    b = bz[j][g].at(t);
                  } else {
                    b = bv[i];
                    a = av[i];
                  }
                  if constexpr (HR) r = rz[i][j][g].at(t);
                  h[t] = epi_chain_h<EPI, ACT, HA, HR>(acc[i][j][4 * g + t], b, a, r, args.gelu_tab, narrow);
                }
                out[i][j][g] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
              }
        };
        NarrowFast fast;
        chain(fast);
        if (__builtin_amdgcn_ballot_w64(fast.nan)) {
          NarrowExact exact;
          chain(exact);
        }
        const bool al = ((uintptr_t)Cptr & 7) == 0 && (EPI == EPI_CONV || (args.ldc & 3) == 0);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          if (rows[i] >= M) continue;
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              uint16_t* p = Cptr + out_off(i, j, g);
              if (al) {
                *reinterpret_cast<uint2*>(p) = out[i][j][g];
              } else {
                p[0] = (uint16_t)(out[i][j][g].x & 0xffffu);
                p[1] = (uint16_t)(out[i][j][g].x >> 16);
                p[2] = (uint16_t)(out[i][j][g].y & 0xffffu);
                p[3] = (uint16_t)(out[i][j][g].y >> 16);
              }
            }
        }
      };
      const bool ha = EPI == EPI_CONV && cadd != nullptr, hr = res != nullptr;
      if constexpr (EPI == EPI_CONV) {
        if (ha && hr) run(std::true_type{}, std::true_type{});
        else if (ha) run(std::true_type{}, std::false_type{});
        else if (hr) run(std::false_type{}, std::true_type{});
        else run(std::false_type{}, std::false_type{});
      } else {
        if (hr) run(std::false_type{}, std::true_type{});
        else run(std::false_type{}, std::false_type{});
      }
      return;
    }
  }
  if constexpr (EPI == EPI_LINEAR || EPI == EPI_CONV) {
    if (epi_tile_fast<T, EPI, BN>(args, un)) {
      const T* bias = reinterpret_cast<const T*>(args.bias);
      const T* res = reinterpret_cast<const T*>(args.residual);
      T* Cptr = reinterpret_cast<T*>(args.c);
      const bool has_b = bias != nullptr, has_r = res != nullptr;
      const int col_base = (int)un.n0 + wn * WN + lane_col;  // + j*32 + 8*g
      int rows[FM], rrows[FM];  // rows, and rows clamped into the matrix for the reads
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        rows[i] = (int)un.m0 + wm * WM + i * 32 + (lane & 31);
        rrows[i] = rows[i] < M ? rows[i] : M - 1;
      }
      Raw4<T> rz[FM][FN][4] = {};
      if constexpr (EPI == EPI_LINEAR) {
        Raw4<T> bz[FN][4] = {};
        if (has_b) {
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) bz[j][g] = load_raw4<T>(bias + col_base + j * 32 + 8 * g);
        }
        if (has_r) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g)
                rz[i][j][g] = load_raw4<T>(res + (int64_t)rrows[i] * args.ld_res + col_base + j * 32 + 8 * g);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              float v[4], b[4], r[4];
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                v[t] = acc[i][j][4 * g + t];
                b[t] = bz[j][g].at(t);
                r[t] = rz[i][j][g].at(t);
              }
              epi_math<T, EPI, ACT>(v, b, has_b, 0.0f, false, r, has_r, args.gelu_tab);
              if (rows[i] < M) store_cols<T>(Cptr + (int64_t)rows[i] * args.ldc + col_base + j * 32 + 8 * g, v, 4);
            }
      } else {
        // conv: row = output channel, col = output pixel; the tile lies in image img (NCHW store)
        const T* cadd = reinterpret_cast<const T*>(args.chan_add);
        const int OHW = (int)(args.OH * args.OW);
        const int img = (int)args.div_ohw.div((uint32_t)un.n0);
        const int pix_base = col_base - img * OHW;
        float bv[FM], av[FM];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          bv[i] = has_b ? Elem<T>::load(bias, rrows[i]) : 0.0f;
          av[i] = cadd ? Elem<T>::load(cadd, img * args.chan_add_ld + rrows[i]) : 0.0f;
        }
        if (has_r) {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
              for (int g = 0; g < 4; ++g)
                rz[i][j][g] = load_raw4<T>(res + ((int64_t)img * M + rrows[i]) * OHW + pix_base + j * 32 + 8 * g);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              float v[4], r[4];
              const float b[4] = {bv[i], bv[i], bv[i], bv[i]};
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                v[t] = acc[i][j][4 * g + t];
                r[t] = rz[i][j][g].at(t);
              }
              epi_math<T, EPI, ACT>(v, b, true, av[i], cadd != nullptr, r, has_r);
              if (rows[i] < M)
                store_cols<T>(Cptr + ((int64_t)img * M + rows[i]) * OHW + pix_base + j * 32 + 8 * g, v, 4);
            }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int row = (int)un.m0 + wm * WM + i * 32 + (lane & 31);
    if (row < M) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int col0 = (int)un.n0 + wn * WN + j * 32 + 8 * g + lane_col;
          float v[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = acc[i][j][4 * g + t];
          emit4<T, EPI, ACT>(args, un.bz, row, col0, v);
        }
      }
    }
  }
}

template <typename T, int BM, int BN, int WGM, int MODE, int EPI, int ACT, bool CONV_FAST>
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
  const int kc = (tid % CH_PER_ROW) * VEC;  // k offset of this thread's chunks within a tile
  const uint32_t G = gridDim.x;
  const uint32_t nk_total = (uint32_t)ceil_div(args.K, BK);

  // ---- loader state (the unit whose tiles are being fetched) --------------------------
  // Every global read is a buffer load whose byte offset is either the chunk's address or
  // kOOB: the buffer's range check returns zeros for the latter, so rows past M/N, chunks past
  // K, the conv's padding taps and fetches past the last unit need no branches (a branch here
  // makes the compiler wait for every outstanding load before the LDS stores, serialising the
  // prefetch).
  constexpr uint32_t kOOB = 0x80000000u;
  constexpr int ES = (int)sizeof(T);
  __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
  uint32_t a_off[A_CH];
  uint32_t b_off[MODE == MODE_NN ? 1 : B_CH];
  int conv_iy[MODE == MODE_CONV ? B_CH : 1], conv_ix[MODE == MODE_CONV ? B_CH : 1];
  // CONV_FAST: per chunk the element offset of tap (0, 0) at this thread's channel (negative
  // in the padding) and the bitmask of the filter taps that land inside the image; per tile the
  // (tap, ky, kx, channel) of the loader cursor, stepped by counters instead of divided out.
  int c_base[MODE == MODE_CONV ? B_CH : 1];
  uint32_t c_mask[MODE == MODE_CONV ? B_CH : 1];
  int l_tap = 0, l_ky = 0, l_kx = 0, l_ch = 0;
  uint32_t l_u = blockIdx.x;  // loader cursor: unit, K tile within the unit
  int64_t l_k = 0;
  GemmUnit lun{};
  int64_t l_n0 = 0;

  auto set_loader = [&]() {
    lun = decode_unit<BM, BN>(args, l_u, nk_total);
    l_n0 = lun.n0;
    a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const T*>(args.a) + lun.bz * args.stride_a), (short)0, (int)args.a_bytes, 0x00020000);
    b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const T*>(args.b) + (MODE == MODE_CONV ? 0 : lun.bz * args.stride_b)), (short)0,
        (int)args.b_bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int64_t row = lun.m0 + (tid + i * 256) / CH_PER_ROW;
      a_off[i] = row < args.M ? ((uint32_t)row * (uint32_t)args.lda + (uint32_t)kc) * (uint32_t)ES : kOOB;
    }
    if constexpr (MODE == MODE_NT) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int64_t row = lun.n0 + (tid + i * 256) / CH_PER_ROW;
        b_off[i] = row < args.N ? ((uint32_t)row * (uint32_t)args.ldb + (uint32_t)kc) * (uint32_t)ES : kOOB;
      }
    } else if constexpr (MODE == MODE_CONV) {
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const int64_t p = lun.n0 + (tid + i * 256) / CH_PER_ROW;
        const bool ok = p < args.N;
        const uint32_t pp = ok ? (uint32_t)p : 0u;
        const uint32_t img = args.div_ohw.div(pp), pix = pp - img * args.div_ohw.d;
        const uint32_t oyu = args.div_ow.div(pix);
        const int oy = (int)oyu, ox = (int)(pix - oyu * args.div_ow.d);
        // rows past N get an origin no tap can reach, so every tap tests out of bounds
        conv_iy[i] = ok ? oy * (int)args.sh - (int)args.ph : -(1 << 28);
        conv_ix[i] = ox * (int)args.sw - (int)args.pw;
        // element offset of x_nhwc[img, iy0, ix0, kc] (iy0/ix0 may lie in the padding; only
        // in-bounds taps are ever turned into a real offset)
        b_off[i] = (img * (uint32_t)args.H * (uint32_t)args.W) * (uint32_t)args.Cp + (uint32_t)kc;
        if constexpr (CONV_FAST) {
          const int H = (int)args.H, W = (int)args.W, KW = (int)args.KW, KH = (int)args.KH_;
          const int iy0 = conv_iy[i], ix0 = conv_ix[i];
          c_base[i] = ok ? (int)b_off[i] + (iy0 * W + ix0) * (int)args.Cp : 0;
          uint32_t m = 0;
          for (int ky = 0; ky < KH; ++ky) {
            const int iy = iy0 + ky * (int)args.dh;
            for (int kx = 0; kx < KW; ++kx) {
              const int ix = ix0 + kx * (int)args.dw;
              if (ok && iy >= 0 && iy < H && ix >= 0 && ix < W) m |= 1u << (ky * KW + kx);
            }
          }
          c_mask[i] = m;
        }
      }
      if constexpr (CONV_FAST) {
        const int k0 = (int)(lun.kt0 * BK), Cp = (int)args.Cp, KW = (int)args.KW;
        l_tap = k0 / Cp;
        l_ch = k0 - l_tap * Cp;
        l_ky = l_tap / KW;
        l_kx = l_tap - l_ky * KW;
      }
    }
  };
  if (l_u < args.units) set_loader();

  constexpr int NRB = MODE == MODE_NN ? B_CH_NN : B_CH;
  // Two register stages: step s+2 is requested while step s is multiplied, so every global
  // load has two steps of MFMA work (plus a barrier) to arrive.
  uint4 ra0[A_CH], rb0[NRB], ra1[A_CH], rb1[NRB];

  auto bload = [&](const __amdgpu_buffer_rsrc_t& r, uint32_t off) -> uint4 {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
  };

  // Fetches the loader cursor's tile into (ra, rb) and advances the cursor.  Past the last
  // unit every offset is kOOB (the loads return zeros and are never consumed).
  auto load_next = [&](uint4(&ra)[A_CH], uint4(&rb)[NRB]) {
    const bool live = l_u < args.units;
    const int64_t k0 = (lun.kt0 + l_k) * BK;
    const uint32_t kb = (uint32_t)(k0 * ES);
    if constexpr (MODE == MODE_CONV && CONV_FAST) {
      // K = taps * Cp is a whole number of tiles: every chunk of a live tile is in range.  Rows
      // past M carry a_off = kOOB, and kOOB + kb (< 2^32) is still beyond the buffer.
#pragma unroll
      for (int i = 0; i < A_CH; ++i) ra[i] = bload(a_rsrc, a_off[i] + kb);
      const int tap_off = (l_ky * (int)args.dh * (int)args.W + l_kx * (int)args.dw) * (int)args.Cp + l_ch;
#pragma unroll
      for (int i = 0; i < B_CH; ++i) {
        const bool ok = live && ((c_mask[i] >> l_tap) & 1u);
        rb[i] = bload(b_rsrc, ok ? (uint32_t)(c_base[i] + tap_off) * (uint32_t)ES : kOOB);
      }
      if (live) {
        l_ch += BK;
        if (l_ch == (int)args.Cp) {
          l_ch = 0;
          ++l_tap;
          if (++l_kx == (int)args.KW) {
            l_kx = 0;
            ++l_ky;
          }
        }
      }
    } else {
      const bool kin = live && k0 + kc < args.K;  // K % VEC == 0: a chunk is entirely in or out
#pragma unroll
      for (int i = 0; i < A_CH; ++i) ra[i] = bload(a_rsrc, kin ? a_off[i] + kb : kOOB);
      if constexpr (MODE == MODE_NT) {
#pragma unroll
        for (int i = 0; i < B_CH; ++i) rb[i] = bload(b_rsrc, kin ? b_off[i] + kb : kOOB);
      } else if constexpr (MODE == MODE_NN) {
#pragma unroll
        for (int i = 0; i < B_CH_NN; ++i) {
          const int c = tid + i * 256;
          const int64_t k = k0 + c / NB_CH_ROW, n = l_n0 + (c % NB_CH_ROW) * VEC;
          const bool ok = live && k < args.K && n < args.N;  // N % VEC == 0: chunks are whole
          rb[i] = bload(b_rsrc, ok ? (uint32_t)((k * args.ldb + n) * ES) : kOOB);
        }
      } else {
        // Implicit im2col, generic: k = (ky*KW + kx)*Cp + ch decoded per chunk (a tile may
        // straddle taps when Cp is not a multiple of BK).
        const int W = (int)args.W, H = (int)args.H, Cp = (int)args.Cp, KW = (int)args.KW;
        const int k = (int)k0 + kc;
        const int tap = k / Cp;
        const int ch = k - tap * Cp - kc;
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
    }
    // advance (uniform across the workgroup)
    if (live && ++l_k == lun.nkt) {
      l_k = 0;
      l_u += G;
      if (l_u < args.units) set_loader();
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
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  };
  zero_acc();

  // All of a K tile's fragments are read from LDS first and the MFMAs issued back to back
  // after one wait: reading each step's fragments right before its MFMA (into the same
  // registers) exposes the LDS latency once per MFMA instead of once per tile.
  constexpr int KS = BK / Mfma<T>::KI;
  auto compute = [&](int buf) {
    const T* a_base = &As[buf][(wm * WM + (lane & 31)) * LDK];
    const T* b_base = &Bs[buf][(wn * WN + (lane & 31)) * LDK];
    typename Mfma<T>::Frag af[KS][FM], bf[KS][FN];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
      for (int i = 0; i < FM; ++i) af[kk][i] = Mfma<T>::load(a_base + i * 32 * LDK, kk * Mfma<T>::KI, lane);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[kk][j] = Mfma<T>::load(b_base + j * 32 * LDK, kk * Mfma<T>::KI, lane);
    }
    // keep the scheduler from sinking each read back next to its MFMA
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = Mfma<T>::mma(bf[kk][j], af[kk][i], acc[i][j]);
  };

  auto finish_unit = [&](const GemmUnit& un) {
    gemm_finish_unit<T, BM, BN, WGM, EPI, ACT>(args, un, acc, lane, wm, wn);
  };

  // compute cursor
  uint32_t c_u = blockIdx.x;
  int64_t c_k = 0;
  if (c_u >= args.units) return;  // (the launcher sizes the grid to at most `units`)
  GemmUnit cun = decode_unit<BM, BN>(args, c_u, nk_total);
  // Multiplies the step in LDS buffer `buf`; at a unit's last K tile writes its results and
  // moves on.  Returns false after the workgroup's last unit.
  auto step = [&](int buf) -> bool {
    compute(buf);
    if (++c_k == cun.nkt) {
      finish_unit(cun);
      zero_acc();
      c_k = 0;
      c_u += G;
      if (c_u >= args.units) return false;
      cun = decode_unit<BM, BN>(args, c_u, nk_total);
    }
    return true;
  };

  load_next(ra0, rb0);
  load_next(ra1, rb1);
  store_tiles(0, ra0, rb0);
  __syncthreads();
  while (true) {
    // even step in buffer 0; the next step is landing in stage 1
    load_next(ra0, rb0);
    if (!step(0)) break;
    store_tiles(1, ra1, rb1);
    __syncthreads();
    // odd step in buffer 1; the next step is landing in stage 0
    load_next(ra1, rb1);
    if (!step(1)) break;
    store_tiles(0, ra0, rb0);
    __syncthreads();
  }
}

// Sums the K slices of a split GEMM in slice order and applies the epilogue; one thread per
// 4 consecutive outputs of a row.  The slices are read eight at a time, all loads of a group in
// flight together (one memory round trip per group instead of one per slice).
template <typename T, int EPI, int ACT>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const GemmArgs args) {
  const int64_t n4 = ceil_div(args.N, 4);
  const int64_t total = args.M * n4;
  const int64_t slice = args.M * args.ld_partial;
  const int ks = (int)args.ksplit;
  // The linear and conv epilogues over at most 8 slices (every split the planners choose):
  // 32-bit indices, and each thread issues its epilogue operands (bias, addend, residual)
  // ahead of its slices in one straight-line block, so it waits for one memory round trip
  // rather than two (slices past ks re-read the last one, in range, and are not added).
  constexpr bool kFast = EPI == EPI_LINEAR || EPI == EPI_CONV;
  const int OHW = (int)(args.OH * args.OW);
  if (kFast && ks <= 8 && total < (int64_t(1) << 31) && (EPI == EPI_LINEAR || OHW % 4 == 0)) {
    const uint32_t un4 = (uint32_t)n4, ut = (uint32_t)total;
    const int N = (int)args.N, M = (int)args.M;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < ut; i += gridDim.x * blockDim.x) {
      const uint32_t row = i / un4;
      const int col0 = (int)(i - row * un4) * 4;
      const int nv = N - col0 < 4 ? N - col0 : 4;
      // range-checked buffer loads: an absent operand has an empty range and reads zeros, so
      // the block has no branch and the loads stay ahead of the slices
      float b[4], r[4], av = 0.0f;
      T* dst;
      const bool has_b = args.bias != nullptr, has_r = args.residual != nullptr, has_a = args.chan_add != nullptr;
      if constexpr (EPI == EPI_LINEAR) {
        const __amdgpu_buffer_rsrc_t b_rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void*)args.bias, (short)0, has_b ? N * (int)sizeof(T) : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t r_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)args.residual, (short)0, has_r ? (int)(((int64_t)(M - 1) * args.ld_res + N) * (int64_t)sizeof(T)) : 0,
            0x00020000);
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
          const int c = col0 + t4 < N ? col0 + t4 : N - 1;
          if constexpr (sizeof(T) == 2) {
            b[t4] = h2f_bits(__builtin_amdgcn_raw_buffer_load_b16(b_rsrc, c * 2, 0, 0));
            r[t4] = h2f_bits(__builtin_amdgcn_raw_buffer_load_b16(r_rsrc, (int)(((int64_t)row * args.ld_res + c) * 2), 0, 0));
          } else {
            b[t4] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b_rsrc, c * 4, 0, 0));
            r[t4] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_rsrc, (int)(((int64_t)row * args.ld_res + c) * 4), 0, 0));
          }
        }
        dst = reinterpret_cast<T*>(args.c) + (int64_t)row * args.ldc + col0;
      } else {
        // row = output channel, col = output pixel (image-major; OHW % 4 == 0, so the 4
        // pixels lie in one image and are contiguous); NCHW store
        const int img = (int)args.div_ohw.div((uint32_t)col0);
        const int64_t addr = ((int64_t)img * M + row) * OHW + (col0 - img * OHW);
        const int B = (int)(N / OHW);
        const __amdgpu_buffer_rsrc_t b_rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void*)args.bias, (short)0, has_b ? M * (int)sizeof(T) : 0, 0x00020000);
        const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)args.chan_add, (short)0, has_a ? (int)(((int64_t)(B - 1) * args.chan_add_ld + M) * (int64_t)sizeof(T)) : 0,
            0x00020000);
        const __amdgpu_buffer_rsrc_t r_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)args.residual, (short)0, has_r ? (int)((int64_t)B * M * OHW * (int64_t)sizeof(T)) : 0, 0x00020000);
        float bv;
        if constexpr (sizeof(T) == 2) {
          bv = h2f_bits(__builtin_amdgcn_raw_buffer_load_b16(b_rsrc, (int)row * 2, 0, 0));
          av = h2f_bits(__builtin_amdgcn_raw_buffer_load_b16(a_rsrc, (img * args.chan_add_ld + (int)row) * 2, 0, 0));
#pragma unroll
          for (int t4 = 0; t4 < 4; ++t4)
            r[t4] = h2f_bits(__builtin_amdgcn_raw_buffer_load_b16(r_rsrc, (int)((addr + (t4 < nv ? t4 : 0)) * 2), 0, 0));
        } else {
          bv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b_rsrc, (int)row * 4, 0, 0));
          av = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(a_rsrc, (img * args.chan_add_ld + (int)row) * 4, 0, 0));
#pragma unroll
          for (int t4 = 0; t4 < 4; ++t4)
            r[t4] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_rsrc, (int)((addr + (t4 < nv ? t4 : 0)) * 4), 0, 0));
        }
        b[0] = b[1] = b[2] = b[3] = bv;
        dst = reinterpret_cast<T*>(args.c) + addr;
      }
      const float* p = args.partial + (int64_t)row * args.ld_partial + col0;
      float4 t[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) t[k] = *reinterpret_cast<const float4*>(p + (int64_t)(k < ks ? k : ks - 1) * slice);
      float4 s = t[0];
#pragma unroll
      for (int k = 1; k < 8; ++k)
        if (k < ks) {
          s.x += t[k].x;
          s.y += t[k].y;
          s.z += t[k].z;
          s.w += t[k].w;
        }
      float v[4] = {s.x, s.y, s.z, s.w};
      if constexpr (EPI == EPI_LINEAR)
        epi_math<T, EPI, ACT>(v, b, has_b, 0.0f, false, r, has_r, args.gelu_tab);
      else
        epi_math<T, EPI, ACT>(v, b, true, av, has_a, r, has_r);
      store_cols<T>(dst, v, nv);
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(i / n4);
    const int col0 = (int)(i - (int64_t)row * n4) * 4;
    const float* p = args.partial + (int64_t)row * args.ld_partial + col0;
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int k0 = 0; k0 < ks; k0 += 8) {
      float4 t[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < ks) t[k] = *reinterpret_cast<const float4*>(p + (int64_t)(k0 + k) * slice);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k0 + k >= ks) break;
        if (k0 + k == 0) {
          s = t[0];
        } else {
          s.x += t[k].x;
          s.y += t[k].y;
          s.z += t[k].z;
          s.w += t[k].w;
        }
      }
    }
    float v[4] = {s.x, s.y, s.z, s.w};
    emit4<T, EPI, ACT>(args, 0, row, col0, v);
  }
}

}  // namespace mthip
