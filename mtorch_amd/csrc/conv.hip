// conv2d (NCHW in, NCHW out) as an implicit GEMM on MFMA.
//
//   Y[o, pixel] = sum_{ky,kx,c} Wp[o, (ky,kx,c)] * X_nhwc[img, oy*s-p+ky*d, ox*s-p+kx*d, c]
//
// The activation is staged once as NHWC with the channel count padded to a whole 16-byte
// chunk (Cp), and the weight as [O][KH][KW][Cp], so every im2col chunk the GEMM gathers is a
// single aligned 16-byte load of Cp-contiguous channels.  Rows of the GEMM are output channels
// and columns are output pixels, so the MFMA output lanes walk consecutive pixels and the
// NCHW store stays coalesced.  Bias and an optional residual are applied in the epilogue.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "conv_halo.h"
#include "gemm_core.h"

namespace mthip {

int launch_conv_gemm(int device, int dtype, const GemmArgs& a, hipStream_t s);
int try_stream_conv1x1(int device, const void* x_nhwc, const void* wp, const void* b, void* y, const void* residual,
                       int64_t B, int64_t HW, int64_t Cp, int64_t O, hipStream_t s);

namespace {

// xp[b][hw][cp] = x[b][c][hw] (0 for c >= C), through a 32x32 LDS tile.
template <typename T>
__global__ void nchw_to_nhwc_pad_kernel(const T* __restrict__ x, T* __restrict__ xp, int64_t C, int64_t Cp,
                                        int64_t HW) {
  __shared__ T tile[32][33];
  const int64_t b = blockIdx.z;
  const int64_t hw0 = (int64_t)blockIdx.x * 32, c0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int j = ty; j < 32; j += 8) {
    const int64_t c = c0 + j, hw = hw0 + tx;
    T v = T(0);
    if (c < C && hw < HW) v = x[(b * C + c) * HW + hw];
    tile[j][tx] = v;
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int64_t hw = hw0 + j, c = c0 + tx;
    if (hw < HW && c < Cp) xp[(b * HW + hw) * Cp + c] = tile[tx][j];
  }
}

// Nearest 2x upsampling of NCHW x[B][C][H][W] written channels-last: xp[b][(2y+dy)*2W + 2x+dx][c]
// = x[b][c][y][x] (0 for c >= C) -- interpolate(scale_factor=2, mode="nearest") and the conv's
// layout change in one pass.  A 32-pixel x 32-channel tile of x goes through LDS; each element
// is stored at its four output pixels.
template <typename T>
__global__ void upsample2x_to_nhwc_pad_kernel(const T* __restrict__ x, T* __restrict__ xp, int64_t C, int64_t Cp,
                                              int64_t H, int64_t W) {
  __shared__ T tile[32][33];
  const int64_t b = blockIdx.z, HW = H * W;
  const int64_t hw0 = (int64_t)blockIdx.x * 32, c0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int j = ty; j < 32; j += 8) {
    const int64_t c = c0 + j, hw = hw0 + tx;
    T v = T(0);
    if (c < C && hw < HW) v = x[(b * C + c) * HW + hw];
    tile[j][tx] = v;
  }
  __syncthreads();
  const int64_t W2 = 2 * W;
  for (int j = ty; j < 32; j += 8) {
    const int64_t hw = hw0 + j, c = c0 + tx;
    if (hw < HW && c < Cp) {
      const int64_t yy = hw / W, xx = hw - yy * W;
      T* dst = xp + ((b * 4 * HW) + 2 * yy * W2 + 2 * xx) * Cp + c;
      const T v = tile[tx][j];
      dst[0] = v;
      dst[Cp] = v;
      dst[W2 * Cp] = v;
      dst[W2 * Cp + Cp] = v;
    }
  }
}

// The same layout change for 16-bit data with HW and Cp multiples of 8, in 16-byte pieces: a
// 64-pixel x 64-channel tile read as 8-pixel runs of one channel, written as 8-channel runs of
// one pixel (the scalar kernel above moves 2 bytes per lane each way).
__global__ __launch_bounds__(256) void nchw_to_nhwc_pad_vec_kernel(const uint16_t* __restrict__ x,
                                                                   uint16_t* __restrict__ xp, int64_t C, int64_t Cp,
                                                                   int64_t HW) {
  constexpr int PITCH = 72;  // halves per LDS channel row (16-byte multiple)
  __shared__ __align__(16) uint16_t tile[64 * PITCH];
  const int64_t b = blockIdx.z;
  const int64_t hw0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int v = (int)threadIdx.x + 256 * r;
    const int cl = v >> 3, pv = v & 7;
    const int64_t c = c0 + cl, p = hw0 + pv * 8;
    uint4 d = make_uint4(0u, 0u, 0u, 0u);
    if (c < C && p < HW) d = *reinterpret_cast<const uint4*>(x + (b * C + c) * HW + p);
    *reinterpret_cast<uint4*>(&tile[cl * PITCH + pv * 8]) = d;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int v = (int)threadIdx.x + 256 * r;
    const int pl = v >> 3, cv = v & 7;
    const int64_t p = hw0 + pl, c = c0 + cv * 8;
    if (p < HW && c < Cp) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)tile[(cv * 8 + 2 * i) * PITCH + pl] | ((uint32_t)tile[(cv * 8 + 2 * i + 1) * PITCH + pl] << 16);
      *reinterpret_cast<uint4*>(xp + (b * HW + p) * Cp + c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// wp[o][ky][kx][cp] = w[o][c][ky][kx] (0 for c >= C).
template <typename T>
__global__ void pack_weight_kernel(const T* __restrict__ w, T* __restrict__ wp, int64_t O, int64_t C, int64_t Cp,
                                   int64_t KH, int64_t KW) {
  const int64_t n = O * KH * KW * Cp;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t c = i % Cp;
    int64_t t = i / Cp;
    const int64_t kx = t % KW;
    t /= KW;
    const int64_t ky = t % KH;
    const int64_t o = t / KH;
    wp[i] = c < C ? w[((o * C + c) * KH + ky) * KW + kx] : T(0);
  }
}

// Direct convolution for grouped convs (not on the SD path): one lane per output element,
// fp32 accumulation in (c, ky, kx) order.
template <typename T>
__global__ void conv_direct_kernel(const T* __restrict__ x, const T* __restrict__ w, const T* __restrict__ bias,
                                   const T* __restrict__ residual, T* __restrict__ y, int64_t B, int64_t C, int64_t H,
                                   int64_t W, int64_t O, int64_t KH, int64_t KW, int64_t OH, int64_t OW, int64_t sh,
                                   int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw, int64_t groups) {
  const int64_t n = B * O * OH * OW;
  const int64_t Cg = C / groups, Og = O / groups;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t ox = i % OW;
    int64_t t = i / OW;
    const int64_t oy = t % OH;
    t /= OH;
    const int64_t o = t % O;
    const int64_t b = t / O;
    const int64_t c0 = (o / Og) * Cg;
    float acc = 0.0f;
    for (int64_t c = 0; c < Cg; ++c)
      for (int64_t ky = 0; ky < KH; ++ky) {
        const int64_t iy = oy * sh - ph + ky * dh;
        if (iy < 0 || iy >= H) continue;
        for (int64_t kx = 0; kx < KW; ++kx) {
          const int64_t ix = ox * sw - pw + kx * dw;
          if (ix < 0 || ix >= W) continue;
          acc += Elem<T>::load(x, ((b * C + c0 + c) * H + iy) * W + ix) * Elem<T>::load(w, ((o * Cg + c) * KH + ky) * KW + kx);
        }
      }
    if (bias) acc += Elem<T>::load(bias, o);
    if (residual) acc = Elem<T>::round_trip(acc) + Elem<T>::load(residual, i);
    Elem<T>::store(y, i, acc);
  }
}

template <typename T>
int launch_pack_weight(const void* w, void* wp, int64_t O, int64_t C, int64_t KH, int64_t KW, hipStream_t s) {
  const int64_t Cp = ceil_div(C, Mfma<T>::VEC) * Mfma<T>::VEC;
  const int64_t n = O * KH * KW * Cp;
  hipLaunchKernelGGL(pack_weight_kernel<T>, dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256), 4096))),
                     dim3(256), 0, s, (const T*)w, (T*)wp, O, C, Cp, KH, KW);
  return check_launch("pack_weight_kernel");
}

int halo_cu_count(int device) {
  static int cached[64] = {0};
  if (device < 0 || device >= 64) return 256;
  if (cached[device] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n < 1) n = 256;
    cached[device] = n;
  }
  return cached[device];
}

template <int BM, int TR, int TW>
int launch_halo(int device, HaloArgs h, hipStream_t s) {
  h.tiles_m = (int)ceil_div(h.O, BM);
  h.row_blocks = (int)ceil_div(h.H, TR);
  const int ncb = h.Cp / 64;
  // Split the channel blocks when the units alone leave CUs idle (the 16x16 and 8x8 latents).
  const int64_t base = (int64_t)h.tiles_m * h.row_blocks * h.B;
  const int cus = halo_cu_count(device);
  int ks = 1;
  if (base * 4 < (int64_t)cus * 3) ks = (int)std::min<int64_t>(ncb, std::max<int64_t>(1, cus / base));
  if (const char* f = std::getenv("MTHIP_CONV_HALO_KSPLIT")) ks = std::max(1, std::min(ncb, std::atoi(f)));
  h.cb_per_split = (int)ceil_div(ncb, ks);
  h.ksplit = (int)ceil_div(ncb, h.cb_per_split);
  // Unit order: the images vary fastest (the two units that read one weight slice run side by
  // side on one XCD) when a unit's weight slice is over twice its input patch, 9*BM rows against
  // (TR+2)*(TW+2) (every SD shape but the 48-channel whole-image 16x16 units); graph-replayed:
  // 8x8 1280->1280 19.2 -> 16.5 us, 64x64 and 32x32 2 % faster, 16x16 2 % slower, UNet 5.74 ->
  // 5.71 ms.  MTHIP_CONV_HALO_IMGFAST=0/1 forces it.
  h.img_fast = 9 * BM > 2 * (TR + 2) * (TW + 2) ? 1 : 0;
  if (const char* f = std::getenv("MTHIP_CONV_HALO_IMGFAST")) h.img_fast = std::atoi(f) != 0;
  const int64_t units = base * h.ksplit;
  MTHIP_REQUIRE(units < (int64_t(1) << 31), "conv: too many units");
  h.units = (int)units;
  void* ws = nullptr;
  const int64_t N = (int64_t)h.B * h.H * h.W;
  if (h.ksplit > 1) {
    h.ld_partial = (int)(ceil_div(N, 4) * 4);
    if (int rc = mthip_malloc(device, (size_t)((int64_t)h.ksplit * h.O * h.ld_partial) * sizeof(float), &ws)) return rc;
    h.partial = static_cast<float*>(ws);
  }
  // two producer waves (2 % over one at 64x64 and 32x32, bit-identical)
  const bool ha = h.ksplit == 1 && h.chan_add != nullptr, hr = h.ksplit == 1 && h.residual != nullptr;
  if (ha && hr)
    hipLaunchKernelGGL((conv3x3_halo_kernel<BM, TR, TW, 1, 6, true, true, 2>), dim3((unsigned)units), dim3(384), 0, s, h);
  else if (ha)
    hipLaunchKernelGGL((conv3x3_halo_kernel<BM, TR, TW, 1, 6, true, false, 2>), dim3((unsigned)units), dim3(384), 0, s, h);
  else if (hr)
    hipLaunchKernelGGL((conv3x3_halo_kernel<BM, TR, TW, 1, 6, false, true, 2>), dim3((unsigned)units), dim3(384), 0, s, h);
  else
    hipLaunchKernelGGL((conv3x3_halo_kernel<BM, TR, TW, 1, 6, false, false, 2>), dim3((unsigned)units), dim3(384), 0, s, h);
  int rc = check_launch("conv3x3_halo_kernel");
  if (rc == MTHIP_OK && h.ksplit > 1) {
    GemmArgs a{};
    a.M = h.O;
    a.N = N;
    a.c = h.y;
    a.bias = h.bias;
    a.residual = h.residual;
    a.chan_add = h.chan_add;
    a.chan_add_ld = h.chan_add_ld;
    a.OH = h.H;
    a.OW = h.W;
    a.div_ohw = FastDiv((uint32_t)(h.H * h.W));
    a.partial = h.partial;
    a.ld_partial = h.ld_partial;
    a.ksplit = h.ksplit;
    const int64_t work = a.M * ceil_div(a.N, 4);
    const unsigned rg = (unsigned)std::min<int64_t>(ceil_div(work, 256), 8192);
    hipLaunchKernelGGL((gemm_splitk_reduce_kernel<uint16_t, EPI_CONV, MTHIP_ACT_NONE>), dim3(rg), dim3(256), 0, s, a);
    rc = check_launch("gemm_splitk_reduce_kernel(conv)");
  }
  if (ws) mthip_free(device, ws);  // stream-ordered: reused only by later work
  return rc;
}

// fp16 3x3 stride-1 pad-1 convs whose padded channel count is a whole number of 64-channel
// blocks and whose width is one of the SD latent widths take the halo kernel; returns -1 for
// the rest (MTHIP_CONV_HALO=0 sends every conv to the implicit GEMM).
int try_conv_halo(int device, const void* xp, const void* wp, const void* b, void* y, int64_t B, int64_t H, int64_t W,
                  int64_t Cp, int64_t O, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
                  int64_t dh, int64_t dw, const void* residual, const void* chan_add, int64_t chan_add_ld,
                  hipStream_t s) {
  static const bool enabled = [] {
    const char* e = std::getenv("MTHIP_CONV_HALO");
    return e == nullptr || std::atoi(e) != 0;
  }();
  if (!enabled || KH != 3 || KW != 3 || sh != 1 || sw != 1 || ph != 1 || pw != 1 || dh != 1 || dw != 1) return -1;
  if (Cp % 64 != 0 || O < 64 || !(W == 64 || W == 32 || W == 16 || W == 8)) return -1;
  if (((uintptr_t)b & 1) || ((uintptr_t)residual & 7) || ((uintptr_t)xp & 15) || ((uintptr_t)wp & 15)) return -1;
  if (B * H * W * Cp * 2 >= (int64_t(1) << 31) || O * 9 * Cp * 2 >= (int64_t(1) << 31) ||
      B * O * H * W * 2 >= (int64_t(1) << 31) || B * chan_add_ld * 2 >= (int64_t(1) << 31))
    return -1;
  HaloArgs h{};
  h.x = xp;
  h.w = wp;
  h.y = y;
  h.bias = b;
  h.residual = residual;
  h.chan_add = chan_add;
  h.chan_add_ld = (int)chan_add_ld;
  h.B = (int)B;
  h.H = (int)H;
  h.W = (int)W;
  h.Cp = (int)Cp;
  h.O = (int)O;
  h.x_bytes = (int)(B * H * W * Cp * 2);
  h.w_bytes = (int)(O * 9 * Cp * 2);
  switch (W) {
    case 64: return launch_halo<80, 2, 64>(device, h, s);
    case 32: return launch_halo<80, 2, 32>(device, h, s);
    case 16: {
      // 48 channels x a whole 16x16 image per unit (four pixel fragments per wave: a weight
      // tile feeds 4x the MFMAs of the 80 x 4x16 unit) when its units, split over K, still
      // fill three quarters of the CUs -- the 1280-channel convs of SD's 16x16 latent
      // (1280->1280: 39.6 -> 24.8 us with the split-K reduction); smaller convs keep 80 x 4x16.
      const int64_t base = ceil_div(O, 48) * ceil_div(H, 16) * B;
      const int64_t cus = halo_cu_count(device);
      const int64_t ks = std::min<int64_t>(Cp / 64, std::max<int64_t>(1, cus / base));
      const int64_t units = base * ceil_div(Cp / 64, ceil_div(Cp / 64, ks));
      if (units * 4 >= cus * 3) return launch_halo<48, 16, 16>(device, h, s);
      return launch_halo<80, 4, 16>(device, h, s);
    }
    default: return launch_halo<80, 8, 8>(device, h, s);
  }
}

// The implicit GEMM over an input already staged channels-last: xp[B][H][W][Cp].
template <typename T>
int run_conv_gemm_nhwc(int device, int dtype, const void* xp, const void* wp, const void* b, void* y, int64_t B,
                       int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW, int64_t sh, int64_t sw,
                       int64_t ph, int64_t pw, int64_t dh, int64_t dw, const void* residual, hipStream_t s,
                       const void* chan_add = nullptr, int64_t chan_add_ld = 0) {
  const int64_t OH = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
  const int64_t OW = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
  if (B == 0 || OH <= 0 || OW <= 0) return MTHIP_OK;
  const int64_t Cp = ceil_div(C, Mfma<T>::VEC) * Mfma<T>::VEC;
  const int64_t K = KH * KW * Cp;
  if (O * K * (int64_t)sizeof(T) >= (int64_t(1) << 31) || B * H * W * Cp * (int64_t)sizeof(T) >= (int64_t(1) << 31))
    return fail(MTHIP_ERR_UNSUPPORTED, "mthip_conv2d: operands above 2 GiB are not supported");
  if constexpr (sizeof(T) == 2) {
    const int rc = try_conv_halo(device, xp, wp, b, y, B, H, W, Cp, O, KH, KW, sh, sw, ph, pw, dh, dw, residual,
                                 chan_add, chan_add_ld, s);
    if (rc >= 0) return rc;
    if (KH == 1 && KW == 1 && sh == 1 && sw == 1 && ph == 0 && pw == 0 && !chan_add) {
      const int rs = try_stream_conv1x1(device, xp, wp, b, y, residual, B, H * W, Cp, O, s);
      if (rs >= 0) return rs;
    }
  }
  GemmArgs a{};
  a.M = O;
  a.N = B * OH * OW;
  a.K = K;
  a.a = wp;
  a.lda = K;
  a.b = xp;
  a.c = y;
  a.bias = b;
  a.residual = residual;
  a.chan_add = chan_add;
  a.chan_add_ld = chan_add_ld;
  a.H = H;
  a.W = W;
  a.Cp = Cp;
  a.OH = OH;
  a.OW = OW;
  a.KW = KW;
  a.KH_ = KH;
  a.sh = sh;
  a.sw = sw;
  a.ph = ph;
  a.pw = pw;
  a.dh = dh;
  a.dw = dw;
  a.a_bytes = O * K * (int64_t)sizeof(T);
  a.b_bytes = B * H * W * Cp * (int64_t)sizeof(T);
  return launch_conv_gemm(device, dtype, a, s);
}

// groups == 1 with a packed weight: stage x as NHWC, then the implicit GEMM.
template <typename T>
int run_conv_gemm(int device, int dtype, const void* x, const void* wp, const void* b, void* y, int64_t B, int64_t C,
                  int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t ph,
                  int64_t pw, int64_t dh, int64_t dw, const void* residual, hipStream_t s) {
  const int64_t OH = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
  const int64_t OW = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
  if (B == 0 || OH <= 0 || OW <= 0) return MTHIP_OK;
  const int64_t Cp = ceil_div(C, Mfma<T>::VEC) * Mfma<T>::VEC;
  const int64_t HW = H * W;
  if (B * HW * Cp * (int64_t)sizeof(T) >= (int64_t(1) << 31))
    return fail(MTHIP_ERR_UNSUPPORTED, "mthip_conv2d: operands above 2 GiB are not supported");
  void* xp = nullptr;
  if (int rc = mthip_malloc(device, (size_t)(B * HW * Cp) * sizeof(T), &xp)) return rc;
  int rc;
  if (sizeof(T) == 2 && HW % 8 == 0 && Cp % 8 == 0 && ((uintptr_t)x & 15) == 0 && B <= 65535 &&
      ceil_div(HW, 64) < (int64_t(1) << 31) && ceil_div(Cp, 64) <= 65535) {
    dim3 grid((unsigned)ceil_div(HW, 64), (unsigned)ceil_div(Cp, 64), (unsigned)B);
    hipLaunchKernelGGL(nchw_to_nhwc_pad_vec_kernel, grid, dim3(256), 0, s, (const uint16_t*)x, (uint16_t*)xp, C, Cp,
                       HW);
    rc = check_launch("nchw_to_nhwc_pad_vec_kernel");
  } else {
    dim3 grid((unsigned)ceil_div(HW, 32), (unsigned)ceil_div(Cp, 32), (unsigned)B);
    hipLaunchKernelGGL(nchw_to_nhwc_pad_kernel<T>, grid, dim3(256), 0, s, (const T*)x, (T*)xp, C, Cp, HW);
    rc = check_launch("nchw_to_nhwc_pad_kernel");
  }
  if (rc == MTHIP_OK)
    rc = run_conv_gemm_nhwc<T>(device, dtype, xp, wp, b, y, B, C, H, W, O, KH, KW, sh, sw, ph, pw, dh, dw, residual,
                               s);
  mthip_free(device, xp);  // stream-ordered: reused only by work enqueued after this conv
  return rc;
}

template <typename T>
int run_conv(int device, int dtype, const void* x, const void* w, const void* b, void* y, int64_t B, int64_t C,
             int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW, int64_t sh, int64_t sw, int64_t ph, int64_t pw,
             int64_t dh, int64_t dw, int64_t groups, const void* residual, hipStream_t s) {
  const int64_t OH = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
  const int64_t OW = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
  if (B == 0 || O == 0 || OH <= 0 || OW <= 0) return MTHIP_OK;
  if (groups != 1) {
    const int64_t n = B * O * OH * OW;
    const unsigned g = (unsigned)std::min<int64_t>(ceil_div(n, 256), 8192);
    hipLaunchKernelGGL(conv_direct_kernel<T>, dim3(g), dim3(256), 0, s, (const T*)x, (const T*)w, (const T*)b,
                       (const T*)residual, (T*)y, B, C, H, W, O, KH, KW, OH, OW, sh, sw, ph, pw, dh, dw, groups);
    return check_launch("conv_direct_kernel");
  }
  const int64_t Cp = ceil_div(C, Mfma<T>::VEC) * Mfma<T>::VEC;
  void* wp = nullptr;
  if (int rc = mthip_malloc(device, (size_t)(O * KH * KW * Cp) * sizeof(T), &wp)) return rc;
  int rc = launch_pack_weight<T>(w, wp, O, C, KH, KW, s);
  if (rc == MTHIP_OK)
    rc = run_conv_gemm<T>(device, dtype, x, wp, b, y, B, C, H, W, O, KH, KW, sh, sw, ph, pw, dh, dw, residual, s);
  mthip_free(device, wp);
  return rc;
}

}  // namespace
}  // namespace mthip

using namespace mthip;

extern "C" int mthip_conv2d(int device, int dtype, const void* x, const void* w, const void* b, void* y, int64_t B,
                            int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW, int64_t stride_h,
                            int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dil_h, int64_t dil_w,
                            int64_t groups, const void* residual) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_conv2d: dtype must be F16 or F32");
  MTHIP_REQUIRE(B >= 0 && C > 0 && H > 0 && W > 0 && O > 0 && KH > 0 && KW > 0, "mthip_conv2d: bad extents");
  MTHIP_REQUIRE(stride_h > 0 && stride_w > 0 && dil_h > 0 && dil_w > 0 && pad_h >= 0 && pad_w >= 0,
                "mthip_conv2d: bad stride/padding/dilation");
  MTHIP_REQUIRE(groups > 0 && C % groups == 0 && O % groups == 0, "mthip_conv2d: bad groups");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16)
    return run_conv<uint16_t>(device, dtype, x, w, b, y, B, C, H, W, O, KH, KW, stride_h, stride_w, pad_h, pad_w,
                              dil_h, dil_w, groups, residual, s);
  return run_conv<float>(device, dtype, x, w, b, y, B, C, H, W, O, KH, KW, stride_h, stride_w, pad_h, pad_w, dil_h,
                         dil_w, groups, residual, s);
}

extern "C" int64_t mthip_conv2d_packed_bytes(int dtype, int64_t O, int64_t C, int64_t KH, int64_t KW) {
  if (dtype != MTHIP_F16 && dtype != MTHIP_F32) return -1;
  const int64_t vec = dtype == MTHIP_F16 ? 8 : 4;
  return O * KH * KW * ceil_div(C, vec) * vec * (dtype == MTHIP_F16 ? 2 : 4);
}

extern "C" int mthip_conv2d_pack_weight(int device, int dtype, const void* w, void* wp, int64_t O, int64_t C,
                                        int64_t KH, int64_t KW) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_conv2d_pack_weight: dtype must be F16 or F32");
  MTHIP_REQUIRE(O > 0 && C > 0 && KH > 0 && KW > 0, "mthip_conv2d_pack_weight: bad extents");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  return dtype == MTHIP_F16 ? launch_pack_weight<uint16_t>(w, wp, O, C, KH, KW, s)
                            : launch_pack_weight<float>(w, wp, O, C, KH, KW, s);
}

extern "C" int mthip_conv2d_prepacked(int device, int dtype, const void* x, const void* wp, const void* b, void* y,
                                      int64_t B, int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW,
                                      int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dil_h,
                                      int64_t dil_w, const void* residual) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_conv2d_prepacked: dtype must be F16 or F32");
  MTHIP_REQUIRE(B >= 0 && C > 0 && H > 0 && W > 0 && O > 0 && KH > 0 && KW > 0, "mthip_conv2d_prepacked: bad extents");
  MTHIP_REQUIRE(stride_h > 0 && stride_w > 0 && dil_h > 0 && dil_w > 0 && pad_h >= 0 && pad_w >= 0,
                "mthip_conv2d_prepacked: bad stride/padding/dilation");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16)
    return run_conv_gemm<uint16_t>(device, dtype, x, wp, b, y, B, C, H, W, O, KH, KW, stride_h, stride_w, pad_h,
                                   pad_w, dil_h, dil_w, residual, s);
  return run_conv_gemm<float>(device, dtype, x, wp, b, y, B, C, H, W, O, KH, KW, stride_h, stride_w, pad_h, pad_w,
                              dil_h, dil_w, residual, s);
}

extern "C" int mthip_upsample2x_to_nhwc(int device, int dtype, const void* x, void* xp, int64_t B, int64_t C,
                                        int64_t Cp, int64_t H, int64_t W) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_upsample2x_to_nhwc: dtype must be F16 or F32");
  MTHIP_REQUIRE(B >= 0 && C > 0 && Cp >= C && H > 0 && W > 0 && B <= 65535, "mthip_upsample2x_to_nhwc: bad extents");
  MTHIP_REQUIRE(B * 4 * H * W * Cp < (int64_t(1) << 40) && ceil_div(H * W, 32) < (int64_t(1) << 31) &&
                    ceil_div(Cp, 32) <= 65535,
                "mthip_upsample2x_to_nhwc: output too large");
  if (B == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  dim3 grid((unsigned)ceil_div(H * W, 32), (unsigned)ceil_div(Cp, 32), (unsigned)B);
  if (dtype == MTHIP_F16)
    hipLaunchKernelGGL(upsample2x_to_nhwc_pad_kernel<uint16_t>, grid, dim3(256), 0, s, (const uint16_t*)x,
                       (uint16_t*)xp, C, Cp, H, W);
  else
    hipLaunchKernelGGL(upsample2x_to_nhwc_pad_kernel<float>, grid, dim3(256), 0, s, (const float*)x, (float*)xp, C,
                       Cp, H, W);
  return check_launch("upsample2x_to_nhwc_pad_kernel");
}

extern "C" int mthip_conv2d_nhwc(int device, int dtype, const void* x_nhwc, const void* wp, const void* b, void* y,
                                 int64_t B, int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW,
                                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w, int64_t dil_h,
                                 int64_t dil_w, const void* residual, const void* chan_add, int64_t chan_add_ld) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_conv2d_nhwc: dtype must be F16 or F32");
  MTHIP_REQUIRE(chan_add == nullptr || chan_add_ld >= O, "mthip_conv2d_nhwc: chan_add row stride below O");
  MTHIP_REQUIRE(B >= 0 && C > 0 && H > 0 && W > 0 && O > 0 && KH > 0 && KW > 0, "mthip_conv2d_nhwc: bad extents");
  MTHIP_REQUIRE(stride_h > 0 && stride_w > 0 && dil_h > 0 && dil_w > 0 && pad_h >= 0 && pad_w >= 0,
                "mthip_conv2d_nhwc: bad stride/padding/dilation");
  MTHIP_REQUIRE(((uintptr_t)x_nhwc & 15) == 0 && ((uintptr_t)wp & 15) == 0,
                "mthip_conv2d_nhwc: x_nhwc and wp must be 16-byte aligned");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  if (dtype == MTHIP_F16)
    return run_conv_gemm_nhwc<uint16_t>(device, dtype, x_nhwc, wp, b, y, B, C, H, W, O, KH, KW, stride_h, stride_w,
                                        pad_h, pad_w, dil_h, dil_w, residual, s, chan_add, chan_add_ld);
  return run_conv_gemm_nhwc<float>(device, dtype, x_nhwc, wp, b, y, B, C, H, W, O, KH, KW, stride_h, stride_w, pad_h,
                                   pad_w, dil_h, dil_w, residual, s, chan_add, chan_add_ld);
}
