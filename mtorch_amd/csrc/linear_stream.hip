// Launchers of the streamed fp16 GEMM kernel (gemm_stream.h): the token-tile / K-split plan,
// linears without an activation and the channels-last 1x1 convs with an NCHW output.  In a
// translation unit of their own so that they build beside the tile GEMMs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "gemm_core.h"
#include "gemm_stream.h"

namespace mthip {
namespace {

int env_flag(const char* name, int dflt) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : dflt;
}

int cu_count(int device) {
  static int cached[64] = {0};
  if (device < 0 || device >= 64) return 256;
  if (cached[device] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n < 1) n = 256;
    cached[device] = n;
  }
  return cached[device];
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }


// Token tile and K split of the streamed kernel from a makespan model: a persistent workgroup
// per CU runs ceil(units / CUs) units of `steps` K steps each plus an epilogue, and a split adds
// the fp32 slices' write and read and the reduction launch.  Per-step and per-unit costs (µs) of
// 64- and 128-token units come from graph-replayed sweeps: a 128-token step (eight compute
// waves, two per SIMD) takes ~0.6 µs against ~0.4 for a 64-token step (four), so 128-token
// units win where they still give every CU a unit (8192x320x1280 + residual: 18.7 -> 14.9 us,
// 8192x960x320: 17.8 -> 16.3) and lose where they halve the units of a chip-filling 64-token
// plan (2048x640x2560: 16.1 against 22.6).  MTHIP_GEMM_STREAM_BT=64 or 128 forces one.
void stream_plan(int64_t M, int64_t N, int64_t K, int64_t cus, int& best_bt, int64_t& best_ks) {
  const int64_t nk = K / 64, groups = nk / 5;
  const double step_us[2] = {0.40, 0.60}, epi_us = 0.4;
  const double reduce_us = env_flag("MTHIP_GEMM_REDUCE_US", 3);  // fixed cost of a reduction launch
  const int force_bt = env_flag("MTHIP_GEMM_STREAM_BT", 0);
  best_bt = 64;
  best_ks = 1;
  double best = 0.0;
  for (int bi = 0; bi < 2; ++bi) {
    const int bt = bi ? 128 : 64;
    if (force_bt && force_bt != bt) continue;
    for (int64_t ks = 1; ks <= std::min<int64_t>(8, groups); ++ks) {
      if (groups % ks) continue;
      const int64_t units = ceil_div(M, bt) * ceil_div(N, 80) * ks;
      double t = (double)ceil_div(units, cus) * ((double)(nk / ks) * step_us[bi] + epi_us);
      if (ks > 1) t += reduce_us + (double)((ks + 1) * M * N * 4) / 3.0e6;
      if (best == 0.0 || t < best) {
        best = t;
        best_bt = bt;
        best_ks = ks;
      }
    }
  }
}

// Launches the streamed kernel over sa (operands, bias, residual, layout already set) with the
// planned tile and split, then the slice reduction (r: the reduction's GemmArgs, EPI_LINEAR
// row-major or EPI_CONV NCHW).
template <bool NCHW, bool GELU = false>
int launch_stream(int device, StreamArgs sa, GemmArgs r, int64_t K, hipStream_t s) {
  const int64_t M = sa.M, N = sa.N, cus = cu_count(device);
  int bt;
  int64_t ks;
  stream_plan(M, N, K, cus, bt, ks);
  sa.tiles_m = (int)ceil_div(M, bt);
  sa.tiles_n = (int)ceil_div(N, 80);
  sa.ksplit = (int)ks;
  sa.steps = (int)(K / 64 / ks);
  sa.units = sa.tiles_m * sa.tiles_n * sa.ksplit;
  // consecutive units share the operand with fewer tiles (held in the XCD's L2)
  sa.m_fast = sa.tiles_m <= sa.tiles_n ? 1 : 0;
  void* ws = nullptr;
  if (ks > 1) {
    const int64_t rows = NCHW ? N : M, cols = NCHW ? M : N;
    r.ld_partial = ceil_div(cols, 4) * 4;
    r.ksplit = ks;
    if (int rc = mthip_malloc(device, (size_t)(ks * rows * r.ld_partial) * sizeof(float), &ws)) return rc;
    r.partial = static_cast<float*>(ws);
    sa.partial = r.partial;
    sa.ld_partial = (int)r.ld_partial;
  }
  int64_t g = std::min<int64_t>(sa.units, cus);
  if (g > 8) g = g / 8 * 8;
  const bool hr = sa.residual != nullptr && ks == 1;
  if constexpr (GELU) {
    if (bt == 128)
      hipLaunchKernelGGL((gemm_stream_kernel<128, false, false, true>), dim3((unsigned)g), dim3(640), 0, s, sa);
    else
      hipLaunchKernelGGL((gemm_stream_kernel<64, false, false, true>), dim3((unsigned)g), dim3(320), 0, s, sa);
  } else if (bt == 128) {
    if (hr)
      hipLaunchKernelGGL((gemm_stream_kernel<128, true, NCHW>), dim3((unsigned)g), dim3(640), 0, s, sa);
    else
      hipLaunchKernelGGL((gemm_stream_kernel<128, false, NCHW>), dim3((unsigned)g), dim3(640), 0, s, sa);
  } else {
    if (hr)
      hipLaunchKernelGGL((gemm_stream_kernel<64, true, NCHW>), dim3((unsigned)g), dim3(320), 0, s, sa);
    else
      hipLaunchKernelGGL((gemm_stream_kernel<64, false, NCHW>), dim3((unsigned)g), dim3(320), 0, s, sa);
  }
  int rc = check_launch("gemm_stream_kernel");
  if (rc == MTHIP_OK && ks > 1) {
    const int64_t work = r.M * ceil_div(r.N, 4);
    const unsigned rg = (unsigned)std::min<int64_t>(ceil_div(work, 256), 8192);
    if constexpr (NCHW)
      hipLaunchKernelGGL((gemm_splitk_reduce_kernel<uint16_t, EPI_CONV, MTHIP_ACT_NONE>), dim3(rg), dim3(256), 0, s, r);
    else if constexpr (GELU)
      hipLaunchKernelGGL((gemm_splitk_reduce_kernel<uint16_t, EPI_LINEAR, MTHIP_ACT_GELU>), dim3(rg), dim3(256), 0, s, r);
    else
      hipLaunchKernelGGL((gemm_splitk_reduce_kernel<uint16_t, EPI_LINEAR, MTHIP_ACT_NONE>), dim3(rg), dim3(256), 0, s, r);
    rc = check_launch("gemm_splitk_reduce_kernel(stream)");
  }
  if (ws) mthip_free(device, ws);  // stream-ordered: reused only by later work
  return rc;
}

}  // namespace

// fp16 1x1 stride-1 unpadded convs of a channels-last activation (x_nhwc [B][HW][Cp], Cp == K a
// multiple of 320, HW % 4 == 0) with an NCHW output: the streamed kernel's NCHW mode -- the
// SD transformer's proj_out and the ResBlock shortcuts.  MTHIP_CONV_STREAM=0 turns it off
// (1, the default: up to 1280 output channels; 2: wherever it applies).  Returns -1 when it
// does not apply.  (Shared with conv.hip.)
int try_stream_conv1x1(int device, const void* x_nhwc, const void* wp, const void* b, void* y, const void* residual,
                       int64_t B, int64_t HW, int64_t Cp, int64_t O, hipStream_t s) {
  const int mode = env_flag("MTHIP_CONV_STREAM", 1);
  if (!mode || (mode == 1 && O > 1280)) return -1;
  const int64_t M = B * HW;
  if (Cp % 320 != 0 || HW % 4 != 0 || O % 16 != 0 || ((uintptr_t)y & 7) || ((uintptr_t)b & 1) ||
      ((uintptr_t)residual & 7) || !aligned16(x_nhwc) || !aligned16(wp))
    return -1;
  if (M * O >= (int64_t(1) << 30) || M * Cp >= (int64_t(1) << 30) || O * Cp >= (int64_t(1) << 30)) return -1;
  StreamArgs sa{};
  sa.a = x_nhwc;
  sa.b = wp;
  sa.c = y;
  sa.bias = b;
  sa.residual = residual;
  sa.M = (int)M;
  sa.N = (int)O;
  sa.lda = (int)Cp;
  sa.ldb = (int)Cp;
  sa.a_bytes = (int)(M * Cp * 2);
  sa.b_bytes = (int)(O * Cp * 2);
  sa.hw = (int)HW;
  sa.div_hw = FastDiv((uint32_t)HW);
  // the slice reduction as the conv GEMM's: rows = output channels, columns = pixels
  GemmArgs r{};
  r.M = O;
  r.N = M;
  r.c = y;
  r.bias = b;
  r.residual = residual;
  r.OH = HW;
  r.OW = 1;
  r.div_ohw = FastDiv((uint32_t)HW);
  return launch_stream<true>(device, sa, r, Cp, s);
}

// fp16 linears without an activation, or with GELU and no residual (the gelu of each narrowed
// value looked up in a.gelu_tab), whose K is a multiple of 320 (units of whole 5-step ring
// cycles) can take the streamed kernel (gemm_stream.h); MTHIP_GEMM_STREAM=0 turns it off.
// Returns -1 when it does not apply.
int try_stream_linear(int device, const GemmArgs& a, hipStream_t s) {
  const int mode = env_flag("MTHIP_GEMM_STREAM", 1);
  if (!mode) return -1;
  const bool gelu = a.act == MTHIP_ACT_GELU;
  if (a.act != MTHIP_ACT_NONE && !(gelu && a.residual == nullptr && a.gelu_tab != nullptr)) return -1;
  const int64_t M = a.M, N = a.N, K = a.K;
  // Where it wins (SD projections, graph-replayed): up to 1280 output channels with K >= 640 --
  // 512x1280x1280 13.5 -> 9.7 us, 2048x640x2560 19.7 -> 15.4, 512x1280x5120 22.3 -> 20.0,
  // 8192x320x1280 19.1 -> 17.7, 2048x640x640 8.9 -> 8.2 -- and, with 128-token units, K = 320
  // over >= 8192 tokens (8192x320x320 8.7 -> 8.2, with the residual 9.7 -> 9.3, 8192x960x320
  // 17.8 -> 16.3); the wide ones stay on the DTL GEMM (512x3840x1280 12.1 against 12.3,
  // 2048x1920x640 14.5 against 15.2).  MTHIP_GEMM_STREAM=2 takes it wherever it applies.
  if (mode == 1 && !(N <= 1280 && (K >= 640 || M >= 8192))) return -1;
  if (K == 0 || K % 320 != 0 || N % 16 != 0 || a.ldc % 4 != 0 || ((uintptr_t)a.c & 7) || ((uintptr_t)a.bias & 7))
    return -1;
  if (a.residual && (a.ld_res % 4 != 0 || ((uintptr_t)a.residual & 7))) return -1;
  if (!aligned16(a.a) || !aligned16(a.b) || a.lda % 8 != 0 || a.ldb % 8 != 0) return -1;
  if (M * a.ldc >= (int64_t(1) << 31) || (a.residual && M * a.ld_res >= (int64_t(1) << 31)) ||
      M * a.lda >= (int64_t(1) << 30) || N * a.ldb >= (int64_t(1) << 30))
    return -1;
  StreamArgs sa{};
  sa.a = a.a;
  sa.b = a.b;
  sa.c = a.c;
  sa.bias = a.bias;
  sa.residual = a.residual;
  sa.M = (int)M;
  sa.N = (int)N;
  sa.lda = (int)a.lda;
  sa.ldb = (int)a.ldb;
  sa.ldc = (int)a.ldc;
  sa.ld_res = (int)a.ld_res;
  sa.a_bytes = (int)a.a_bytes;
  sa.b_bytes = (int)a.b_bytes;
  if (gelu) {
    sa.gelu_tab = a.gelu_tab;
    return launch_stream<false, true>(device, sa, a, K, s);
  }
  return launch_stream<false>(device, sa, a, K, s);
}

}  // namespace mthip
