// linear / matmul / addmm entry points over the MFMA GEMM core.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "gemm_core.h"

namespace mthip {
namespace {

// Tile shape per problem: large 128x128 tiles when they alone fill the 256 CUs at least
// once, otherwise narrower tiles so small SD shapes (N = 320, few rows) still spread out.
enum TileKind { T128x128, T128x64, T64x128, T64x64 };

TileKind pick_tile(int64_t M, int64_t N, int64_t batch) {
  auto tiles = [&](int64_t bm, int64_t bn) { return ceil_div(M, bm) * ceil_div(N, bn) * batch; };
  if (tiles(128, 128) >= 256) return T128x128;
  if (tiles(128, 64) >= 256) return N <= 64 || M >= N ? T128x64 : T64x128;
  if (tiles(64, 128) >= 256) return T64x128;
  return T64x64;
}

template <typename T, int MODE, int EPI>
int launch_gemm(const GemmArgs& a, int64_t batch, hipStream_t s) {
  const TileKind tk = pick_tile(a.M, a.N, batch);
  constexpr int BK = sizeof(T) == 2 ? 32 : 16;
  auto grid = [&](int bm, int bn) {
    return dim3((unsigned)ceil_div(a.N, bn), (unsigned)ceil_div(a.M, bm), (unsigned)batch);
  };
  MTHIP_REQUIRE(batch <= 65535, "gemm: batch must be <= 65535");
  switch (tk) {
    case T128x128:
      MTHIP_REQUIRE(ceil_div(a.M, 128) <= 65535, "gemm: M too large");
      hipLaunchKernelGGL((gemm_kernel<T, 128, 128, BK, 2, MODE, EPI>), grid(128, 128), dim3(256), 0, s, a);
      break;
    case T128x64:
      MTHIP_REQUIRE(ceil_div(a.M, 128) <= 65535, "gemm: M too large");
      hipLaunchKernelGGL((gemm_kernel<T, 128, 64, BK, 2, MODE, EPI>), grid(128, 64), dim3(256), 0, s, a);
      break;
    case T64x128:
      MTHIP_REQUIRE(ceil_div(a.M, 64) <= 65535, "gemm: M too large");
      hipLaunchKernelGGL((gemm_kernel<T, 64, 128, BK, 2, MODE, EPI>), grid(64, 128), dim3(256), 0, s, a);
      break;
    default:
      MTHIP_REQUIRE(ceil_div(a.M, 64) <= 65535, "gemm: M too large");
      hipLaunchKernelGGL((gemm_kernel<T, 64, 64, BK, 2, MODE, EPI>), grid(64, 64), dim3(256), 0, s, a);
      break;
  }
  return check_launch("gemm_kernel");
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// Shared with conv.hip.
int launch_conv_gemm(int dtype, const GemmArgs& a, hipStream_t s) {
  if (dtype == MTHIP_F16) return launch_gemm<uint16_t, MODE_CONV, EPI_CONV>(a, 1, s);
  return launch_gemm<float, MODE_CONV, EPI_CONV>(a, 1, s);
}

}  // namespace mthip

using namespace mthip;

extern "C" {

int mthip_linear(int device, int dtype, const void* x, int64_t lda, const void* w, int64_t ldw, const void* b,
                 void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int act, const void* residual,
                 int64_t ld_res) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_linear: dtype must be F16 or F32");
  MTHIP_REQUIRE(M >= 0 && N >= 0 && K >= 0, "mthip_linear: negative extent");
  MTHIP_REQUIRE(lda >= K && ldw >= K && ldy >= N, "mthip_linear: leading dimension smaller than the row");
  MTHIP_REQUIRE(act >= MTHIP_ACT_NONE && act <= MTHIP_ACT_SILU, "mthip_linear: unknown activation");
  if (M == 0 || N == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  GemmArgs a{};
  a.M = M;
  a.N = N;
  a.K = K;
  a.a = x;
  a.lda = lda;
  a.b = w;
  a.ldb = ldw;
  a.c = y;
  a.ldc = ldy;
  a.bias = b;
  a.act = act;
  a.residual = residual;
  a.ld_res = ld_res;
  const int vec = dtype == MTHIP_F16 ? 8 : 4;
  a.vec_ok = aligned16(x) && aligned16(w) && lda % vec == 0 && ldw % vec == 0;
  if (K == 0) {
    // Empty reduction: the reference still adds the bias (and applies the tail ops).
    a.K = 0;
  }
  if (dtype == MTHIP_F16) return launch_gemm<uint16_t, MODE_NT, EPI_LINEAR>(a, 1, s);
  return launch_gemm<float, MODE_NT, EPI_LINEAR>(a, 1, s);
}

int mthip_gemm(int device, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void* a_ptr, int64_t lda,
               int64_t stride_a, const void* b_ptr, int64_t ldb, int64_t stride_b, int b_trans, void* c, int64_t ldc,
               int64_t stride_c, double alpha, double beta, const void* c_in, int64_t c_in_rs, int64_t c_in_cs,
               int64_t stride_c_in) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_gemm: dtype must be F16 or F32");
  MTHIP_REQUIRE(batch >= 0 && M >= 0 && N >= 0 && K >= 0, "mthip_gemm: negative extent");
  if (batch == 0 || M == 0 || N == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  GemmArgs a{};
  a.M = M;
  a.N = N;
  a.K = K;
  a.a = a_ptr;
  a.lda = lda;
  a.stride_a = stride_a;
  a.b = b_ptr;
  a.ldb = ldb;
  a.stride_b = stride_b;
  a.c = c;
  a.ldc = ldc;
  a.stride_c = stride_c;
  a.alpha = (float)alpha;
  a.beta = (float)beta;
  a.c_in = c_in;
  a.c_in_rs = c_in_rs;
  a.c_in_cs = c_in_cs;
  a.stride_c_in = stride_c_in;
  const int vec = dtype == MTHIP_F16 ? 8 : 4;
  a.vec_ok = aligned16(a_ptr) && aligned16(b_ptr) && lda % vec == 0 && ldb % vec == 0 && stride_a % vec == 0 &&
             stride_b % vec == 0;
  if (b_trans) {
    if (dtype == MTHIP_F16) return launch_gemm<uint16_t, MODE_NT, EPI_GEMM>(a, batch, s);
    return launch_gemm<float, MODE_NT, EPI_GEMM>(a, batch, s);
  }
  if (dtype == MTHIP_F16) return launch_gemm<uint16_t, MODE_NN, EPI_GEMM>(a, batch, s);
  return launch_gemm<float, MODE_NN, EPI_GEMM>(a, batch, s);
}

}  // extern "C"
