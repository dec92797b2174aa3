// linear / matmul / addmm entry points over the MFMA GEMM core.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>

#include "gemm_core.h"
#include "gemm_dtl.h"

namespace mthip {
namespace {

// Workgroup tile and wave layout (4 waves): T128x128 = 2x2 waves of 64x64, T128x64w4 = 4x1
// waves of 32x64, T64x128w1 = 1x4 waves of 64x32, T64x64 = 2x2 waves of 32x32.
enum TileKind { T128x128, T128x64w4, T64x128w1, T64x64 };

TileKind pick_tile(int MODE, int64_t M, int64_t N, int64_t batch) {
  // MTHIP_GEMM_TILE=0..3 forces a tile shape (tuning sweeps); unset selects by problem size.
  if (const char* force = std::getenv("MTHIP_GEMM_TILE")) {
    const int t = std::atoi(force);
    if (t >= 0 && t <= 3) return static_cast<TileKind>(t);
  }
  (void)M;
  (void)batch;
  // 64x64 everywhere: in isolation 128x128 tiles ran some large convs 5-20% faster, but inside
  // the UNet step (bias/residual epilogues, split-K interplay) they were 13% slower in total;
  // the four resident 64x64 workgroups per CU also hide the short K loops of the linears.
  (void)MODE;
  (void)N;
  return T64x64;
}

// Tuning switches for sweeps: MTHIP_GEMM_SPLITK=0 disables K splitting, MTHIP_GEMM_PERSIST=0
// launches one workgroup per unit, MTHIP_GEMM_XCD=0/1 forces the plain / XCD-contiguous unit
// order (default: XCD-contiguous), MTHIP_GEMM_MFAST=0/1 forces which tile dimension varies
// fastest (default: the one with fewer tiles), MTHIP_GEMM_SPLIT_TARGET sets the split-K units
// per CU.
int env_flag(const char* name, int dflt) {
  const char* e = std::getenv(name);
  return e ? std::atoi(e) : dflt;
}
bool splitk_enabled() { return env_flag("MTHIP_GEMM_SPLITK", 1) != 0; }
bool persist_enabled() { return env_flag("MTHIP_GEMM_PERSIST", 1) != 0; }
int xcd_mode() { return env_flag("MTHIP_GEMM_XCD", 2); }
int split_target() { return std::max(1, env_flag("MTHIP_GEMM_SPLIT_TARGET", 4)); }

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

// The kernel instance behind a tile choice: DS > 0 selects the direct-to-LDS fp16 kernel
// with DS stages, DS == 0 the register-staged kernel.
template <typename T, int BM, int BN, int MODE, int EPI, int ACT, bool FAST, int WGM, int DS>
constexpr auto gemm_kernel_ptr() {
  if constexpr (DS > 0) {
    static_assert(sizeof(T) == 2 && (MODE == MODE_NT || (MODE == MODE_CONV && FAST)), "direct-to-LDS: fp16, k-contiguous");
    return &gemm_dtl_kernel<BM, BN, WGM, MODE, EPI, ACT, DS>;
  } else {
    return &gemm_kernel<T, BM, BN, WGM, MODE, EPI, ACT, FAST>;
  }
}

// Resident workgroups per CU of one kernel instance (registers and LDS decide it).
template <typename T, int BM, int BN, int MODE, int EPI, int ACT, bool FAST, int WGM, int DS>
int resident_per_cu() {
  static const int v = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemm_kernel_ptr<T, BM, BN, MODE, EPI, ACT, FAST, WGM, DS>(),
                                                     256, 0) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  return v;
}

// Sizes the persistent grid, splits K when the output tiles cannot fill the chip, launches the
// GEMM (and the slice reduction).
template <typename T, int BM, int BN, int MODE, int EPI, int ACT, bool FAST, int WGM = 2, int DS = 0>
int launch_tile(int device, GemmArgs a, int64_t batch, hipStream_t s) {
  constexpr int BK = Mfma<T>::BK;
  a.tiles_m = ceil_div(a.M, BM);
  a.tiles_n = ceil_div(a.N, BN);
  const int64_t nk = std::max<int64_t>(ceil_div(a.K, BK), 1);
  const int64_t tiles = a.tiles_m * a.tiles_n * batch;
  const int64_t slots = (int64_t)cu_count(device) * resident_per_cu<T, BM, BN, MODE, EPI, ACT, FAST, WGM, DS>();
  int64_t ksplit = 1;
  if (batch == 1 && nk >= 16 && splitk_enabled() && EPI != EPI_GEGLU) {
    if (DS > 0) {
      // Pick the slice count with the shortest modelled makespan: the persistent grid runs
      // ceil(units / slots) rounds of ceil(nk / ksplit) K tiles, and every extra slice adds an
      // fp32 M x N write here plus its read in the reduction kernel.  (640 tiles on 768 slots
      // gain nothing from 2 slices -- 2 rounds of half the K -- and would pay the reduction.)
      constexpr double kStepUs = 0.6, kReduceBytesPerUs = 3.0e6;
      const double kReduceFixedUs = env_flag("MTHIP_GEMM_REDUCE_US", 3);
      double best = 0.0;
      const int64_t max_split = std::min<int64_t>(16, nk / 8);
      for (int64_t ks = 1; ks <= max_split; ++ks) {
        const int64_t rounds = ceil_div(tiles * ks, slots);
        double t = (double)(rounds * ceil_div(nk, ks)) * kStepUs;
        if (ks > 1) t += kReduceFixedUs + (double)((ks + 1) * a.M * a.N * 4) / kReduceBytesPerUs;
        if (ks == 1 || t < best) {
          best = t;
          ksplit = ks;
        }
      }
      if (const char* force = std::getenv("MTHIP_GEMM_KSPLIT")) ksplit = std::max(1, std::min(16, std::atoi(force)));
    } else {
      // Register-staged kernel: split single-batch problems with fewer tiles than about
      // `split_target` units per CU and >= 32 K tiles into enough slices to reach that, each
      // slice keeping >= 16 K tiles.
      const int64_t target = (int64_t)cu_count(device) * split_target();
      if (tiles < target && nk >= 32)
        ksplit = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(ceil_div(target, tiles), nk / 16), 16));
    }
  }
  a.kt_per_split = ceil_div(nk, ksplit);
  a.ksplit = ceil_div(nk, a.kt_per_split);  // no empty slice
  a.units = tiles * a.ksplit;
  MTHIP_REQUIRE(a.units < (int64_t(1) << 31) && a.N < (int64_t(1) << 31) && a.M < (int64_t(1) << 31),
                "gemm: problem too large (tiles, rows or columns beyond 2^31)");
  a.div_tiles_n = FastDiv((uint32_t)a.tiles_n);
  a.div_tiles_m = FastDiv((uint32_t)a.tiles_m);
  a.div_ksplit = FastDiv((uint32_t)a.ksplit);
  if (MODE == MODE_CONV) {
    a.div_ohw = FastDiv((uint32_t)(a.OH * a.OW));
    a.div_ow = FastDiv((uint32_t)a.OW);
  }
  int64_t g = persist_enabled() ? std::min(a.units, slots) : a.units;
  if (g > 8 && g < a.units) g = g / 8 * 8;  // a multiple of 8 keeps each XCD on its own run of tiles
  // Unit order and L2 reuse: each XCD takes a contiguous band of the operand with more tiles
  // and walks all tiles of the other operand fastest, so it holds 1/8 of the large operand
  // and all of the small one.  (Dealt round-robin instead, a conv's XCD would see every 8th
  // pixel tile and fetch every 3x3 halo row from memory: 2.9x the operand bytes, measured.)
  const int xm = xcd_mode();
  a.xcd_remap = xm == 0 ? 0 : 1;
  a.m_fast = a.tiles_m * batch <= a.tiles_n ? 1 : 0;
  if (const char* f = std::getenv("MTHIP_GEMM_MFAST")) a.m_fast = std::atoi(f) != 0;
  void* ws = nullptr;
  if (a.ksplit > 1) {
    a.ld_partial = ceil_div(a.N, 4) * 4;
    if (int rc = mthip_malloc(device, (size_t)(a.ksplit * a.M * a.ld_partial) * sizeof(float), &ws)) return rc;
    a.partial = static_cast<float*>(ws);
  }
  hipLaunchKernelGGL((gemm_kernel_ptr<T, BM, BN, MODE, EPI, ACT, FAST, WGM, DS>()), dim3((unsigned)g), dim3(256), 0, s, a);
  int rc = check_launch("gemm_kernel");
  if constexpr (EPI == EPI_GEGLU) return rc;
  if (rc == MTHIP_OK && a.ksplit > 1) {
    const int64_t work = a.M * ceil_div(a.N, 4);
    const unsigned rg = (unsigned)std::min<int64_t>(ceil_div(work, 256), 8192);
    hipLaunchKernelGGL((gemm_splitk_reduce_kernel<T, EPI, ACT>), dim3(rg), dim3(256), 0, s, a);
    rc = check_launch("gemm_splitk_reduce_kernel");
  }
  if (ws) mthip_free(device, ws);  // stream-ordered: reused only by later work
  return rc;
}

// Direct-to-LDS tile shapes (fp16, k-contiguous operands): MTHIP_GEMM_DTL=0 turns the kernel
// off, MTHIP_GEMM_DTL_TILE=0..5 forces one of
//   0: 64x64 (2x2 waves of 32x32), 3 stages     1: 64x64, 4 stages
//   2: 128x64 (2x2 waves of 64x32), 3 stages    3: 64x128 (2x2 waves of 32x64), 3 stages
//   4: 128x128 (2x2 waves of 64x64), 3 stages   5: 128x128, 2 stages
bool dtl_enabled() { return env_flag("MTHIP_GEMM_DTL", 1) != 0; }

// Default shape per problem, from sweeps of the SD-1.5 GEMMs and convs (fp16, batch 2):
// convs over more than 128 output pixels with a multiple of 128 output channels take 128x64
// (5-18% over 64x64 at 640 and 1280 channels; at 320 channels the third 128-row tile is half
// empty and 64x64 is 9% faster), the 8x8 convs (long K, split) and every conv with K >= 2048
// 64x64 with 4 stages (the SD stride-2 downsampling convs, graph-replayed with the layout pass:
// 320 @64x64 27.4 -> 26.3 us, 640 @32x32 27.4 -> 24.6 us against 64x64 / 128x64 with 3 stages,
// which date from before the 3x3 stride-1 convs moved to the halo kernel); linears take
// 64x64 (3 stages) up to K = 1280, 4 stages beyond, 64x128 when M*N is large, 128x128 with 2
// stages for the big square problems.
int dtl_tile_for(int MODE, int64_t M, int64_t N, int64_t K) {
  const int forced = env_flag("MTHIP_GEMM_DTL_TILE", -1);
  if (forced >= 0) return forced;
  if (MODE == MODE_CONV) return (N <= 128 || K >= 2048) ? 1 : M % 128 == 0 ? 2 : 0;
  if (M >= 4096 && N >= 4096 && K >= 2048) return 5;
  if (K >= 2048) return 1;
  if (M * N >= (int64_t)2048 * 1920 && K >= 640) return 3;
  return 0;
}

template <int MODE, int EPI, int ACT>
int launch_dtl(int device, const GemmArgs& a, int64_t batch, hipStream_t s) {
  using T = uint16_t;
  constexpr bool F = MODE == MODE_CONV;
  if constexpr (EPI == EPI_GEGLU) {
    // MTHIP_GEMM_GEGLU_TILE: 0 = 128x64 (4x1 waves of 32x64), 1 = 128x128 (2x2 waves of 64x64)
    // with 3 stages, 2 = 128x128 with 2 stages.  By default 128x128 / 2 stages where the 128x64
    // tiles number >= 2560 or, over >= 512 rows, <= 640 (SD feed-forward, graph-replayed:
    // 8192x2560x320 43.7 -> 38.9 us, 512x10240x1280 30.7 -> 29.4; 4096x2560x320 22.7 against
    // 23.6 and 2048x5120x640 even stay on 128x64; 3 stages hold one workgroup per CU and lose
    // everywhere).
    const int64_t t64 = ceil_div(a.M, 128) * ceil_div(a.N, 64) * batch;
    const int dflt = (t64 >= 2560 || (a.M >= 512 && t64 <= 640)) ? 2 : 0;
    switch (env_flag("MTHIP_GEMM_GEGLU_TILE", dflt)) {
      case 1:
        return launch_tile<T, 128, 128, MODE, EPI, ACT, F, 2, 3>(device, a, batch, s);
      case 2:
        return launch_tile<T, 128, 128, MODE, EPI, ACT, F, 2, 2>(device, a, batch, s);
      default:
        return launch_tile<T, 128, 64, MODE, EPI, ACT, F, 4, 3>(device, a, batch, s);
    }
  } else if constexpr (ACT != MTHIP_ACT_NONE) {
    switch (env_flag("MTHIP_GEMM_DTL_TILE", 0)) {
      case 3:
        return launch_tile<T, 64, 128, MODE, EPI, ACT, F, 2, 3>(device, a, batch, s);
      case 5:
        return launch_tile<T, 128, 128, MODE, EPI, ACT, F, 2, 2>(device, a, batch, s);
      default:
        return launch_tile<T, 64, 64, MODE, EPI, ACT, F, 2, 3>(device, a, batch, s);
    }
  } else {
    switch (dtl_tile_for(MODE, a.M, a.N, a.K)) {
      case 1:
        return launch_tile<T, 64, 64, MODE, EPI, ACT, F, 2, 4>(device, a, batch, s);
      case 2:
        return launch_tile<T, 128, 64, MODE, EPI, ACT, F, 2, 3>(device, a, batch, s);
      case 3:
        return launch_tile<T, 64, 128, MODE, EPI, ACT, F, 2, 3>(device, a, batch, s);
      case 4:
        return launch_tile<T, 128, 128, MODE, EPI, ACT, F, 2, 3>(device, a, batch, s);
      case 5:
        return launch_tile<T, 128, 128, MODE, EPI, ACT, F, 2, 2>(device, a, batch, s);
      default:
        return launch_tile<T, 64, 64, MODE, EPI, ACT, F, 2, 3>(device, a, batch, s);
    }
  }
}

template <typename T, int MODE, int EPI, int ACT, bool FAST>
int launch_gemm_tiles(int device, const GemmArgs& a, int64_t batch, hipStream_t s) {
  if constexpr (sizeof(T) == 2 && (MODE == MODE_NT || (MODE == MODE_CONV && FAST))) {
    if (dtl_enabled()) return launch_dtl<MODE, EPI, ACT>(device, a, batch, s);
  }
  switch (pick_tile(MODE, a.M, a.N, batch)) {
    case T128x128:
      return launch_tile<T, 128, 128, MODE, EPI, ACT, FAST>(device, a, batch, s);
    case T128x64w4:
      return launch_tile<T, 128, 64, MODE, EPI, ACT, FAST, 4>(device, a, batch, s);
    case T64x128w1:
      return launch_tile<T, 64, 128, MODE, EPI, ACT, FAST, 1>(device, a, batch, s);
    default:
      return launch_tile<T, 64, 64, MODE, EPI, ACT, FAST>(device, a, batch, s);
  }
}

template <typename T, int MODE, int EPI, bool FAST>
int launch_gemm_fast(int device, const GemmArgs& a, int64_t batch, hipStream_t s) {
  if constexpr (EPI == EPI_LINEAR) {
    switch (a.act) {
      case MTHIP_ACT_GELU:
        return launch_gemm_tiles<T, MODE, EPI, MTHIP_ACT_GELU, FAST>(device, a, batch, s);
      case MTHIP_ACT_GELU_TANH:
        return launch_gemm_tiles<T, MODE, EPI, MTHIP_ACT_GELU_TANH, FAST>(device, a, batch, s);
      case MTHIP_ACT_SILU:
        return launch_gemm_tiles<T, MODE, EPI, MTHIP_ACT_SILU, FAST>(device, a, batch, s);
      default:
        break;
    }
  }
  return launch_gemm_tiles<T, MODE, EPI, MTHIP_ACT_NONE, FAST>(device, a, batch, s);
}

template <typename T, int MODE, int EPI>
int launch_gemm(int device, const GemmArgs& a, int64_t batch, hipStream_t s) {
  return launch_gemm_fast<T, MODE, EPI, false>(device, a, batch, s);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// dst[b][r][c] = c < cols ? src[b*sbs + r*lds + c] : 0 for c < ldd: stages an operand whose
// rows are not whole 16-byte chunks into a zero-padded, aligned copy.
template <typename T>
__global__ void pad_rows_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t rows, int64_t cols,
                                int64_t lds, int64_t sbs, int64_t ldd) {
  const int64_t b = blockIdx.y;
  const int64_t n = rows * ldd;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / ldd, c = i - r * ldd;
    dst[b * n + i] = c < cols ? src[b * sbs + r * lds + c] : T(0);
  }
}

// Stages `rows x cols` (row stride lds, batch stride sbs, `batches` copies) into a fresh
// buffer with rows padded to `ldd` elements.  Returns 0 and the buffer (owned by the caller).
template <typename T>
int pad_operand(int device, hipStream_t s, const void* src, int64_t batches, int64_t rows, int64_t cols, int64_t lds,
                int64_t sbs, int64_t ldd, void** out) {
  if (int rc = mthip_malloc(device, (size_t)(batches * rows * ldd) * sizeof(T), out)) return rc;
  const int64_t n = rows * ldd;
  const unsigned g = (unsigned)std::min<int64_t>(std::max<int64_t>(ceil_div(n, 256), 1), 2048);
  hipLaunchKernelGGL(pad_rows_kernel<T>, dim3(g, (unsigned)batches), dim3(256), 0, s, (const T*)src, (T*)*out, rows,
                     cols, lds, sbs, ldd);
  return check_launch("pad_rows_kernel");
}

constexpr int64_t kMaxBufferBytes = (int64_t(1) << 31) - 1;

// fp16 gelu of every half value, as mtorch's fp16 path computes it (tensor.cpp:17225-17235):
// a GEGLU gate is always an fp16 value, so the fused epilogue looks its gelu up instead of
// evaluating a double-precision erf per element.  Filled once per device.
__device__ __align__(16) uint16_t g_gelu_f16_table[65536];

__global__ void gelu_f16_table_kernel(uint16_t* tab) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 65536) tab[i] = f2h_fast(gelu_ref_f16(h2f_exact((uint16_t)i)));
}

const uint16_t* gelu_f16_table(int device, hipStream_t s) {
  static const uint16_t* ptr[64] = {nullptr};
  static std::mutex init_mutex;  // first use from several host threads fills the table once
  if (device < 0 || device >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(init_mutex);
  if (!ptr[device]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_gelu_f16_table)) != hipSuccess) return nullptr;
    hipLaunchKernelGGL(gelu_f16_table_kernel, dim3(256), dim3(256), 0, s, static_cast<uint16_t*>(p));
    if (hipGetLastError() != hipSuccess) return nullptr;
    // Under stream capture the fill is only recorded (it runs with each replay, ahead of the
    // GEMM that reads the table), so the table counts as ready only after an eager fill.
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) return nullptr;
    if (st != hipStreamCaptureStatusNone) return static_cast<const uint16_t*>(p);
    ptr[device] = static_cast<const uint16_t*>(p);
  }
  return ptr[device];
}

}  // namespace

const uint16_t* gelu_f16_lookup(int device, hipStream_t s) { return gelu_f16_table(device, s); }

// Shared with conv.hip.  The fast im2col (tap bitmasks) needs Cp % BK == 0 and <= 32 taps.
int launch_conv_gemm(int device, int dtype, const GemmArgs& a, hipStream_t s) {
  // With the padded channel count a multiple of BK, no K tile straddles two filter taps.
  if (dtype == MTHIP_F16) {
    if (a.Cp % Mfma<uint16_t>::BK == 0 && a.KH_ * a.KW <= 32)
      return launch_gemm_fast<uint16_t, MODE_CONV, EPI_CONV, true>(device, a, 1, s);
    return launch_gemm_fast<uint16_t, MODE_CONV, EPI_CONV, false>(device, a, 1, s);
  }
  if (a.Cp % Mfma<float>::BK == 0 && a.KH_ * a.KW <= 32)
    return launch_gemm_fast<float, MODE_CONV, EPI_CONV, true>(device, a, 1, s);
  return launch_gemm_fast<float, MODE_CONV, EPI_CONV, false>(device, a, 1, s);
}

namespace {

// c = narrow(beta * c_in) (0 without c_in): addmm / baddbmm at alpha = 0, where the reference
// skips the product (tensor.cpp:25320, 25621), so an inf or NaN in the operands never reaches the
// output while one in c_in does (0 * inf = NaN even at beta = 0, tensor.cpp:25256).
template <typename T>
__global__ __launch_bounds__(256) void gemm_beta_only_kernel(const GemmArgs a, int64_t batch) {
  const int64_t total = batch * a.M * a.N;
  const T* cin = reinterpret_cast<const T*>(a.c_in);
  T* c = reinterpret_cast<T*>(a.c);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t col = i % a.N, t = i / a.N, row = t % a.M, bz = t / a.M;
    const float v = cin ? a.beta * Elem<T>::load(cin, bz * a.stride_c_in + row * a.c_in_rs + col * a.c_in_cs) : 0.0f;
    Elem<T>::store(c, bz * a.stride_c + row * a.ldc + col, v);
  }
}

}  // namespace

// The streamed-kernel launcher for linears (linear_stream.hip); -1 where it does not apply.
int try_stream_linear(int device, const GemmArgs& a, hipStream_t s);

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
  if (dtype == MTHIP_F16 && act == MTHIP_ACT_GELU) {
    a.gelu_tab = gelu_f16_table(device, s);
    if (!a.gelu_tab) return fail(MTHIP_ERR_HIP, "mthip_linear: gelu table setup failed");
  }
  const int vec = dtype == MTHIP_F16 ? 8 : 4;
  const int64_t es = dtype == MTHIP_F16 ? 2 : 4;
  const bool vec_ok = aligned16(x) && aligned16(w) && lda % vec == 0 && ldw % vec == 0 && K % vec == 0;
  void* xp = nullptr;
  void* wp = nullptr;
  if (!vec_ok) {
    // Zero-padded aligned copies of both operands (K rounded up to a whole chunk).
    const int64_t Kp = ceil_div(K, vec) * vec;
    int rc = dtype == MTHIP_F16 ? pad_operand<uint16_t>(device, s, x, 1, M, K, lda, 0, Kp, &xp)
                                : pad_operand<float>(device, s, x, 1, M, K, lda, 0, Kp, &xp);
    if (rc == MTHIP_OK)
      rc = dtype == MTHIP_F16 ? pad_operand<uint16_t>(device, s, w, 1, N, K, ldw, 0, Kp, &wp)
                              : pad_operand<float>(device, s, w, 1, N, K, ldw, 0, Kp, &wp);
    if (rc != MTHIP_OK) {
      mthip_free(device, xp);
      return rc;
    }
    a.a = xp;
    a.b = wp;
    a.lda = a.ldb = Kp;
    a.K = Kp;
  }
  a.a_bytes = ((M - 1) * a.lda + a.K) * es;
  a.b_bytes = ((N - 1) * a.ldb + a.K) * es;
  int rc;
  if (a.a_bytes > kMaxBufferBytes || a.b_bytes > kMaxBufferBytes)
    rc = fail(MTHIP_ERR_UNSUPPORTED, "mthip_linear: operands above 2 GiB are not supported");
  else if (dtype == MTHIP_F16) {
    rc = (act == MTHIP_ACT_NONE || act == MTHIP_ACT_GELU) ? try_stream_linear(device, a, s) : -1;
    if (rc < 0) rc = launch_gemm<uint16_t, MODE_NT, EPI_LINEAR>(device, a, 1, s);
  } else {
    rc = launch_gemm<float, MODE_NT, EPI_LINEAR>(device, a, 1, s);
  }
  mthip_free(device, xp);  // stream-ordered: reused only by later work
  mthip_free(device, wp);
  return rc;
}

int mthip_linear_geglu(int device, int dtype, const void* x, int64_t lda, const void* w, const void* b, void* y,
                       int64_t ldy, int64_t M, int64_t N, int64_t K) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_linear_geglu: dtype must be F16 or F32");
  MTHIP_REQUIRE(M >= 0 && N >= 0 && K >= 0 && N % 32 == 0, "mthip_linear_geglu: N must be a multiple of 32");
  MTHIP_REQUIRE(lda >= K && ldy >= N, "mthip_linear_geglu: leading dimension smaller than the row");
  const int vec = dtype == MTHIP_F16 ? 8 : 4;
  MTHIP_REQUIRE(aligned16(x) && aligned16(w) && lda % vec == 0 && K % vec == 0,
                "mthip_linear_geglu: operands must be 16-byte aligned with K a multiple of 16 bytes");
  if (M == 0 || N == 0) return MTHIP_OK;
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  const int64_t es = dtype == MTHIP_F16 ? 2 : 4;
  GemmArgs a{};
  a.M = M;
  a.N = 2 * N;  // interleaved value/gate columns
  a.K = K;
  a.a = x;
  a.lda = lda;
  a.b = w;
  a.ldb = K;
  a.c = y;
  a.ldc = ldy;
  a.bias = b;
  a.a_bytes = ((M - 1) * lda + K) * es;
  a.b_bytes = (2 * N * K) * es;
  MTHIP_REQUIRE(a.a_bytes <= kMaxBufferBytes && a.b_bytes <= kMaxBufferBytes,
                "mthip_linear_geglu: operands above 2 GiB are not supported");
  if (dtype == MTHIP_F16) {
    a.gelu_tab = gelu_f16_table(device, s);
    if (!a.gelu_tab) return fail(MTHIP_ERR_HIP, "mthip_linear_geglu: gelu table setup failed");
    if (dtl_enabled()) return launch_dtl<MODE_NT, EPI_GEGLU, MTHIP_ACT_NONE>(device, a, 1, s);
    return launch_tile<uint16_t, 128, 64, MODE_NT, EPI_GEGLU, MTHIP_ACT_NONE, false, 4>(device, a, 1, s);
  }
  return launch_tile<float, 128, 64, MODE_NT, EPI_GEGLU, MTHIP_ACT_NONE, false, 4>(device, a, 1, s);
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
  if (alpha == 0.0) {
    const int64_t total = batch * M * N;
    const unsigned grid = (unsigned)std::min<int64_t>(ceil_div(total, 256), 4096);
    if (dtype == MTHIP_F16)
      hipLaunchKernelGGL(gemm_beta_only_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, a, batch);
    else
      hipLaunchKernelGGL(gemm_beta_only_kernel<float>, dim3(grid), dim3(256), 0, s, a, batch);
    return check_launch("gemm_beta_only_kernel");
  }
  const int vec = dtype == MTHIP_F16 ? 8 : 4;
  const int64_t es = dtype == MTHIP_F16 ? 2 : 4;
  const int64_t b_cols = b_trans ? K : N;   // contiguous extent of a B row
  const int64_t b_rows = b_trans ? N : K;
  bool a_ok = aligned16(a_ptr) && lda % vec == 0 && stride_a % vec == 0 && K % vec == 0;
  bool b_ok = aligned16(b_ptr) && ldb % vec == 0 && stride_b % vec == 0 && b_cols % vec == 0;
  void* ap = nullptr;
  void* bp = nullptr;
  int rc = MTHIP_OK;
  if (!a_ok || !b_ok) {
    // Zero-padded aligned copies; K (and, for a [K, N] B, N) rounded up to whole chunks.
    const int64_t Kp = ceil_div(K, vec) * vec;
    const int64_t a_batches = stride_a == 0 ? 1 : batch, b_batches = stride_b == 0 ? 1 : batch;
    rc = dtype == MTHIP_F16 ? pad_operand<uint16_t>(device, s, a_ptr, a_batches, M, K, lda, stride_a, Kp, &ap)
                            : pad_operand<float>(device, s, a_ptr, a_batches, M, K, lda, stride_a, Kp, &ap);
    const int64_t bcp = ceil_div(b_cols, vec) * vec;
    if (rc == MTHIP_OK)
      rc = dtype == MTHIP_F16 ? pad_operand<uint16_t>(device, s, b_ptr, b_batches, b_rows, b_cols, ldb, stride_b, bcp, &bp)
                              : pad_operand<float>(device, s, b_ptr, b_batches, b_rows, b_cols, ldb, stride_b, bcp, &bp);
    if (rc == MTHIP_OK) {
      a.a = ap;
      a.lda = Kp;
      a.stride_a = stride_a == 0 ? 0 : M * Kp;
      a.b = bp;
      a.ldb = bcp;
      a.stride_b = stride_b == 0 ? 0 : b_rows * bcp;
      // K-padding of a [K, N] B adds zero rows: extend K only when both operands carry it.
      if (b_trans) a.K = Kp;
    }
  }
  if (rc == MTHIP_OK) {
    // A row is read in whole 16-byte chunks and the buffer range check drops any dword that
    // crosses a_bytes, so the extent covers the last row's final chunk (the padded copy holds
    // zeros there; unpadded rows have K a multiple of the chunk).
    a.a_bytes = ((M - 1) * a.lda + ceil_div(a.K, vec) * vec) * es;
    a.b_bytes = b_trans ? ((N - 1) * a.ldb + a.K) * es : ((K - 1) * a.ldb + ceil_div(N, vec) * vec) * es;
    if (a.a_bytes > kMaxBufferBytes || a.b_bytes > kMaxBufferBytes) {
      rc = fail(MTHIP_ERR_UNSUPPORTED, "mthip_gemm: operands above 2 GiB per batch are not supported");
    } else if (b_trans) {
      rc = dtype == MTHIP_F16 ? launch_gemm<uint16_t, MODE_NT, EPI_GEMM>(device, a, batch, s)
                              : launch_gemm<float, MODE_NT, EPI_GEMM>(device, a, batch, s);
    } else {
      rc = dtype == MTHIP_F16 ? launch_gemm<uint16_t, MODE_NN, EPI_GEMM>(device, a, batch, s)
                              : launch_gemm<float, MODE_NN, EPI_GEMM>(device, a, batch, s);
    }
  }
  mthip_free(device, ap);
  mthip_free(device, bp);
  return rc;
}

}  // extern "C"
