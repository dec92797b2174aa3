// fp16 MFMA GEMM with direct-to-LDS operand loads (gfx950), for the k-contiguous operand
// sources: x.W^T (MODE_NT) and the implicit im2col of an NHWC activation whose padded channel
// count is a multiple of the K tile (MODE_CONV, at most 32 filter taps).  Same work
// decomposition, unit order, split-K and epilogues as gemm_kernel in gemm_core.h; what differs
// is how K tiles reach LDS.
//
// Operands go global -> LDS with buffer_load_dwordx4 ... lds: each instruction moves 64 x 16 B,
// lane l's 16 bytes landing at LDS base + 16*l, so a wave instruction fills 8 consecutive
// 128-byte tile rows (one K tile = 64 halves per row).  No registers stage the data and no
// ds_write is issued; the K position is the instruction's scalar offset, so stepping K costs no
// vector instructions for A and for linear B.  LDS rows are unpadded with the 16-byte chunk c
// of row r stored at chunk c ^ ((r >> 1) & 7): LDS serves 256 bytes per clock (64 banks), and
// the 16 lanes of one ds_read_b128 pass -- rows r..r+15 of one fragment column -- then cover
// all 64 banks.  The swizzle is applied on the global side: lane l of an instruction fetches
// the logical chunk that belongs at its fixed LDS slot.
//
// K tiles rotate through S stages (S-1 tiles in flight while one is multiplied); each stage is a
// separate LDS array selected by a compile-time stage number, so every LDS address is a
// register plus an immediate.  Per step: wait until this wave's loads of the step have landed
// (an explicit vmcnt wait: see dma16 for why the compiler's own is kept out), barrier
// (everyone's have, and everyone has finished reading the stage about to be refilled), issue
// the loads S-1 steps ahead, multiply.
#pragma once

#include <type_traits>

#include "gemm_core.h"

namespace mthip {

template <int N>
using ic = std::integral_constant<int, N>;

// s_waitcnt immediate that waits for vmcnt <= n only (expcnt and lgkmcnt left at their maxima).
constexpr int vmcnt_only(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

// LDS byte address of a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(uint8_t* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)p;
}

// One 64 x 16-byte direct-to-LDS load: lane l's 16 bytes from buffer offset voff + soff land at
// LDS byte address lds + 16*l.  The LDS address reaches the instruction through readfirstlane,
// which the compiler cannot see through: the load then carries no alias scope, and the
// compiler's wait insertion does not tie later LDS reads to it (it cannot tell the stage arrays
// apart across the unrolled loop and would wait for loads of the next stage too).  Ordering is
// the kernel's own: every stage is read only after an explicit vmcnt wait and a barrier.
__device__ __forceinline__ void dma16(const __amdgpu_buffer_rsrc_t& r, uint32_t lds, uint32_t voff, uint32_t soff) {
  const uint32_t a = __builtin_amdgcn_readfirstlane(lds);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(uintptr_t)a, 16, voff, soff, 0,
                                           0);
}

template <int BM, int BN, int WGM, int MODE, int EPI, int ACT, int S>
__global__ __launch_bounds__(256) void gemm_dtl_kernel(const GemmArgs args) {
  using T = uint16_t;
  constexpr int BK = 64;  // halves per K tile: 128-byte LDS rows
  constexpr int WGN = 4 / WGM;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int AI = BM / 32, BI = BN / 32;  // 8-row DMA instructions per wave per K tile
  constexpr int L = AI + BI;                 // loads per wave per K tile
  static_assert(MODE == MODE_NT || MODE == MODE_CONV, "k-contiguous operands only");
  static_assert(S >= 2 && S <= 4, "2..4 stages");
  static_assert(FM >= 1 && FN >= 1 && WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert((S - 2) * L <= 63, "vmcnt range");

  __shared__ __align__(16) uint8_t sa0[BM * 128], sa1[BM * 128], sa2[S > 2 ? BM * 128 : 16], sa3[S > 3 ? BM * 128 : 16];
  __shared__ __align__(16) uint8_t sb0[BN * 128], sb1[BN * 128], sb2[S > 2 ? BN * 128 : 16], sb3[S > 3 ? BN * 128 : 16];
  auto SA = [&](auto st) -> uint8_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sa0;
    else if constexpr (s == 1) return sa1;
    else if constexpr (s == 2) return sa2;
    else return sa3;
  };
  auto SB = [&](auto st) -> uint8_t* {
    constexpr int s = decltype(st)::value;
    if constexpr (s == 0) return sb0;
    else if constexpr (s == 1) return sb1;
    else if constexpr (s == 2) return sb2;
    else return sb3;
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS targets are scalar
  const int wm = wave % WGM, wn = wave / WGM;
  const uint32_t G = gridDim.x;
  const uint32_t nk_total = (uint32_t)ceil_div(args.K, BK);
  constexpr uint32_t kOOB = 0x80000000u;  // beyond every buffer: the range check returns zeros

  // Tile row and logical chunk of this lane in DMA instruction i of an operand issuing I
  // instructions per wave: rows (wave*I + i)*8 .. +8, lane l at row +l/8, LDS chunk l%8.
  auto dma_row = [&](int I, int i) { return (wave * I + i) * 8 + (lane >> 3); };
  auto dma_chunk = [&](int row) { return (lane & 7) ^ ((row >> 1) & 7); };

  // ---- loader state (the unit whose tiles are being fetched).  All extents, offsets and
  //      counters are 32-bit: the launcher keeps units, rows and columns below 2^31 and both
  //      operands below 2 GiB.
  const int M = (int)args.M, N = (int)args.N, K = (int)args.K;
  const uint32_t units = (uint32_t)args.units;
  const bool k_tail = (K % BK) != 0;
  __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
  uint32_t a_off[AI], b_off[BI];
  int a_kc[AI], b_kc[BI];  // element k offset of the lane's chunk (K tails)
  int c_base[MODE == MODE_CONV ? BI : 1];
  uint32_t c_mask[MODE == MODE_CONV ? BI : 1];
  // conv: the loader tile's tap (bit index into c_mask), its kx, channel offset within the tap,
  // and the tap's element offset (ky*dh*W + kx*dw)*Cp relative to tap (0, 0)
  int l_tap = 0, l_kx = 0, l_ch = 0, l_tap_el = 0;
  uint32_t l_u = blockIdx.x;
  int l_k = 0, l_nkt = 1;
  uint32_t l_kb = 0;  // byte offset of the loader's K tile along a row
  int l_kleft = 0;    // K - k0 of the loader's K tile

  // A unit's tile origin, K range and batch.  A loader past the last unit gets out-of-range
  // offsets and a K range it never leaves, so the step path needs no liveness tests.  The
  // body is straight-line (the dead case is selects over the last unit's values): with an early
  // return the compiler merges differing stores through a selected address and the loader
  // state ends up in scratch memory.
  auto set_loader = [&]() {
    const bool dead = l_u >= units;
    const GemmUnit un = decode_unit<BM, BN>(args, dead ? units - 1 : l_u, nk_total);
    const int m0 = (int)un.m0, n0 = (int)un.n0, kt0 = (int)un.kt0;
    l_nkt = dead ? 0x7fffffff : (int)un.nkt;
    l_kb = (uint32_t)kt0 * (BK * 2);
    l_kleft = dead ? 0 : K - kt0 * BK;
    a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const T*>(args.a) + un.bz * args.stride_a), (short)0, (int)args.a_bytes, 0x00020000);
    b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const T*>(args.b) + (MODE == MODE_CONV ? 0 : un.bz * args.stride_b)), (short)0,
        (int)args.b_bytes, 0x00020000);
    // Row r = (wave*I + i)*8 + l/8 of instruction i: its chunk is (l & 7) ^ (l / 16) ^ 4 when
    // wave*I + i is odd (8 | 8(wave*I + i)), so the byte offset is one per-lane multiply plus
    // wave-uniform steps.
    const uint32_t lda2 = (uint32_t)args.lda * 2u;
    const uint32_t a_lane = (uint32_t)(m0 + dma_row(AI, 0)) * lda2;
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const int r = dma_row(AI, i), c = dma_chunk(r);
      a_kc[i] = c * 8;
      a_off[i] = m0 + r < M && !dead ? a_lane + (uint32_t)(i * 8) * lda2 + (uint32_t)c * 16u : kOOB;
    }
    if constexpr (MODE == MODE_NT) {
      const uint32_t ldb2 = (uint32_t)args.ldb * 2u;
      const uint32_t b_lane = (uint32_t)(n0 + dma_row(BI, 0)) * ldb2;
#pragma unroll
      for (int i = 0; i < BI; ++i) {
        const int r = dma_row(BI, i), c = dma_chunk(r);
        b_kc[i] = c * 8;
        b_off[i] = n0 + r < N && !dead ? b_lane + (uint32_t)(i * 8) * ldb2 + (uint32_t)c * 16u : kOOB;
      }
    } else {
      const int H = (int)args.H, W = (int)args.W, KW = (int)args.KW, KH = (int)args.KH_, Cp = (int)args.Cp;
      const int dh = (int)args.dh, dw = (int)args.dw, sh = (int)args.sh, sw = (int)args.sw;
      const int ph = (int)args.ph, pw = (int)args.pw;
#pragma unroll
      for (int i = 0; i < BI; ++i) {
        const int r = dma_row(BI, i), c = dma_chunk(r);
        b_kc[i] = c * 8;
        const int p = n0 + r;
        const bool ok = p < N;
        const uint32_t pp = ok ? (uint32_t)p : 0u;
        const uint32_t img = args.div_ohw.div(pp), pix = pp - img * args.div_ohw.d;
        const uint32_t oyu = args.div_ow.div(pix);
        const int iy0 = (int)oyu * sh - ph;
        const int ix0 = (int)(pix - oyu * args.div_ow.d) * sw - pw;
        // element offset of x_nhwc[img, iy0, ix0, 8c] (negative in the padding; only taps that
        // land inside the image are turned into an address)
        c_base[i] = ok ? (((int)img * H + iy0) * W + ix0) * Cp + c * 8 : 0;
        uint32_t cols = 0;
        for (int kx = 0; kx < KW; ++kx) {
          const int ix = ix0 + kx * dw;
          cols |= (ix >= 0 && ix < W ? 1u : 0u) << kx;
        }
        uint32_t m = 0;
        for (int ky = 0; ky < KH; ++ky) {
          const int iy = iy0 + ky * dh;
          m |= (iy >= 0 && iy < H ? cols : 0u) << (ky * KW);
        }
        c_mask[i] = ok && !dead ? m : 0u;
      }
      const int k0 = kt0 * BK;
      l_tap = k0 / Cp;
      l_ch = k0 - l_tap * Cp;
      const int ky = l_tap / KW;
      l_kx = l_tap - ky * KW;
      l_tap_el = (ky * dh * W + l_kx * dw) * Cp;
    }
  };
  set_loader();

  // Issues the loader cursor's K tile into stage st and advances the cursor.  Every step issues
  // exactly L loads per wave (zeros past the last unit), which the vmcnt accounting relies on.
  auto issue = [&](auto st) {
    const uint32_t sa = lds_addr(SA(st)), sb = lds_addr(SB(st));
    const uint32_t kb = l_kb;
    if constexpr (MODE == MODE_NT) {
      if (!k_tail || l_kleft >= BK) {
#pragma unroll
        for (int i = 0; i < AI; ++i) dma16(a_rsrc, sa + (wave * AI + i) * 1024, a_off[i], kb);
#pragma unroll
        for (int i = 0; i < BI; ++i) dma16(b_rsrc, sb + (wave * BI + i) * 1024, b_off[i], kb);
      } else {
        // the last tile of an unaligned K: a chunk past K would read the next row's data
#pragma unroll
        for (int i = 0; i < AI; ++i)
          dma16(a_rsrc, sa + (wave * AI + i) * 1024, a_kc[i] < l_kleft ? a_off[i] : kOOB, kb);
#pragma unroll
        for (int i = 0; i < BI; ++i)
          dma16(b_rsrc, sb + (wave * BI + i) * 1024, b_kc[i] < l_kleft ? b_off[i] : kOOB, kb);
      }
    } else {
      // K = taps * Cp is a whole number of tiles and a tile never straddles two taps.
#pragma unroll
      for (int i = 0; i < AI; ++i) dma16(a_rsrc, sa + (wave * AI + i) * 1024, a_off[i], kb);
      const uint32_t chb = (uint32_t)l_ch * 2u;
#pragma unroll
      for (int i = 0; i < BI; ++i) {
        const bool in = (c_mask[i] >> l_tap) & 1u;
        dma16(b_rsrc, sb + (wave * BI + i) * 1024, in ? (uint32_t)(c_base[i] + l_tap_el) * 2u : kOOB, chb);
      }
      // Advance (channel, tap) with selects: a branchy update lets the compiler merge the
      // counters' stores through a selected address, which keeps them out of registers.
      const int Cp = (int)args.Cp;
      const int nch = l_ch + BK;
      const bool next_tap = nch == Cp;
      const int nkx = l_kx + (next_tap ? 1 : 0);
      const bool next_row = nkx == (int)args.KW;
      l_ch = next_tap ? 0 : nch;
      l_tap += next_tap ? 1 : 0;
      l_kx = next_row ? 0 : nkx;
      l_tap_el += (next_tap ? (int)args.dw * Cp : 0) +
                  (next_row ? ((int)args.dh * (int)args.W - (int)args.KW * (int)args.dw) * Cp : 0);
    }
    l_kb += BK * 2;
    l_kleft -= BK;
    if (++l_k == l_nkt) {
      l_k = 0;
      l_u += G;
      set_loader();
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

  // Fragment reads: lane l reads row (l%32) of each 32-row block at logical chunk 2*kk + l/32.
  // The blocks start at multiples of 32 rows, so the swizzle term is ((l%32) >> 1) & 7 for all.
  int a_rd[4], b_rd[4];
  {
    const int sw = ((lane & 31) >> 1) & 7, hi = lane >> 5;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      a_rd[kk] = (wm * WM + (lane & 31)) * 128 + (((2 * kk + hi) ^ sw) << 4);
      b_rd[kk] = (wn * WN + (lane & 31)) * 128 + (((2 * kk + hi) ^ sw) << 4);
    }
  }
  auto compute = [&](auto st) {
    const uint8_t* sa = SA(st);
    const uint8_t* sb = SB(st);
    halfx8 af[4][FM], bf[4][FN];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int i = 0; i < FM; ++i) af[kk][i] = *reinterpret_cast<const halfx8*>(sa + a_rd[kk] + i * 32 * 128);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[kk][j] = *reinterpret_cast<const halfx8*>(sb + b_rd[kk] + j * 32 * 128);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[kk][j], af[kk][i], acc[i][j], 0, 0, 0);
  };

  uint32_t c_u = blockIdx.x;
  if (c_u >= units) return;  // (the launcher sizes the grid to at most `units`)
  int c_k = 0;
  int c_nkt = (int)decode_unit<BM, BN>(args, c_u, nk_total).nkt;

  auto step = [&](auto st) -> bool {
    constexpr int s = decltype(st)::value;
    __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 2) * L));
    __builtin_amdgcn_s_barrier();
    issue(ic<(s + S - 1) % S>{});
    compute(st);
    if (++c_k == c_nkt) {
      gemm_finish_unit<T, BM, BN, WGM, EPI, ACT>(args, decode_unit<BM, BN>(args, c_u, nk_total), acc, lane, wm, wn);
      zero_acc();
      c_k = 0;
      c_u += G;
      if (c_u >= units) return false;
      c_nkt = (int)decode_unit<BM, BN>(args, c_u, nk_total).nkt;
    }
    return true;
  };

  issue(ic<0>{});
  if constexpr (S > 2) issue(ic<1>{});
  if constexpr (S > 3) issue(ic<2>{});
  while (true) {
    if (!step(ic<0>{})) break;
    if (!step(ic<1>{})) break;
    if constexpr (S > 2)
      if (!step(ic<2>{})) break;
    if constexpr (S > 3)
      if (!step(ic<3>{})) break;
  }
  // DMA writes still in flight target this workgroup's LDS: let them land before it is released.
  __builtin_amdgcn_s_waitcnt(0);
}

}  // namespace mthip
