// 3x3 stride-1 pad-1 conv (fp16, NHWC input with Cp % 64 == 0) on MFMA, with the input halo
// kept in LDS across the nine filter taps.
//
//   Y[o, y, x] = sum_{cb, ky, kx, c < 64} Wp[o, ky, kx, 64cb + c] * X[img, y + ky - 1, x + kx - 1, 64cb + c]
//
// A workgroup computes one unit: BM output channels x TR output rows x TW (= W) columns of one
// image, over a range of 64-channel blocks (all of them, or one K slice when the launcher splits
// K).  Per channel block it stages the input patch -- (TR+2) x (TW+2) pixels x 64 channels, zero
// outside the image -- into LDS once, and the nine taps then read their fragments from it at
// shifted pixel positions; only the weights stream per tap.  Against an im2col tile, which
// fetches every input pixel once per tap, this divides the activation bytes from L2 by about
// 9 / (1 + 2/TR): at TR = 2 a unit moves 126 KB per 64 channels for 11.8 MFLOP (94 FLOP/B)
// where a 64x64 im2col tile moves 16 KB per 0.5 MFLOP (32 FLOP/B).
//
// Four compute waves, one per SIMD, and one or two producer waves that issue every load.
// Operands go global -> LDS with direct-to-LDS buffer loads (no staging registers, no
// ds_write): an instruction moves 64 x 16 B, i.e. eight 128-byte rows (one row = one pixel's or
// one output channel's 64 channels), with row r's 16-byte chunk c stored at chunk c ^ ((r >> 1)
// & 7) so that the 16 lanes of one ds_read_b128 pass (16 consecutive rows, one logical chunk)
// cover all 64 banks whatever row they start at.  Pixels outside the image (the padding) and
// rows past the last output channel are fetched from an out-of-range offset, which the buffer
// range check turns into zeros.  Issuing a load costs the issuing wave tens of cycles; on the
// compute waves that time would come out of the MFMA pipe, so the compute waves issue none.
//
// MFMA: v_mfma_f32_16x16x32_f16 with the pixel fragment as the A operand (16 pixels x 32 k) and
// the weight fragment as B (32 k x 16 channels), so lane l's accumulator holds pixels
// 4*(l/16) .. +3 of channel l%16: four consecutive pixels of one NCHW row, stored as 8 bytes.
// The compute waves split the unit WGM (channels) x 4/WGM (pixels).
//
// Pipeline (one step = one tap of one channel block, 2 x 32 k).  The producer's slot for step s
// (after the barrier that opens it) issues the weights of step s + SW - 1 into a ring of SW
// stages and, in the slots of taps 0..6 of channel block j, a seventh of block j + 1's patch into
// the other of two patch buffers.  Before each barrier the producer waits (a compile-time vmcnt
// per tap) until the next step's operands have landed; the compute waves wait until their LDS
// reads of the current step are in registers, so after the barrier the stage about to be
// refilled is free.  A compute wave's step is then one straight-line block: the LDS reads of
// step s + 1 into its other fragment register set, interleaved one-to-one with the MFMAs of
// step s.
#pragma once

#include "gemm_core.h"
#include "gemm_dtl.h"

namespace mthip {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct HaloArgs {
  const void* x;  // NHWC [B][H][W][Cp]
  const void* w;  // packed [O][3][3][Cp]
  void* y;        // NCHW [B][O][H][W]
  const void* bias;
  const void* residual;  // NCHW like y, or null
  const void* chan_add;  // [B][chan_add_ld], or null
  int chan_add_ld;
  int B, H, W, Cp, O;
  int tiles_m, row_blocks, ksplit, cb_per_split, units;
  int img_fast;  // 1: the image index varies fastest in the unit order (units that share weights adjacent)
  int x_bytes, w_bytes;
  float* partial;  // ksplit > 1: [ksplit][O][ld_partial] fp32, columns = img*H*W + pixel
  int ld_partial;
};

// Load bookkeeping of producer wave P of NPW, fixed at compile time.  LW weight instructions per
// slot; the next block's LP patch instructions spread over the slots of taps 0..6 (PPS per
// slot), each slot issuing its patch part ahead of its weights.  Producer P issues the
// instructions gi with gi % NPW == P of every slot, and waits only for its own.  TR, PW: output
// rows and patch row width of the unit (patch instruction gi holds patch pixels 8gi .. 8gi+7,
// row-major).
template <int LW, int LP, int SW, int NPW, int P, int TR, int PW, int PD>
struct HaloSchedule {
  static constexpr int PPS = (LP + 6) / 7;
  static constexpr int patch_in(int tap) {
    return tap > 6 ? 0 : (LP - tap * PPS < 0 ? 0 : (LP - tap * PPS < PPS ? LP - tap * PPS : PPS));
  }
  static constexpr int mine(int g0, int g1) {  // instructions gi in [g0, g1) with gi % NPW == P
    int n = 0;
    for (int gi = g0; gi < g1; ++gi) n += gi % NPW == P ? 1 : 0;
    return n;
  }
  static constexpr int w_loads() { return mine(0, LW); }
  static constexpr int p_loads(int tap) { return mine(tap * PPS, tap * PPS + patch_in(tap)); }
  static constexpr int slot_loads(int tap) { return w_loads() + p_loads(tap); }
  static constexpr int last_patch_tap() {
    int t = 0;
    for (int tap = 0; tap <= 6; ++tap)
      if (p_loads(tap) > 0) t = tap;
    return t;
  }
  // Loads allowed in flight at the wait that precedes step s (tap T): the weights of step s were
  // the last load of the slot of step s - SW + 1, so every load of slots s - SW + 2 .. s - 1 may
  // still be in flight; at tap 0 the block's patch must have landed too, whose last part was
  // issued in the slot of tap last_patch_tap() of the previous block, ahead of that slot's
  // weights.
  static constexpr int pending(int T) {
    int n = 0;
    for (int d = 1; d <= SW - 2; ++d) n += slot_loads((T - d + 18) % 9);
    if (T == 0) {
      int m = w_loads();
      for (int t = last_patch_tap() + 1; t <= 8; ++t) m += slot_loads(t);
      n = n < m ? n : m;
    }
    return n;
  }
  // Patch instructions that tap t reads: the pixels of patch rows 0 .. t/3 + TR - 1.
  static constexpr int need(int t) {
    const int n = ((t / 3 + TR) * PW + 7) / 8;
    return n < LP ? n : LP;
  }
  // The first channel block has no previous block to stream its patch under.  Its loads go out
  // in row order with each tap's rows ahead of that tap's weights (pre(k): taps k = 0 .. SW-2),
  // then the rest of the patch; the prologue issues pre(0 .. PD-1) only, and the slot of step
  // s issues pre(PD + s) (with the rest of the patch after pre(SW-2)) ahead of its own loads,
  // so that step 0 waits only for the top TR rows and tap 0's weights and the first block's
  // ~80 KB spread over its first slots instead of all being requested before step 0 can
  // start.  Loads allowed in flight at the wait that precedes step T of that block:
  // everything this producer issued after its last load that step T reads.
  static constexpr int first_pending(int T) {
    int pos = 0, req = 0, pi = 0;
    const int nT = need(T);
    for (int s = -1; s < T; ++s) {  // s = -1: the prologue; s >= 0: the slot of step s
      int k_lo = 0, k_hi = 0;
      bool rest = false;
      if (s < 0) {
        k_hi = PD;
        rest = PD == SW - 1;
      } else if (PD + s <= SW - 2) {
        k_lo = PD + s;
        k_hi = k_lo + 1;
        rest = k_lo == SW - 2;
      }
      for (int k = k_lo; k < k_hi; ++k) {
        for (; pi < need(k); ++pi)
          if (pi % NPW == P) {
            ++pos;
            if (pi < nT) req = pos;
          }
        for (int g = 0; g < LW; ++g)
          if (g % NPW == P) {
            ++pos;
            if (k == T) req = pos;
          }
      }
      if (rest)
        for (; pi < LP; ++pi)
          if (pi % NPW == P) {
            ++pos;
            if (pi < nT) req = pos;
          }
      if (s >= 0) {  // the slot's own loads: block 1's patch part, then the weights of step s + SW - 1
        pos += p_loads(s);
        for (int g = 0; g < LW; ++g)
          if (g % NPW == P) {
            ++pos;
            if (s + SW - 1 == T) req = pos;
          }
      }
    }
    return pos - req;
  }
  static constexpr bool fits() {
    for (int t = 0; t < 9; ++t)
      if (pending(t) > 63 || first_pending(t) > 63) return false;
    return true;
  }
};

// HAS_A / HAS_R: the epilogue adds chan_add / residual (fixed at compile time so that the
// epilogue is one straight-line block; a K-split launch writes fp32 partials and uses neither).
// NPW producer waves (waves NW .. NW + NPW - 1) share the loads: one wave keeps at most 63
// loads in flight (the vmcnt range), which at the L2's latency under this load caps one
// producer's direct-to-LDS stream at ~25 B/clk.
template <int BM, int TR, int TW, int WGM, int SW, bool HAS_A, bool HAS_R, int NPW>
__global__ __launch_bounds__(64 * (4 + NPW)) void conv3x3_halo_kernel(const HaloArgs args) {
  constexpr int NW = 4;                 // compute waves (the others are producers)
  constexpr int WGN = NW / WGM;
  constexpr int NPX = TR * TW;          // output pixels per unit
  constexpr int PW = TW + 2, PH = TR + 2;
  constexpr int NP = PH * PW;           // patch pixels
  constexpr int WMO = BM / WGM, WNP = NPX / WGN;
  constexpr int FC = WMO / 16, FP = WNP / 16;
  constexpr int LW = BM / 8;            // weight DMA instructions per step
  constexpr int LP = (NP + 7) / 8;      // patch DMA instructions per channel block
  constexpr uint32_t WSTAGE = BM * 128, PBUF = LP * 8 * 128;
  constexpr int PD = 1;                 // pre(k) of the first block issued in the prologue
  using Sched0 = HaloSchedule<LW, LP, SW, NPW, 0, TR, PW, PD>;
  static_assert(WGM * WGN == NW && WMO % 16 == 0 && WNP % 16 == 0 && TW % 4 == 0 && BM % 8 == 0, "tile shape");
  static_assert(SW >= 3 && SW <= 9 && 18 % SW == 0, "weight ring depth: 3, 6 or 9");
  static_assert(Sched0::fits() && HaloSchedule<LW, LP, SW, NPW, NPW - 1, TR, PW, PD>::fits(), "vmcnt range");
  static_assert(PD >= 1 && PD <= SW - 1 && SW - 1 - PD <= 5, "first-block loads outside slots 0 .. 4");
  static_assert(NPW >= 1 && NPW <= 2, "one or two producer waves");
  static_assert((size_t)(2 * PBUF + SW * WSTAGE) <= 160 * 1024, "LDS");
  static_assert(PBUF < 65536 && (SW - 1) * WSTAGE < 65536, "LDS read offsets are 16-bit immediates");

  __shared__ __align__(16) uint8_t lds[2 * PBUF + SW * WSTAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr uint32_t kOOB = 0x80000000u;

  // ---- unit: (image, row block, K slice, channel tile), channel tiles fastest; units are
  //      renumbered so each XCD (workgroups dealt round-robin) takes a contiguous range.
  const uint32_t U = (uint32_t)args.units, U8 = U / 8, u0 = blockIdx.x;
  const uint32_t q = u0 < 8 * U8 ? (u0 % 8) * U8 + u0 / 8 : u0;
  // Channel tiles fastest (neighbouring units share the input rows), or with img_fast the
  // images (neighbouring units, on one XCD, share the weight slice: small images, where the
  // weights outweigh the input patch)
  uint32_t rest = q;
  int img = 0;
  if (args.img_fast) {
    img = (int)(rest % (uint32_t)args.B);
    rest /= (uint32_t)args.B;
  }
  const int mb = (int)(rest % (uint32_t)args.tiles_m);
  rest /= (uint32_t)args.tiles_m;
  const int split = (int)(rest % (uint32_t)args.ksplit);
  rest /= (uint32_t)args.ksplit;
  const int rb = (int)(rest % (uint32_t)args.row_blocks);
  if (!args.img_fast) img = (int)(rest / (uint32_t)args.row_blocks);
  const int H = args.H, W = args.W, Cp = args.Cp, O = args.O;
  const int o0 = mb * BM, y0 = rb * TR;
  const int ncb_total = Cp / 64;
  const int cb0 = split * args.cb_per_split;
  const int ncb = min(args.cb_per_split, ncb_total - cb0);
  const int HW = H * W;

  // =============================================================================== producer
  auto producer = [&](auto p_c) {
    constexpr int P = decltype(p_c)::value;
    using Sched = HaloSchedule<LW, LP, SW, NPW, P, TR, PW, PD>;
    const __amdgpu_buffer_rsrc_t x_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)args.x, (short)0, args.x_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t w_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)args.w, (short)0, args.w_bytes, 0x00020000);
    // per-lane offsets, fixed for the unit; the channel block and the tap go in soffset
    // Per-lane offsets, fixed for the unit; the channel block and the tap go in soffset.  Lane l
    // covers row 8gi + l/8 of instruction gi and 16-byte chunk (l & 7) ^ ((row >> 1) & 7), which
    // is (l & 7) ^ (l / 16) ^ 4(gi & 1) since 8 | 8gi.  Everything else that varies with gi is a
    // compile-time constant or wave-uniform, so the offsets cost one multiply per side and a few
    // adds, compares and selects per instruction (they stand between the wave's start and its
    // first load).
    const int Cp2 = Cp * 2;
    const int l3 = lane >> 3;
    const uint32_t chunk0 = (uint32_t)((lane & 7) ^ (lane >> 4)) * 16u;
    uint32_t w_off[LW], p_off[LP];
    const uint32_t wrow = 9u * (uint32_t)Cp2;  // bytes of one output channel's packed weights
    const uint32_t wlane = (uint32_t)(o0 + l3) * wrow;
#pragma unroll
    for (int gi = 0; gi < LW; ++gi)
      w_off[gi] = o0 + gi * 8 + l3 < O ? wlane + (uint32_t)(gi * 8) * wrow + (chunk0 ^ (gi & 1 ? 64u : 0u)) : kOOB;
    // Patch pixel pp = 8gi + l/8 lies in patch row pr = pp / PW, column pc = pp % PW, i.e. at
    // input pixel (y0 - 1 + pr, pc - 1).  With q = 8gi / PW and r = 8gi % PW fixed at compile
    // time, pr = q + wrap where wrap = (r + l/8 >= PW), and since the launcher sets TW == W
    // (PW = W + 2) the input pixel index is plane + pp - 2 pr with plane = (img H + y0 - 1) W - 1.
    // Offsets are computed modulo 2^32; every in-image pixel's comes out exact (< x_bytes).
    const uint32_t plane = (uint32_t)((img * H + y0 - 1) * TW - 1 + l3) * (uint32_t)Cp2;
#pragma unroll
    for (int gi = 0; gi < LP; ++gi) {
      const int q = gi * 8 / PW, r = gi * 8 % PW;
      const bool wrap = r + 7 >= PW && r + l3 >= PW;
      const int pc = r + l3 - (wrap ? PW : 0);
      const int iy = y0 - 1 + q + (wrap ? 1 : 0);
      const bool ok = (gi * 8 + 7 < NP || gi * 8 + l3 < NP) && (uint32_t)iy < (uint32_t)H && pc >= 1 && pc <= TW;
      const uint32_t off = plane + (uint32_t)(gi * 8 - 2 * q) * (uint32_t)Cp2 - (wrap ? 2u * (uint32_t)Cp2 : 0u);
      p_off[gi] = ok ? off + (chunk0 ^ (gi & 1 ? 64u : 0u)) : kOOB;
    }
    const uint32_t base = lds_addr(lds);
    // weights of step (block j2 of the slice, tap t2) into `stage`; past the slice the last block
    // is loaded again (in range, into a stage no step reads)
    auto issue_w = [&](int j2, int t2, int stage) {
      const uint32_t dst = base + 2 * PBUF + (uint32_t)stage * WSTAGE;
      const uint32_t soff = (uint32_t)((cb0 + min(j2, ncb - 1)) * 128 + t2 * Cp2);
#pragma unroll
      for (int gi = P; gi < LW; gi += NPW) dma16(w_rsrc, dst + gi * 1024, w_off[gi], soff);
    };
    // patch instructions [G0, G1) of block j2 into buffer `buf` (past the slice: the last block
    // again, into the buffer the last block does not use)
    auto issue_p = [&](auto g0_c, auto g1_c, int j2, int buf) {
      constexpr int G0 = decltype(g0_c)::value, G1 = decltype(g1_c)::value;
      const uint32_t dst = base + (uint32_t)buf * PBUF;
      const uint32_t soff = (uint32_t)(cb0 + min(j2, ncb - 1)) * 128u;
#pragma unroll
      for (int gi = G0; gi < G1; ++gi)
        if (gi % NPW == P) dma16(x_rsrc, dst + gi * 1024, p_off[gi], soff);
    };
    // block 0's patch in row order, the rows of tap k ahead of the weights of step k (pre(k),
    // k = 0 .. SW-2), then the rest of the patch: pre(0 .. PD-1) here, the others in the first
    // block's slots (first_pending counts this order)
    auto pre = [&](auto k_c) {
      constexpr int k = decltype(k_c)::value;
      issue_p(ic<k == 0 ? 0 : Sched::need(k - 1)>{}, ic<Sched::need(k)>{}, 0, 0);
      issue_w(0, k, k);
      if constexpr (k == SW - 2) issue_p(ic<Sched::need(SW - 2)>{}, ic<LP>{}, 0, 0);
    };
    pre(ic<0>{});
    if constexpr (PD > 1) pre(ic<1>{});
    if constexpr (PD > 2) pre(ic<2>{});
    if constexpr (PD > 3) pre(ic<3>{});
    if constexpr (PD > 4) pre(ic<4>{});
    if constexpr (PD > 5) pre(ic<5>{});
    if constexpr (PD > 6) pre(ic<6>{});
    if constexpr (PD > 7) pre(ic<7>{});
    // step s = 9j + T of a block of parity JP: wait for step s's operands, the barrier that
    // opens step s, then slot s
    auto slot = [&](int j, auto jp_c, auto t_c, auto first_c) {
      constexpr int JP = decltype(jp_c)::value, T = decltype(t_c)::value;
      constexpr int STAGE = (9 * JP + T + SW - 1) % SW;  // ring stage of step s + SW - 1 (SW | 18)
      constexpr int WC = (T + SW - 1) / 9, WT = (T + SW - 1) % 9;
      constexpr int PPS = Sched::PPS;
      constexpr int PEND = decltype(first_c)::value ? Sched::first_pending(T) : Sched::pending(T);
      __builtin_amdgcn_s_waitcnt(vmcnt_only(PEND));
      __builtin_amdgcn_s_barrier();
      if constexpr (decltype(first_c)::value && PD + T <= SW - 2) pre(ic<PD + T>{});
      if constexpr (Sched::patch_in(T) > 0)
        issue_p(ic<T * PPS>{}, ic<T * PPS + Sched::patch_in(T)>{}, j + 1, 1 - JP);
      issue_w(j + WC, WT, STAGE);
    };
    auto block = [&](int j, auto jp_c, auto first_c) {
      slot(j, jp_c, ic<0>{}, first_c);
      slot(j, jp_c, ic<1>{}, first_c);
      slot(j, jp_c, ic<2>{}, first_c);
      slot(j, jp_c, ic<3>{}, first_c);
      slot(j, jp_c, ic<4>{}, first_c);
      slot(j, jp_c, ic<5>{}, first_c);
      slot(j, jp_c, ic<6>{}, first_c);
      slot(j, jp_c, ic<7>{}, first_c);
      slot(j, jp_c, ic<8>{}, first_c);
    };
    block(0, ic<0>{}, ic<1>{});
    int j = 1;
    for (; j + 1 < ncb; j += 2) {
      block(j, ic<1>{}, ic<0>{});
      block(j + 1, ic<0>{}, ic<0>{});
    }
    if (j < ncb) block(j, ic<1>{}, ic<0>{});
    // the barrier the compute waves pass at the end of their last step (its operands are the
    // clamped loads of the slots past the slice; nothing reads them)
    __builtin_amdgcn_s_barrier();
    // DMA writes still in flight target this workgroup's LDS: let them land before leaving.
    __builtin_amdgcn_s_waitcnt(0);
  };
  if (wave >= NW) {
    if (NPW == 1 || wave == NW)
      producer(ic<0>{});
    else
      producer(ic<NPW - 1>{});
    return;
  }

  // =========================================================================== compute waves
  const int wm = wave % WGM, wn = wave / WGM;

  // ---- epilogue operands (bias, channel addend, residual), read first: they arrive under the
  //      K loop.  Range-checked buffer loads: a null operand gets an empty range and reads
  //      zeros, so there is no branch and no wait here.
  using T = uint16_t;
  const T* bias = reinterpret_cast<const T*>(args.bias);
  const T* res = reinterpret_cast<const T*>(args.residual);
  const T* cadd = reinterpret_cast<const T*>(args.chan_add);
  T* Y = reinterpret_cast<T*>(args.y);
  const __amdgpu_buffer_rsrc_t b_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)bias, (short)0, bias ? O * 2 : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t c_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)cadd, (short)0, cadd ? (args.B - 1) * args.chan_add_ld * 2 + O * 2 : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t r_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)res, (short)0, (res && args.ksplit == 1) ? args.B * O * HW * 2 : 0, 0x00020000);
  uint16_t bh[FC], ah[FC];  // raw bits, converted in the epilogue
  int oc[FC];
#pragma unroll
  for (int fc = 0; fc < FC; ++fc) {
    oc[fc] = o0 + wm * WMO + fc * 16 + (lane & 15);
    const int orr = oc[fc] < O ? oc[fc] : O - 1;
    bh[fc] = __builtin_amdgcn_raw_buffer_load_b16(b_rsrc, orr * 2, 0, 0);
    ah[fc] = HAS_A ? __builtin_amdgcn_raw_buffer_load_b16(c_rsrc, (img * args.chan_add_ld + orr) * 2, 0, 0) : 0;
  }
  // The residual is read here, under the K loop, when its registers fit beside the wave's tile
  // (FP * FC <= 10); a wider tile reads it at the epilogue instead of spilling.
  constexpr bool R_EARLY = FP * FC <= 10;
  Raw4<T> rz[FP][FC];
  auto load_residual = [&]() {
#pragma unroll
    for (int fp = 0; fp < FP; ++fp) {
      const int qq = wn * WNP + fp * 16 + 4 * (lane >> 4);
      const int oy = min(y0 + qq / TW, H - 1), ox = qq % TW;
#pragma unroll
      for (int fc = 0; fc < FC; ++fc) {
        const int orr = oc[fc] < O ? oc[fc] : O - 1;
        const auto u = __builtin_amdgcn_raw_buffer_load_b64(r_rsrc, (((img * O + orr) * HW) + oy * W + ox) * 2, 0, 0);
        rz[fp][fc].u = make_uint2(u[0], u[1]);
      }
    }
  };
  if constexpr (HAS_R && R_EARLY) load_residual();

  // ---- LDS read addresses, fixed for the unit: pixel fragment fp at tap t in patch buffer 0
  //      (buffer 1 is + PBUF), weight fragment fc in stage 0 (stage k is + k * WSTAGE); the
  //      second 32 k of either is the address ^ 64.  Every per-step offset is an immediate.
  uint32_t pa[9][FP], wa[FC];
#pragma unroll
  for (int t = 0; t < 9; ++t)
#pragma unroll
    for (int fp = 0; fp < FP; ++fp) {
      const int qq = wn * WNP + fp * 16 + (lane & 15);
      const int pp = (qq / TW) * PW + (qq % TW) + (t / 3) * PW + (t % 3);
      pa[t][fp] = (uint32_t)(pp * 128 + ((((lane >> 4) ^ (pp >> 1)) & 7) << 4));
    }
#pragma unroll
  for (int fc = 0; fc < FC; ++fc) {
    const int r = wm * WMO + fc * 16 + (lane & 15);
    wa[fc] = (uint32_t)(2 * PBUF + r * 128 + ((((lane >> 4) ^ (r >> 1)) & 7) << 4));
  }

  floatx4 acc[FP][FC];
#pragma unroll
  for (int i = 0; i < FP; ++i)
#pragma unroll
    for (int j = 0; j < FC; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  // Fragment registers of two steps: the MFMAs of step s read set s & 1 while the LDS reads of
  // step s + 1 fill the other set.
  halfx8 pf[2][2][FP], wf[2][2][FC];  // [set][kk][fragment]
  auto read_frags = [&](auto set_c, auto tap_c, auto buf_c, auto stage_c) {
    constexpr int set = decltype(set_c)::value, t = decltype(tap_c)::value;
    constexpr uint32_t poff = decltype(buf_c)::value * PBUF, woff = decltype(stage_c)::value * WSTAGE;
#pragma unroll
    for (int fp = 0; fp < FP; ++fp) {
      pf[set][0][fp] = *reinterpret_cast<const halfx8*>(lds + pa[t][fp] + poff);
      pf[set][1][fp] = *reinterpret_cast<const halfx8*>(lds + (pa[t][fp] ^ 64) + poff);
    }
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) {
      wf[set][0][fc] = *reinterpret_cast<const halfx8*>(lds + wa[fc] + woff);
      wf[set][1][fc] = *reinterpret_cast<const halfx8*>(lds + (wa[fc] ^ 64) + woff);
    }
  };

  // prologue: the barrier that opens step 0, step 0's fragments
  __builtin_amdgcn_s_barrier();
  read_frags(ic<0>{}, ic<0>{}, ic<0>{}, ic<0>{});

  // one step s = 9j + T of a block of parity JP: this step's fragments are in registers, the
  // barrier that opens step s + 1 (after it the producer refills stage s), then step s + 1's
  // LDS reads interleaved with step s's MFMAs.  The last step still reads (in range), so the
  // block never branches.
  auto step = [&](auto jp_c, auto t_c) {
    constexpr int JP = decltype(jp_c)::value, T = decltype(t_c)::value;
    constexpr int set = (JP + T) & 1;
    constexpr int T1 = (T + 1) % 9;                // tap of step s + 1
    constexpr int BUF1 = T == 8 ? 1 - JP : JP;     // its patch buffer
    constexpr int STAGE1 = (9 * JP + T + 1) % SW;  // its ring stage (SW | 18)
    __builtin_amdgcn_s_waitcnt(0xc07f);            // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(ic<1 - set>{}, ic<T1>{}, ic<BUF1>{}, ic<STAGE1>{});
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int fp = 0; fp < FP; ++fp)
#pragma unroll
        for (int fc = 0; fc < FC; ++fc)
          acc[fp][fc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[set][kk][fp], wf[set][kk][fc], acc[fp][fc], 0, 0, 0);
    constexpr int NMF = 2 * FP * FC, NDS = 2 * (FP + FC);
    constexpr int A = NDS < NMF ? NDS : NMF;
#pragma unroll
    for (int i = 0; i < A; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (NDS > A) __builtin_amdgcn_sched_group_barrier(0x100, NDS - A, 0);
    if constexpr (NMF > A) __builtin_amdgcn_sched_group_barrier(0x008, NMF - A, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto block = [&](auto jp_c) {
    step(jp_c, ic<0>{});
    step(jp_c, ic<1>{});
    step(jp_c, ic<2>{});
    step(jp_c, ic<3>{});
    step(jp_c, ic<4>{});
    step(jp_c, ic<5>{});
    step(jp_c, ic<6>{});
    step(jp_c, ic<7>{});
    step(jp_c, ic<8>{});
  };
  int j = 0;
  for (; j + 1 < ncb; j += 2) {
    block(ic<0>{});
    block(ic<1>{});
  }
  if (j < ncb) block(ic<0>{});

  // ---- epilogue: lane l of fragment (fp, fc) holds channel o = o0 + wm*WMO + fc*16 + l%16 at
  //      the four pixels wn*WNP + fp*16 + 4*(l/16) .. +3 (one output row, TW % 4 == 0)
  if (args.ksplit > 1) {
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) {
      const int o = oc[fc];
      if (o >= O) continue;
#pragma unroll
      for (int fp = 0; fp < FP; ++fp) {
        const int qq = wn * WNP + fp * 16 + 4 * (lane >> 4);
        const int oy = y0 + qq / TW, ox = qq % TW;
        if (oy < H) {
          float* dst = args.partial + ((int64_t)split * O + o) * args.ld_partial + (int64_t)img * HW + oy * W + ox;
          *reinterpret_cast<float4*>(dst) = make_float4(acc[fp][fc][0], acc[fp][fc][1], acc[fp][fc][2], acc[fp][fc][3]);
        }
      }
    }
    return;
  }
  if constexpr (HAS_R && !R_EARLY) load_residual();
  float bv[FC], av[FC];
#pragma unroll
  for (int fc = 0; fc < FC; ++fc) {
    bv[fc] = h2f_bits(bh[fc]);
    av[fc] = h2f_bits(ah[fc]);
  }
  // conv + bias, then (+ chan_add), then (+ residual), each add narrowed as the unfused op
  // sequence narrows it.  Every value is narrowed with f2h_rtz_* (an add and half a conversion)
  // while a running maximum of |value| watches for what that covers not (NaN, infinities,
  // |value| >= 65520); a wave in which some lane met one redoes all values with f2h_nonnan, and
  // with f2h_generic (NaN payloads as mtorch keeps them) if some lane met a NaN.
  uint2 out[FP][FC];
  float amax = 0.0f;
  auto narrow_pair = [&](float a, float b) {  // packed narrow(a) | narrow(b) << 16
    amax = abs_max_nan(abs_max_nan(amax, a), b);
    return f2h_rtz_pack(a, b);
  };
#pragma unroll
  for (int fp = 0; fp < FP; ++fp)
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) {
      float x[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) x[t] = acc[fp][fc][t] + bv[fc];
      if constexpr (HAS_A) {  // narrowed pairs + the channel's addend, widened inside the add
        const uint32_t p01 = narrow_pair(x[0], x[1]), p23 = narrow_pair(x[2], x[3]), a = ah[fc];
        x[0] = add_halves<false, false>(p01, a);
        x[1] = add_halves<true, false>(p01, a);
        x[2] = add_halves<false, false>(p23, a);
        x[3] = add_halves<true, false>(p23, a);
      }
      if constexpr (HAS_R) {  // pixels t, t+1 of the residual sit in one register like the pair
        const uint32_t p01 = narrow_pair(x[0], x[1]), p23 = narrow_pair(x[2], x[3]);
        x[0] = add_halves<false, false>(p01, rz[fp][fc].u.x);
        x[1] = add_halves<true, true>(p01, rz[fp][fc].u.x);
        x[2] = add_halves<false, false>(p23, rz[fp][fc].u.y);
        x[3] = add_halves<true, true>(p23, rz[fp][fc].u.y);
      }
      out[fp][fc] = make_uint2(narrow_pair(x[0], x[1]), narrow_pair(x[2], x[3]));
    }
  auto epilogue = [&](auto narrow) {
#pragma unroll
    for (int fp = 0; fp < FP; ++fp)
#pragma unroll
      for (int fc = 0; fc < FC; ++fc) {
        uint32_t h[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float x = acc[fp][fc][t] + bv[fc];
          if constexpr (HAS_A) x = h2f_bits((uint16_t)narrow(x)) + av[fc];
          if constexpr (HAS_R) x = h2f_bits((uint16_t)narrow(x)) + rz[fp][fc].at(t);
          h[t] = narrow(x);
        }
        out[fp][fc] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      }
  };
  if (__builtin_amdgcn_ballot_w64(!(amax < 65520.0f))) {
    bool nan_seen = false;
    epilogue([&](float x) {
      nan_seen |= x != x;
      return f2h_nonnan(x);
    });
    if (__builtin_amdgcn_ballot_w64(nan_seen)) epilogue([](float x) { return (uint32_t)f2h_generic(x); });
  }
  // lane l of fragment (fp, fc) holds channel oc[fc] at the four pixels wn*WNP + fp*16 + 4*(l/16)
  // .. +3 of the unit, one output row (TW % 4 == 0).  TW == W, so unit pixel q is image pixel
  // y0*W + q.  When Y is 8-byte aligned each is one 8-byte buffer store whose address is one
  // per-lane offset (+ fp*32 bytes, + fc*16 channels in soffset); rows past H and channels past
  // O get an out-of-range offset, which the store drops.
  if (((uintptr_t)Y & 7) == 0) {
    const __amdgpu_buffer_rsrc_t y_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)Y, (short)0, args.B * O * HW * 2, 0x00020000);
    const int q0 = wn * WNP + 4 * (lane >> 4);
    const uint32_t lane_off = (uint32_t)(((img * O + oc[0]) * HW + y0 * TW + q0) * 2);
#pragma unroll
    for (int fp = 0; fp < FP; ++fp) {
      const bool row_ok = y0 + (q0 + fp * 16) / TW < H;
#pragma unroll
      for (int fc = 0; fc < FC; ++fc) {
        const uint32_t voff = row_ok && oc[fc] < O ? lane_off : kOOB;
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{out[fp][fc].x, out[fp][fc].y}, y_rsrc, voff + fp * 32,
                                              fc * 32 * HW, 0);
      }
    }
    return;
  }
#pragma unroll
  for (int fp = 0; fp < FP; ++fp) {
    const int qq = wn * WNP + fp * 16 + 4 * (lane >> 4);
    const int oy = y0 + qq / TW, ox = qq % TW;
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) {
      if (oy < H && oc[fc] < O) {
        T* dst = Y + ((int64_t)img * O + oc[fc]) * HW + oy * W + ox;
        dst[0] = (T)(out[fp][fc].x & 0xffffu);
        dst[1] = (T)(out[fp][fc].x >> 16);
        dst[2] = (T)(out[fp][fc].y & 0xffffu);
        dst[3] = (T)(out[fp][fc].y >> 16);
      }
    }
  }
}

}  // namespace mthip
