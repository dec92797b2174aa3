// 3x3 stride-1 pad-1 conv (fp16, NHWC input with Cp % 64 == 0) on MFMA, with the input halo
// kept in LDS across the nine filter taps.
//
//   Y[o, y, x] = sum_{cb, ky, kx, c < 64} Wp[o, ky, kx, 64cb + c] * X[img, y + ky - 1, x + kx - 1, 64cb + c]
//
// A workgroup (4 wave64s) computes one unit: BM output channels x TR output rows x TW (= W)
// columns of one image, over a range of 64-channel blocks (all of them, or one K slice when the
// launcher splits K).  Per channel block it stages the input patch -- (TR+2) x (TW+2) pixels x
// 64 channels, zero outside the image -- into LDS once, and the nine taps then read their B
// fragments from it at shifted pixel positions; only the weights stream per tap.  Against an
// im2col tile, which fetches every input pixel once per tap, this divides the activation bytes
// from L2 by about 9 / (1 + 2/TR): at TR = 2 the unit moves 126 KB per 64 channels for
// 11.8 MFLOP (94 FLOP/B) where a 64x64 im2col tile moves 16 KB per 0.5 MFLOP (32 FLOP/B).
//
// Both operands reach LDS with direct-to-LDS buffer loads (no staging registers, no ds_write):
// an instruction moves 64 x 16 B, i.e. eight 128-byte rows (one row = one pixel's or one output
// channel's 64 channels), with row r's 16-byte chunk c stored at chunk c ^ ((r >> 1) & 7) so that
// the 16 lanes of one ds_read_b128 pass (16 consecutive rows, one logical chunk) cover all 64
// banks whatever row they start at.  Pixels outside the image (the padding) and rows past the
// last output channel are fetched from an out-of-range offset, which the buffer range check
// turns into zeros.
//
// MFMA: v_mfma_f32_16x16x32_f16 with the pixel fragment as the A operand (16 pixels x 32 k) and
// the weight fragment as B (32 k x 16 channels), so lane l's accumulator holds pixels
// 4*(l/16) .. +3 of channel l%16: four consecutive pixels of one NCHW row, stored as 8 bytes.
// Waves split the unit WGM (channels) x 4/WGM (pixels).
//
// Pipeline (one step = one tap of one channel block, 2 x 32 k).  Loads: the weights of step
// s + SW - 1 are issued in step s's slot into a ring of SW stages, and at a channel block's tap
// 0 the next block's patch goes into the other of two patch buffers.  Each wave issues the same
// number of loads in every slot (instructions past the operand fetch zeros into slack rows), so
// the wait that opens a step is one of two compile-time vmcnt values: this wave's loads of the
// step's stage (and of the channel block's patch, issued earlier) have landed; the barrier after
// it makes that true for every wave and guarantees the stage about to be refilled has been read
// by all.  LDS serves about 128 bytes per clock per CU, so at this tile the LDS reads (56 KB a
// step) and the DMA writes (14 KB) take longer than the step's MFMAs: the work per step is
// arranged so that they overlap.  With one wave per SIMD that needs the MFMAs and the memory
// instructions interleaved in one straight-line block (a batch of LDS reads issued in front of
// the MFMAs stalls the wave until the LDS has accepted them).  Fragments live in two register
// sets: step s's MFMAs read one while step s + 1's LDS reads fill the other.
#pragma once

#include "gemm_core.h"
#include "gemm_dtl.h"

namespace mthip {

typedef float floatx4 __attribute__((ext_vector_type(4)));

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
  int x_bytes, w_bytes;
  float* partial;  // ksplit > 1: [ksplit][O][ld_partial] fp32, columns = img*H*W + pixel
  int ld_partial;
};

template <int BM, int TR, int TW, int WGM, int SW, int NW>
__global__ __launch_bounds__(64 * NW) void conv3x3_halo_kernel(const HaloArgs args) {
  constexpr int WGN = NW / WGM;
  constexpr int NPX = TR * TW;          // output pixels per unit
  constexpr int PW = TW + 2, PH = TR + 2;
  constexpr int NP = PH * PW;           // patch pixels
  constexpr int WMO = BM / WGM, WNP = NPX / WGN;
  constexpr int FC = WMO / 16, FP = WNP / 16;
  constexpr int LW = BM / 8;            // weight DMA instructions per step
  constexpr int LWW = (LW + NW - 1) / NW;  // ... per wave
  constexpr int LP = (NP + 7) / 8;      // patch DMA instructions per channel block
  constexpr int LPW = (LP + NW - 1) / NW;  // ... per wave
  constexpr int WROWS = LWW * NW * 8;   // weight rows per stage (slack rows take the dummies)
  constexpr int PROWS = LPW * NW * 8;   // patch rows per buffer
  static_assert((NW == 4 || NW == 8) && WGM * WGN == NW && WMO % 16 == 0 && WNP % 16 == 0 && TW % 4 == 0, "tile shape");
  static_assert(SW >= 3 && SW <= 9 && 18 % SW == 0, "weight ring depth: 3, 6 or 9");
  static_assert((SW - 2) * LWW + LPW <= 63, "vmcnt range");
  static_assert((size_t)(2 * PROWS + SW * WROWS) * 128 <= 160 * 1024, "LDS");

  __shared__ __align__(16) uint8_t lds[(2 * PROWS + SW * WROWS) * 128];
  uint8_t* const patch_lds = lds;
  uint8_t* const w_lds = lds + 2 * PROWS * 128;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WGM, wn = wave / WGM;
  constexpr uint32_t kOOB = 0x80000000u;

  // ---- unit: (image, row block, K slice, channel tile), channel tiles fastest; units are
  //      renumbered so each XCD (workgroups dealt round-robin) takes a contiguous range.
  const uint32_t U = (uint32_t)args.units, U8 = U / 8, u0 = blockIdx.x;
  const uint32_t q = u0 < 8 * U8 ? (u0 % 8) * U8 + u0 / 8 : u0;
  const int mb = (int)(q % (uint32_t)args.tiles_m);
  uint32_t rest = q / (uint32_t)args.tiles_m;
  const int split = (int)(rest % (uint32_t)args.ksplit);
  rest /= (uint32_t)args.ksplit;
  const int rb = (int)(rest % (uint32_t)args.row_blocks);
  const int img = (int)(rest / (uint32_t)args.row_blocks);
  const int H = args.H, W = args.W, Cp = args.Cp, O = args.O;
  const int o0 = mb * BM, y0 = rb * TR;
  const int ncb_total = Cp / 64;
  const int cb0 = split * args.cb_per_split;
  const int ncb = min(args.cb_per_split, ncb_total - cb0);

  const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)args.x, (short)0, args.x_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)args.w, (short)0, args.w_bytes, 0x00020000);

  // ---- epilogue operands (bias, channel addend, residual), read before any operand load: they
  //      arrive under the K loop, and being older than every DMA they never hold up its waits.
  const int HW = H * W;
  using T = uint16_t;
  const T* bias = reinterpret_cast<const T*>(args.bias);
  const T* res = reinterpret_cast<const T*>(args.residual);
  const T* cadd = reinterpret_cast<const T*>(args.chan_add);
  T* Y = reinterpret_cast<T*>(args.y);
  // Range-checked buffer loads: a null operand gets an empty range and reads zeros, so there is
  // no branch (and no wait) in front of the operand loads.
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
    ah[fc] = __builtin_amdgcn_raw_buffer_load_b16(c_rsrc, (img * args.chan_add_ld + orr) * 2, 0, 0);
  }
  Raw4<T> rz[FP][FC];
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

  // ---- per-lane DMA offsets (fixed for the unit; the channel block and tap go in soffset)
  uint32_t w_off[LWW], p_off[LPW];
#pragma unroll
  for (int i = 0; i < LWW; ++i) {
    const int gi = wave * LWW + i;
    const int r = gi * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int o = o0 + r;
    w_off[i] = (gi < LW && o < O) ? ((uint32_t)o * 9u * (uint32_t)Cp + (uint32_t)c * 8u) * 2u : kOOB;
  }
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int gi = wave * LPW + i;
    const int pp = gi * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((pp >> 1) & 7);
    const int pr = pp / PW, pc = pp - (pp / PW) * PW;
    const int iy = y0 - 1 + pr, ix = pc - 1;
    const bool ok = pp < NP && iy >= 0 && iy < H && ix >= 0 && ix < W;
    p_off[i] = ok ? ((((uint32_t)img * (uint32_t)H + (uint32_t)iy) * (uint32_t)W + (uint32_t)ix) * (uint32_t)Cp +
                     (uint32_t)c * 8u) * 2u
                  : kOOB;
  }
  const uint32_t patch_base0 = lds_addr(patch_lds), w_base0 = lds_addr(w_lds);
  constexpr uint32_t PBUF = PROWS * 128, WSTAGE = WROWS * 128;
  const int NS = ncb * 9;
  const int Cp2 = Cp * 2;

  // DMA of step s2's weights (channel block j2 of the slice, tap t2) into ring stage `stage`.
  // A step past the slice re-loads the slice's last block (in range; its stage is never read).
  auto issue_w = [&](int j2, int t2, int stage) {
    const uint32_t dst = w_base0 + (uint32_t)stage * WSTAGE + (uint32_t)wave * (LWW * 1024);
    const int jc = min(j2, ncb - 1);
    const uint32_t soff = (uint32_t)((cb0 + jc) * 128 + t2 * Cp2);
#pragma unroll
    for (int i = 0; i < LWW; ++i) dma16(w_rsrc, dst + i * 1024, w_off[i], soff);
  };
  // DMA of channel block j2's patch into buffer `buf` (past the slice: the last block again,
  // into the buffer the last block does not use).
  auto issue_p = [&](int j2, int buf) {
    const uint32_t dst = patch_base0 + (uint32_t)buf * PBUF + (uint32_t)wave * (LPW * 1024);
    const uint32_t soff = (uint32_t)(cb0 + min(j2, ncb - 1)) * 128u;
#pragma unroll
    for (int i = 0; i < LPW; ++i) dma16(x_rsrc, dst + i * 1024, p_off[i], soff);
  };

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

  // Slot s' (opened by the barrier of step s') issues the next block's patch when s' is a tap-0
  // step, then the weights of step s' + SW - 1.  The wait for step s's operands: this wave's
  // loads issued after the step's weights are the weights of the next SW - 2 steps and, when a
  // channel block started within the last SW - 2 steps, its successor's patch.
  auto pending = [](int t) { return (SW - 2) * LWW + ((t >= 1 && t <= SW - 2) ? LPW : 0); };

  // ---- prologue: the first patch, the weights of steps 0 .. SW-2, slot 0, step 0's fragments
  issue_p(0, 0);
#pragma unroll
  for (int k = 0; k < SW - 1; ++k) issue_w(k / 9, k % 9, k);
  __builtin_amdgcn_s_waitcnt(vmcnt_only(pending(0)));
  __builtin_amdgcn_s_barrier();
  issue_p(1, 1);
  issue_w((SW - 1) / 9, (SW - 1) % 9, SW - 1);
  read_frags(ic<0>{}, ic<0>{}, ic<0>{}, ic<0>{});

  // ---- one step s = 9j + T of a channel block j of parity JP.  Every wave has step s's
  //      fragments (lgkmcnt) and step s + 1's operands (vmcnt) -> barrier -> one straight-line
  //      block: the LDS reads of step s + 1 into the other register set and slot s + 1's loads,
  //      interleaved one-to-one with step s's MFMAs (issued as a batch in front of the MFMAs
  //      they would stall the single wave of the SIMD).  The last step still reads (in range)
  //      and loads (clamped), so the block never branches.
  auto step = [&](int j, auto jp_c, auto t_c) {
    constexpr int JP = decltype(jp_c)::value, T = decltype(t_c)::value;
    constexpr int set = (JP + T) & 1;
    constexpr int T1 = (T + 1) % 9;                      // tap of step s + 1
    constexpr int BUF1 = T == 8 ? 1 - JP : JP;           // its patch buffer
    constexpr int STAGE = (3 * JP + T) % SW;             // ring stage of step s (SW | 18)
    constexpr int STAGE1 = (3 * JP + T + 1) % SW;        // ... of step s + 1
    constexpr int WC = (T + SW) / 9, WT = (T + SW) % 9;  // step s + SW relative to block j
    __builtin_amdgcn_s_waitcnt(0xc07f);                  // lgkmcnt(0)
    __builtin_amdgcn_s_waitcnt(vmcnt_only(pending(T1)));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(ic<1 - set>{}, ic<T1>{}, ic<BUF1>{}, ic<STAGE1>{});
    if constexpr (T == 8) issue_p(j + 2, JP);
    issue_w(j + WC, WT, STAGE);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int fp = 0; fp < FP; ++fp)
#pragma unroll
        for (int fc = 0; fc < FC; ++fc)
          acc[fp][fc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[set][kk][fp], wf[set][kk][fc], acc[fp][fc], 0, 0, 0);
    constexpr int NMF = 2 * FP * FC, NDS = 2 * (FP + FC), NVM = LWW + (T == 8 ? LPW : 0);
    constexpr int A = NDS < NMF ? NDS : NMF;                      // MFMA + DS pairs
    constexpr int Bv = NVM < NMF - A ? NVM : NMF - A;             // then MFMA + VMEM pairs
#pragma unroll
    for (int i = 0; i < A; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (NDS > A) __builtin_amdgcn_sched_group_barrier(0x100, NDS - A, 0);
#pragma unroll
    for (int i = 0; i < Bv; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    if constexpr (NVM > Bv) __builtin_amdgcn_sched_group_barrier(0x020, NVM - Bv, 0);
    if constexpr (NMF > A + Bv) __builtin_amdgcn_sched_group_barrier(0x008, NMF - A - Bv, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto block = [&](int j, auto jp_c) {
    step(j, jp_c, ic<0>{});
    step(j, jp_c, ic<1>{});
    step(j, jp_c, ic<2>{});
    step(j, jp_c, ic<3>{});
    step(j, jp_c, ic<4>{});
    step(j, jp_c, ic<5>{});
    step(j, jp_c, ic<6>{});
    step(j, jp_c, ic<7>{});
    step(j, jp_c, ic<8>{});
  };
  int j = 0;
  for (; j + 1 < ncb; j += 2) {
    block(j, ic<0>{});
    block(j + 1, ic<1>{});
  }
  if (j < ncb) block(j, ic<0>{});
  (void)NS;
  // DMA writes still in flight (the zero-fill of the last steps) target this workgroup's LDS.
  __builtin_amdgcn_s_waitcnt(0);

  // ---- epilogue: lane l of fragment (fp, fc) holds channel o = o0 + wm*WMO + fc*16 + l%16 at
  //      the four pixels wn*WNP + fp*16 + 4*(l/16) .. +3 (one output row, TW % 4 == 0)
  if (args.ksplit > 1) {
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) {
      const int o = o0 + wm * WMO + fc * 16 + (lane & 15);
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
  float bv[FC], av[FC];
#pragma unroll
  for (int fc = 0; fc < FC; ++fc) {
    bv[fc] = h2f_bits(bh[fc]);
    av[fc] = h2f_bits(ah[fc]);
  }
#pragma unroll
  for (int fp = 0; fp < FP; ++fp) {
    const int qq = wn * WNP + fp * 16 + 4 * (lane >> 4);
    const int oy = y0 + qq / TW, ox = qq % TW;
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) {
      float v[4], r[4];
      const float b[4] = {bv[fc], bv[fc], bv[fc], bv[fc]};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[t] = acc[fp][fc][t];
        r[t] = rz[fp][fc].at(t);
      }
      epi_math<T, EPI_CONV, MTHIP_ACT_NONE>(v, b, true, av[fc], cadd != nullptr, r, res != nullptr);
      if (oy < H && oc[fc] < O) store_cols<T>(Y + ((int64_t)img * O + oc[fc]) * HW + oy * W + ox, v, 4);
    }
  }
}

}  // namespace mthip
