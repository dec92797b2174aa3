// Streamed fp16 linear layer (gfx950): C[m, n] = sum_k A[m, k] * B[n, k] + bias[n] (+ R[m, n]),
// A the activations (tokens x K), B the weight (N x K), both k-contiguous, fp32 accumulate,
// mtorch's fp16 narrowing of every stored value.
//
// A unit is 80 output channels x BT tokens over a run of K (one slice of the K split); a
// persistent workgroup takes a contiguous run of units (XCD-contiguous numbering) and streams
// their K steps (64 k each) back to back through one LDS ring.  BT/16 compute waves (each owns
// all 80 channels x 16 tokens: FC = 5 channel fragments x one token fragment of
// v_mfma_f32_16x16x32_f16) and a producer wave that issues every direct-to-LDS load.  A
// compute wave reads 12 KB of fragments from LDS per step against 10 MFMAs; one wave per SIMD
// draws LDS at about half the rate two waves per SIMD do (~140 against ~250 bytes per clock per
// CU in a read-only loop), so 128-token units (eight compute waves) keep the LDS busier than
// 64-token units (four).  The
// producer runs SW - 1 steps ahead of the compute waves across unit boundaries, so the next
// unit's first K steps arrive while the compute waves run the previous unit's epilogue -- the
// DTL GEMM instead starts every unit's pipeline from its own loads, which at K = 320 (five
// steps) is most of a unit.
//
// Step protocol: before barrier s the producer waits (a fixed vmcnt) until step s's operands
// have landed and the compute waves until every LDS read of step s - 1 is in registers; after
// it the producer refills the ring stage of step s - 1 with step s + SW - 1.  A compute wave
// runs step s as: the first 32-k half's MFMAs interleaved with the second half's LDS reads,
// barrier s + 1, the second half's MFMAs interleaved with step s + 1's first-half reads.  Units
// hold a multiple of SW steps (the launcher requires K / 64 to be a multiple of 5), so every unit
// starts at ring stage 0 and a group of SW steps has compile-time stages.
//
// NCHW: the 1x1 conv of a channels-last activation (A = x_nhwc [B*HW][Cp], B = the packed weight
// [O][Cp]) stored NCHW, y[img][n][p] for token m = img*HW + p: the MFMA operands swap so that a
// lane's accumulator is 4 consecutive pixels of one output channel (HW % 4 == 0: one image,
// one 8-byte store), the bias is per channel and the residual NCHW like y; K-split partials go
// to [split][N][ld_partial] (channel rows, pixel columns), the layout the conv reduction reads.
//
// LDS stage layout: the 80 weight rows, then the BT token rows, each row 64 halves (128 bytes)
// with 16-byte chunk c at chunk c ^ ((row >> 1) & 7) (the ds_read_b128 passes of a fragment
// cover all 64 banks).  Rows past M or N are fetched from an out-of-range offset and read as
// zeros.
#pragma once

#include "gemm_core.h"
#include "gemm_dtl.h"

namespace mthip {

typedef float floatx4 __attribute__((ext_vector_type(4)));

struct StreamArgs {
  const void* a;  // [M][lda]
  const void* b;  // [N][ldb]
  void* c;        // [M][ldc]
  const void* bias;      // [N] or null
  const void* residual;  // [M][ld_res] or null
  int M, N, lda, ldb, ldc, ld_res;
  int tiles_m, tiles_n, ksplit;
  int steps;   // K steps per unit (a multiple of 5)
  int units;   // tiles_m * tiles_n * ksplit
  int a_bytes, b_bytes;
  float* partial;  // ksplit > 1: [ksplit][M][ld_partial] fp32
  int ld_partial;
  int m_fast;  // 1: consecutive units walk the token tiles of one channel tile
  int hw;          // NCHW: pixels per image
  FastDiv div_hw;  // NCHW: division by hw
  const uint16_t* gelu_tab;  // GELU: the fp16 gelu of every half value
};

// GELU (row-major, no residual): the output is the fp16 gelu of each narrowed value, looked up
// in gelu_tab as the fp16 gelu op (and the tile GEMM's fused epilogue) computes it.
template <int BT, bool HAS_R, bool NCHW = false, bool GELU = false>
__global__ __launch_bounds__((BT / 16 + BT / 64) * 64) void gemm_stream_kernel(const StreamArgs args) {
  static_assert(!(GELU && (HAS_R || NCHW)), "the GELU epilogue is row-major without a residual");
  constexpr int BC = 80, NW = BT / 16, NP = BT / 64, SW = 5;
  constexpr int WT = BT / NW;              // tokens per compute wave
  constexpr int FC = BC / 16, FP = WT / 16;
  constexpr int LW = BC / 8, LA = BT / 8;  // DMA instructions per step
  constexpr int L = LW + LA;
  constexpr uint32_t STAGE = (BC + BT) * 128;
  static_assert(BT % 64 == 0 && FP >= 1, "tokens per unit: a multiple of 64");
  static_assert((size_t)SW * STAGE <= 160 * 1024, "LDS");
  __shared__ __align__(16) uint8_t lds[SW * STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr uint32_t kOOB = 0x80000000u;

  // ---- this workgroup's run of units: workgroups are dealt to the 8 XCDs round-robin, so
  //      workgroup w takes chunk (w % 8) * (G / 8) + w / 8 of G equal runs (G a multiple of 8).
  const uint32_t G = gridDim.x, w = blockIdx.x;
  const uint32_t chunk = (G % 8 == 0) ? (w % 8) * (G / 8) + w / 8 : w;
  const uint32_t U = (uint32_t)args.units;
  const uint32_t u_begin = (uint32_t)(((uint64_t)U * chunk) / G), u_end = (uint32_t)(((uint64_t)U * (chunk + 1)) / G);
  const int M = args.M, N = args.N, steps = args.steps;
  struct Unit {
    int m0, n0, split;
  };
  auto decode = [&](uint32_t u) {
    Unit r;
    const uint32_t tmn = (uint32_t)(args.tiles_m * args.tiles_n);
    r.split = (int)(u / tmn);
    const uint32_t t = u - (uint32_t)r.split * tmn;
    uint32_t tm, tn;
    if (args.m_fast) {
      tm = t % (uint32_t)args.tiles_m;
      tn = t / (uint32_t)args.tiles_m;
    } else {
      tn = t % (uint32_t)args.tiles_n;
      tm = t / (uint32_t)args.tiles_n;
    }
    r.m0 = (int)tm * BT;
    r.n0 = (int)tn * BC;
    return r;
  };

  // =============================================================================== producer
  // NP producer waves share a step's L loads: load i (the LW weight rows, then the LA token
  // rows) goes to producer i % NP, and each waits for its own share.
  auto producer = [&](auto pw_c) {
    constexpr int PW = decltype(pw_c)::value;
    constexpr int MINE = (L - PW + NP - 1) / NP;  // loads of this producer per step
    constexpr int PEND = (SW - 2) * MINE;
    static_assert(PEND <= 63, "vmcnt range");
    const __amdgpu_buffer_rsrc_t a_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)args.a, (short)0, args.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t b_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)args.b, (short)0, args.b_bytes, 0x00020000);
    const uint32_t base = lds_addr(lds);
    uint32_t w_off[LW], a_off[LA];
    uint32_t iu = u_begin;  // unit and step of the next load
    int ij = 0, k0 = 0;
    // Lane l covers row 8gi + l/8 of load gi and 16-byte chunk (l & 7) ^ ((row >> 1) & 7), which
    // is (l & 7) ^ (l / 16) ^ 4(gi & 1) (8 | 8gi, and BC = 80 is a multiple of 16): per unit one
    // multiply per operand, the rest wave-uniform steps.
    const int l3 = lane >> 3;
    const uint32_t chunk0 = (uint32_t)((lane & 7) ^ (lane >> 4)) * 16u;
    const uint32_t ldb2 = (uint32_t)args.ldb * 2u, lda2 = (uint32_t)args.lda * 2u;
    auto set_unit = [&]() {
      const bool live = iu < u_end;
      const Unit un = decode(live ? iu : u_begin);
      k0 = un.split * steps;
      const uint32_t wl = (uint32_t)(un.n0 + l3) * ldb2, al = (uint32_t)(un.m0 + l3) * lda2;
#pragma unroll
      for (int gi = 0; gi < LW; ++gi)
        w_off[gi] = (live && un.n0 + gi * 8 + l3 < N) ? wl + (uint32_t)(gi * 8) * ldb2 + (chunk0 ^ (gi & 1 ? 64u : 0u)) : kOOB;
#pragma unroll
      for (int gi = 0; gi < LA; ++gi)
        a_off[gi] = (live && un.m0 + gi * 8 + l3 < M) ? al + (uint32_t)(gi * 8) * lda2 + (chunk0 ^ (gi & 1 ? 64u : 0u)) : kOOB;
    };
    // this producer's share of one step's loads into ring stage `stage` (past the last unit:
    // out-of-range, zeros)
    auto issue = [&](uint32_t stage) {
      const uint32_t dst = base + stage * STAGE;
      const uint32_t soff = (uint32_t)(k0 + ij) * 128u;
#pragma unroll
      for (int gi = 0; gi < LW; ++gi)
        if (gi % NP == PW) dma16(b_rsrc, dst + gi * 1024, w_off[gi], soff);
#pragma unroll
      for (int gi = 0; gi < LA; ++gi)
        if ((LW + gi) % NP == PW) dma16(a_rsrc, dst + (uint32_t)BC * 128u + gi * 1024, a_off[gi], soff);
      if (++ij == steps) {
        ij = 0;
        ++iu;
        set_unit();
      }
    };
    set_unit();
    issue(0);
    issue(1);
    issue(2);
    issue(3);
    const uint32_t total = (u_end - u_begin) * (uint32_t)steps;
    uint32_t stage = SW - 1;
    for (uint32_t s = 0; s < total; ++s) {
      __builtin_amdgcn_s_waitcnt(vmcnt_only(PEND));
      __builtin_amdgcn_s_barrier();
      issue(stage);
      stage = stage == SW - 1 ? 0 : stage + 1;
    }
    // the barrier the compute waves pass at the end of their last step
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_s_waitcnt(0);
  };
  if (wave >= NW) {
    if (NP == 1 || wave == NW) producer(ic<0>{});
    else producer(ic<1>{});
    return;
  }

  // =========================================================================== compute waves
  using T = uint16_t;
  const T* bias = reinterpret_cast<const T*>(args.bias);
  const T* res = reinterpret_cast<const T*>(args.residual);
  T* C = reinterpret_cast<T*>(args.c);
  const __amdgpu_buffer_rsrc_t bias_rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)bias, (short)0, bias ? N * 2 : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t res_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)res, (short)0,
      (HAS_R && args.ksplit == 1) ? (NCHW ? M * N * 2 : ((M - 1) * args.ld_res + N) * 2) : 0, 0x00020000);

  // LDS read addresses in stage 0 (stage k is + k * STAGE; the second 32 k is ^ 64)
  uint32_t wa[FC], pa[FP];
#pragma unroll
  for (int fc = 0; fc < FC; ++fc) {
    const int r = fc * 16 + (lane & 15);
    wa[fc] = (uint32_t)(r * 128 + ((((lane >> 4) ^ (r >> 1)) & 7) << 4));
  }
#pragma unroll
  for (int fp = 0; fp < FP; ++fp) {
    const int r = BC + wave * WT + fp * 16 + (lane & 15);
    pa[fp] = (uint32_t)(r * 128 + ((((lane >> 4) ^ (r >> 1)) & 7) << 4));
  }

  floatx4 acc[FC][FP];
  halfx8 wf[2][FC], pf[2][FP];  // [kk][fragment]: the two 32-k halves of a step
  auto zero_acc = [&]() {
#pragma unroll
    for (int fc = 0; fc < FC; ++fc)
#pragma unroll
      for (int fp = 0; fp < FP; ++fp) acc[fc][fp] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  };
  // this lane's fragments of 32-k half KK of the step in ring stage STAGE_
  auto read_half = [&](auto kk_c, auto stage_c) {
    constexpr int KK = decltype(kk_c)::value;
    constexpr uint32_t off = decltype(stage_c)::value * STAGE, x = KK ? 64u : 0u;
#pragma unroll
    for (int fp = 0; fp < FP; ++fp) pf[KK][fp] = *reinterpret_cast<const halfx8*>(lds + (pa[fp] ^ x) + off);
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) wf[KK][fc] = *reinterpret_cast<const halfx8*>(lds + (wa[fc] ^ x) + off);
  };
  auto mfma_half = [&](auto kk_c) {
    constexpr int KK = decltype(kk_c)::value;
#pragma unroll
    for (int fc = 0; fc < FC; ++fc)
#pragma unroll
      for (int fp = 0; fp < FP; ++fp)
        acc[fc][fp] = NCHW ? __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[KK][fp], wf[KK][fc], acc[fc][fp], 0, 0, 0)
                           : __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[KK][fc], pf[KK][fp], acc[fc][fp], 0, 0, 0);
  };
  // the LDS reads of one half interleaved one-to-one with the MFMAs of the other
  auto interleave = [&]() {
    constexpr int NMF = FP * FC, NDS = FP + FC;
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

  // The current unit's epilogue operands.  The row-major bias is read when the unit starts (it
  // arrives under the K steps; at the epilogue its wait cost a 128-token unit ~2 %), the NCHW
  // bias (one 2-byte load per channel) at the epilogue (3 % faster for the 1x1 convs at 32x32
  // and 16x16); the residual when a 64-token unit starts and at a 128-token unit's epilogue
  // (beside the tile and the fragments of eight compute waves it does not fit in registers).
  // Lane l of fragment (fc, fp) holds channels n0 + fc*16 + 4*(l/16) .. +3 of token
  // m0 + wave*WT + fp*16 + l%16 (NCHW: tokens m0 + wave*WT + fp*16 + 4*(l/16) .. +3 of channel
  // n0 + fc*16 + l%16).
  constexpr bool R_EARLY = BT == 64;
  Unit cur{};
  uint2 bz[FC], rz[FC][FP];
  // this lane's channel and first token of fragment (fc, fp)
  auto chan = [&](int fc) { return cur.n0 + fc * 16 + (NCHW ? (lane & 15) : 4 * (lane >> 4)); };
  auto tok = [&](int fp) { return cur.m0 + wave * WT + fp * 16 + (NCHW ? 4 * (lane >> 4) : (lane & 15)); };
  // NCHW element offset of (token m, channel n): image m / hw, pixel m % hw
  auto nchw_off = [&](int m, int n) {
    const int img = (int)args.div_hw.div((uint32_t)m);
    return (img * N + n) * args.hw + (m - img * args.hw);
  };
  auto load_residual = [&]() {
#pragma unroll
    for (int fc = 0; fc < FC; ++fc)
#pragma unroll
      for (int fp = 0; fp < FP; ++fp) {
        const int n = chan(fc), m = tok(fp);
        const int o = (m < M && n < N) ? (NCHW ? nchw_off(m, n) : m * args.ld_res + n) : 0;
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(res_rsrc, o * 2, 0, 0);
        rz[fc][fp] = make_uint2(v[0], v[1]);
      }
  };
  auto load_bias = [&]() {
#pragma unroll
    for (int fc = 0; fc < FC; ++fc) {
      const int n = chan(fc);
      if constexpr (NCHW) {
        // one channel per lane: its bias in both halves of every word
        const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(bias_rsrc, (n < N ? n : 0) * 2, 0, 0);
        bz[fc] = make_uint2(h | (h << 16), h | (h << 16));
      } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(bias_rsrc, (n < N ? n : 0) * 2, 0, 0);
        bz[fc] = make_uint2(v[0], v[1]);
      }
    }
  };
  auto begin_unit = [&](uint32_t u) {
    cur = decode(u);
    if constexpr (!NCHW) load_bias();
    if constexpr (HAS_R && R_EARLY) load_residual();
    zero_acc();
  };
  auto end_unit = [&]() {
    if (args.ksplit > 1) {
#pragma unroll
      for (int fc = 0; fc < FC; ++fc)
#pragma unroll
        for (int fp = 0; fp < FP; ++fp) {
          const int n = chan(fc), m = tok(fp);
          const int64_t o = NCHW ? ((int64_t)cur.split * N + n) * args.ld_partial + m
                                 : ((int64_t)cur.split * M + m) * args.ld_partial + n;
          if (m < M && n < N)
            *reinterpret_cast<float4*>(args.partial + o) =
                make_float4(acc[fc][fp][0], acc[fc][fp][1], acc[fc][fp][2], acc[fc][fp][3]);
        }
      return;
    }
    if constexpr (NCHW) load_bias();
    if constexpr (HAS_R && !R_EARLY) load_residual();
    // + bias, (narrowed, + residual), narrowed: every value with f2h_rtz_* (a half-spacing add
    // and half a round-toward-zero conversion; the residual added to the narrowed pair inside
    // v_fma_mix_f32), under a running maximum of |value|; a wave that met a NaN, an infinity
    // or |value| >= 65520 redoes its values with f2h_nonnan, and with f2h_generic if one was NaN.
    uint2 out[FC][FP];
    auto bias_at = [&](int fc, int t) {
      const uint32_t bw = t < 2 ? bz[fc].x : bz[fc].y;
      return bias ? h2f_bits((uint16_t)((t & 1) ? bw >> 16 : bw & 0xffffu)) : -0.0f;
    };
    float amax = 0.0f;
    auto narrow_pair = [&](float a, float b) {
      amax = abs_max_nan(abs_max_nan(amax, a), b);
      return f2h_rtz_pack(a, b);
    };
#pragma unroll
    for (int fc = 0; fc < FC; ++fc)
#pragma unroll
      for (int fp = 0; fp < FP; ++fp) {
        float x[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) x[t] = acc[fc][fp][t] + bias_at(fc, t);
        if constexpr (HAS_R) {
          const uint32_t p01 = narrow_pair(x[0], x[1]), p23 = narrow_pair(x[2], x[3]);
          x[0] = add_halves<false, false>(p01, rz[fc][fp].x);
          x[1] = add_halves<true, true>(p01, rz[fc][fp].x);
          x[2] = add_halves<false, false>(p23, rz[fc][fp].y);
          x[3] = add_halves<true, true>(p23, rz[fc][fp].y);
        }
        out[fc][fp] = make_uint2(narrow_pair(x[0], x[1]), narrow_pair(x[2], x[3]));
        if constexpr (GELU) {
          auto g = [&](uint32_t p) {
            return (uint32_t)args.gelu_tab[p & 0xffffu] | ((uint32_t)args.gelu_tab[p >> 16] << 16);
          };
          out[fc][fp] = make_uint2(g(out[fc][fp].x), g(out[fc][fp].y));
        }
      }
    auto chain = [&](auto& narrow) {
#pragma unroll
      for (int fc = 0; fc < FC; ++fc)
#pragma unroll
        for (int fp = 0; fp < FP; ++fp) {
          uint32_t h[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float x = acc[fc][fp][t] + bias_at(fc, t);
            if constexpr (HAS_R) {
              const uint32_t rw = t < 2 ? rz[fc][fp].x : rz[fc][fp].y;
              x = h2f_bits((uint16_t)narrow(x)) + h2f_bits((uint16_t)((t & 1) ? rw >> 16 : rw & 0xffffu));
            }
            h[t] = narrow(x);
            if constexpr (GELU) h[t] = args.gelu_tab[h[t]];
          }
          out[fc][fp] = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
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
    for (int fc = 0; fc < FC; ++fc)
#pragma unroll
      for (int fp = 0; fp < FP; ++fp) {
        const int n = chan(fc), m = tok(fp);
        if (m < M && n < N)
          *reinterpret_cast<uint2*>(C + (NCHW ? (int64_t)nchw_off(m, n) : (int64_t)m * args.ldc + n)) = out[fc][fp];
      }
  };

  // One step (ring stage ST0; the next step's stage ST1), entered with its first 32-k half's
  // fragments in registers: the second half's LDS reads interleaved with the first half's
  // MFMAs, the barrier, then the next step's first-half reads interleaved with the second
  // half's MFMAs.  The barrier sits where every read of this step has completed and none of the
  // next step's has started, so the producer may refill this step's ring stage after it (and the
  // next step's operands are in LDS when it opens).  Half a step of fragments in flight (48
  // registers) instead of a whole step (96) leaves room for two compute waves per SIMD.
  auto step = [&](auto st0_c, auto st1_c) {
    read_half(ic<1>{}, st0_c);
    mfma_half(ic<0>{});
    interleave();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_half(ic<0>{}, st1_c);
    mfma_half(ic<1>{});
    interleave();
  };
  // a group of SW steps starting at ring stage 0
  auto group = [&]() {
    step(ic<0>{}, ic<1>{});
    step(ic<1>{}, ic<2>{});
    step(ic<2>{}, ic<3>{});
    step(ic<3>{}, ic<4>{});
    step(ic<4>{}, ic<0>{});
  };

  // Units end on group boundaries.
  __builtin_amdgcn_s_barrier();
  read_half(ic<0>{}, ic<0>{});
  uint32_t u = u_begin;
  int left = (int)(u_end - u_begin) * steps;  // steps still to run
  int in_unit = 0;
  if (u < u_end) begin_unit(u);
  auto after_group = [&]() {
    left -= SW;
    in_unit += SW;
    if (in_unit == steps) {
      end_unit();
      in_unit = 0;
      if (++u < u_end) begin_unit(u);
    }
  };
  while (left > 0) {
    group();
    after_group();
  }
}

}  // namespace mthip
