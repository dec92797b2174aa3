// scaled_dot_product_attention: flash-style fused kernel on MFMA (fp16) and a wave-per-query
// kernel for fp32 and shapes outside the MFMA instances.
//
// MFMA kernel layout.  A workgroup is 4 wave64s; each wave owns 32 queries of one (batch, head)
// and the workgroup walks the keys in 64-key tiles.  Per 32-key half-tile a wave computes the
// transposed score block S^T = K . Q^T with v_mfma_f32_32x32x16_f16, so lane l holds the scores
// of query (l % 32) against 16 keys: a query's online-softmax max/sum is an in-register
// reduction plus one exchange with lane l^32.  Those accumulator registers, converted to fp16,
// are exactly the B operand of O^T += V^T . P^T (register r <-> key 8*(r/4) + 4*(l/32) + r%4 in
// both products), so P never leaves registers.  K and V are staged in LDS row-major with
// 16-byte writes; the V^T operand of the PV product comes out of LDS through gfx950's
// transposing read (ds_read_b64_tr_b16).  The next tile's K/V are fetched into registers with
// 16-byte range-checked buffer loads while the current tile is multiplied.  Scores are kept in log2 units
// (scale * log2 e folded in) so the exponentials are single v_exp_f32.  Softmax statistics and
// the output accumulator are fp32; fully masked rows end as 0/0 = NaN, as the reference's
// softmax of an all -inf row does (tensor.cpp:30429-30442).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cmath>

#include "common.h"

namespace mthip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

struct FlashArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t qs[3], ks[3], vs[3], os[3];  // element strides: batch, head, sequence (last dim contiguous)
  int64_t H, Hk, Lq, Lk, E, Ev;
  int mask_kind, mask_dtype;
  const void* mask;
  int64_t ms[4];  // mask strides: b, h, q, k
  int causal;
  float scale;  // as given: zero and negative values multiply the scores like any other
  int cus;  // compute units of the device (launch-shape choices)
  // Key splits (flash kernel): workgroup z of gridDim.z takes keys [z * kv_chunk, (z+1) *
  // kv_chunk) and, when gridDim.z > 1, writes its unnormalised accumulator and (max, sum) to
  // part[z][b*H + h][q][pitch] (dims 0 .. DVB*32-1, then max at DVB*32 and sum at DVB*32 + 1,
  // log2 units) for flash_combine_kernel instead of the output.
  int kv_chunk;
  float* part;
  int part_pitch;
};

__device__ __forceinline__ float mask_value(const FlashArgs& a, int64_t b, int64_t h, int64_t q, int64_t k,
                                            float score) {
  if (a.mask_kind == MTHIP_MASK_NONE) return score;
  const int64_t off = b * a.ms[0] + h * a.ms[1] + q * a.ms[2] + k * a.ms[3];
  if (a.mask_kind == MTHIP_MASK_BOOL) return reinterpret_cast<const uint8_t*>(a.mask)[off] ? score : -INFINITY;
  if (a.mask_dtype == MTHIP_F16) return score + h2f_bits(reinterpret_cast<const uint16_t*>(a.mask)[off]);
  return score + reinterpret_cast<const float*>(a.mask)[off];
}

__device__ __forceinline__ uint4 bload(const __amdgpu_buffer_rsrc_t& r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

constexpr uint32_t kOOB = 0x80000000u;

typedef short shortx4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: lane j of each 16-lane group receives halves [j%4] of the 8-byte rows read
// by lanes j/4, j/4+4, j/4+8 and j/4+12 of the group (p points into LDS).
__device__ __forceinline__ halfx4 tr_read16(const uint16_t* p) {
  return __builtin_bit_cast(halfx4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                        (__attribute__((address_space(3))) shortx4*)(const_cast<uint16_t*>(p))));
}

// DK: head dim padded to a multiple of 16 (QK^T K-steps); the value dim is covered by
// DVB = ceil(DK/32) 32-row blocks.  VEC: E and Ev are multiples of 8 and every row stride a
// multiple of 8 elements with 16-byte aligned bases, so K/V/Q move in 16-byte chunks.
// MASK: the mask kind (MTHIP_MASK_*) fixed at compile time, or -1 to read it at run time.
// WAVES: waves per key group; with DS dim parts they serve WAVES/DS blocks of 32 queries, DS
// waves per block, each computing the block's scores and 1/DS of its output dims (DS = 1: a
// wave is a query block).  KG: key groups -- KG sets of WAVES
// waves take the same queries and alternate 64-key tiles (group g the tiles g, g+KG, ...),
// each with its own LDS tile and online softmax; at the end group 0 folds in the others'
// (max, sum, accumulator).  KG = 2 doubles the waves per SIMD on the large self-attentions,
// where one wave's chain (score MFMAs -> softmax VALU -> PV MFMAs) would otherwise leave the
// MFMA and VALU pipes idle.
template <int DK, bool VEC, int MASK, int WAVES, int KG = 1, int DS = 1>
__global__ __launch_bounds__(64 * WAVES * KG) __attribute__((amdgpu_waves_per_eu(KG > 1 ? 4 : 1)))
void flash_fwd_f16_kernel(const FlashArgs a) {
  constexpr int NT = 64 * WAVES;  // threads of one key group
  constexpr int NSTEP = DK / 16;
  constexpr int DVB = (DK + 31) / 32;
  constexpr int BKV = 64;
  constexpr int KP = DK + 8;    // LDS pitch of the K tile (halves)
  constexpr int VRP = DVB * 32 + 8;  // LDS pitch of a V row (halves; 16-byte multiple)
  constexpr int KCHR = DK / 8;  // 16-byte chunks per K row
  constexpr int VCHR = DVB * 4; // 16-byte chunks per V row (DVB*32 dims)
  constexpr int KCH = (BKV * KCHR + NT - 1) / NT;
  constexpr int VCH = (BKV * VCHR + NT - 1) / NT;
  static_assert(KG == 1 || KG == 2, "one or two key groups");
  static_assert(DS == 1 || (KG == 1 && WAVES % DS == 0), "dim parts need one key group");
  constexpr int DVBP = (DVB + DS - 1) / DS;  // 32-dim output blocks per dim part
  // One K/V tile per key group; after the key loop the same memory holds the group merge (one
  // lane's (max, sum) or 16 accumulator values, pitch 17 floats).
  constexpr int TILE = BKV * KP + BKV * VRP;  // halves of one K tile + V tile (16-byte multiple)
  constexpr int XCH = KG > 1 ? NT * 17 * 2 : 0;  // halves of the merge buffer
  __shared__ __align__(16) uint16_t smem[KG * TILE > XCH ? KG * TILE : XCH];

  const int grp = KG > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x / NT)) : 0;  // wave-uniform
  const int tid = (int)threadIdx.x - grp * NT, lane = tid & 63, wave = tid >> 6;
  uint16_t* const Ks = smem + grp * TILE;
  uint16_t* const Vr = Ks + BKV * KP;
  const int hh = lane >> 5, col = lane & 31;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.H, head = bh - b * a.H;
  const int64_t kvh = head / (a.H / a.Hk);
  // DS dim parts: waves wave/DS own query block wave/DS and the output blocks [dp*DVBP,
  // dp*DVBP + DVBP) of it, dp = wave % DS (each computes the block's scores itself).
  const int dp = wave % DS;
  const int64_t q = (int64_t)blockIdx.x * (32 * WAVES / DS) + (wave / DS) * 32 + col;
  // this workgroup's key range [kb, Lk): all keys, or one split of them
  const int kb = (int)blockIdx.z * a.kv_chunk;
  const int Lk = min((int)a.Lk, kb + a.kv_chunk), E = (int)a.E, Ev = (int)a.Ev;
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.q) + b * a.qs[0] + head * a.qs[1];
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k) + b * a.ks[0] + kvh * a.ks[1];
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.v) + b * a.vs[0] + kvh * a.vs[1];

  // Q^T fragments (B operand of S^T): query q, dims step*16 + hh*8 + [0, 8).  A negative scale
  // runs as softmax((-q) k^T |scale|): the sign goes into Q (an exact fp16 negation), so the
  // scores stay in the "larger is heavier" order the running max relies on.
  //
  // KSHIFT (head dims <= 40 in the 48-dim instance, the launcher's choice): Q is taken
  // pre-multiplied by scale * log2(e) (rounded to fp16; scales with |scale * log2 e| outside
  // [2^-10, 1] go to the generic instance, so that product neither overflows nor drops Q's low
  // bits), and padding dim 40 carries -m, the running max, against a K column of ones: the
  // score MFMAs then deliver score * scale * log2(e) - m, the exp2 argument as it stands, where
  // the other instances spend a multiply-add per score (a quarter of the softmax's VALU time
  // next to the exp2 at its quarter rate).  m is kept representable in fp16 while |m| <= 2^15;
  // beyond, dim 40 carries 0 and the lane subtracts m itself.
  constexpr bool KSHIFT = VEC && DK == 48;
  constexpr int KSD = 40;  // the shift dim: qf[KSD / 16][0] of the lanes with hh == 1
  const uint32_t qneg = a.scale < 0.0f ? 0x80008000u : 0u;
  halfx8 qf[NSTEP];
#pragma unroll
  for (int st = 0; st < NSTEP; ++st) {
    const int d0 = st * 16 + hh * 8;
    if constexpr (KSHIFT) {
      uint4 r = make_uint4(0, 0, 0, 0);
      if (q < a.Lq && d0 < E) r = *reinterpret_cast<const uint4*>(Q + q * a.qs[2] + d0);
      const halfx8 raw = __builtin_bit_cast(halfx8, r);
      const float qsc = a.scale * kLog2e;
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[st][j] = (_Float16)((float)raw[j] * qsc);
    } else if constexpr (VEC) {
      uint4 r = make_uint4(0, 0, 0, 0);
      if (q < a.Lq && d0 < E) r = *reinterpret_cast<const uint4*>(Q + q * a.qs[2] + d0);
      r.x ^= qneg;
      r.y ^= qneg;
      r.z ^= qneg;
      r.w ^= qneg;
      qf[st] = __builtin_bit_cast(halfx8, r);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint16_t bits = 0;
        if (q < a.Lq && d0 + j < E) bits = Q[q * a.qs[2] + d0 + j] ^ (uint16_t)qneg;
        qf[st][j] = __builtin_bit_cast(_Float16, bits);
      }
    }
  }

  // Row sums by MFMA: where the value dims leave a padding row in the last 32-dim block (DK not
  // a multiple of 32; Ev <= DK), V's dim Ev is staged as 1 for every key, so O^T row Ev
  // accumulates sum_k P[q][k] -- the sum of the fp16 weights the PV product actually uses -- and
  // the softmax loop skips its 32 adds and exchange per tile.  The lazy rescale scales that row
  // with the rest.  Fixed at compile time: a run-time choice between the two loop bodies costs
  // the two-key-group instance its register budget.  Dim parts (DS > 1) would put the row in
  // another wave's blocks.
  constexpr bool kOnes = DS == 1 && DK % 32 != 0;
  constexpr bool ones = kOnes;

  // K/V staging: chunk c of this thread covers row (c / CHR) and dims 8*(c % CHR) of the tile.
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)K, (short)0, (int)(((int64_t)(Lk > 0 ? Lk - 1 : 0) * a.ks[2] + E) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)V, (short)0, (int)(((int64_t)(Lk > 0 ? Lk - 1 : 0) * a.vs[2] + Ev) * 2), 0x00020000);
  uint4 kreg[KCH], vreg[VCH];
  auto fetch = [&](int kv0) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const int c = tid + i * NT;
        const int key = c / KCHR, d0 = (c % KCHR) * 8;
        const bool ok = c < BKV * KCHR && kv0 + key < Lk && d0 < E;
        kreg[i] = bload(k_rsrc, ok ? (uint32_t)(((int64_t)(kv0 + key) * a.ks[2] + d0) * 2) : kOOB);
      }
      // V chunks go key-fastest across lanes: consecutive rows of pitch VRP put 16 lanes'
      // 16-byte writes on distinct banks.
#pragma unroll
      for (int i = 0; i < VCH; ++i) {
        const int c = tid + i * NT;
        const int key = c % BKV, d0 = (c / BKV) * 8;
        const bool ok = c < BKV * VCHR && kv0 + key < Lk && d0 < Ev;
        vreg[i] = bload(v_rsrc, ok ? (uint32_t)(((int64_t)(kv0 + key) * a.vs[2] + d0) * 2) : kOOB);
      }
    }
  };
  auto stage = [&](int kv0) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < KCH; ++i) {
        const int c = tid + i * NT;
        uint4 val = kreg[i];
        // KSHIFT: dim KSD of every key is 1 (E <= KSD, so the chunk was loaded as zeros)
        if constexpr (KSHIFT)
          if ((c % KCHR) * 8 == KSD) val = make_uint4(0x3c00u, 0u, 0u, 0u);
        if (c < BKV * KCHR) *reinterpret_cast<uint4*>(&Ks[(c / KCHR) * KP + (c % KCHR) * 8]) = val;
      }
#pragma unroll
      for (int i = 0; i < VCH; ++i) {
        const int c = tid + i * NT;
        uint4 val = vreg[i];
        // the sum column: value 1 at dim Ev of every existing key (Ev % 8 == 0 under VEC; the
        // chunk was loaded as zeros)
        if constexpr (kOnes)
          if (ones && (c / BKV) * 8 == Ev && kv0 + c % BKV < Lk) val = make_uint4(0x3c00u, 0u, 0u, 0u);
        if (c < BKV * VCHR) *reinterpret_cast<uint4*>(&Vr[(c % BKV) * VRP + (c / BKV) * 8]) = val;
      }
    } else {
      for (int idx = tid; idx < BKV * DK; idx += NT) {
        const int key = idx / DK, d = idx - key * DK;
        uint16_t bits = 0;
        if (kv0 + key < Lk && d < E) bits = K[(int64_t)(kv0 + key) * a.ks[2] + d];
        Ks[key * KP + d] = bits;
      }
      for (int idx = tid; idx < BKV * DVB * 32; idx += NT) {
        const int key = idx / (DVB * 32), d = idx - key * (DVB * 32);
        uint16_t bits = 0;
        if (kv0 + key < Lk && d < Ev) bits = V[(int64_t)(kv0 + key) * a.vs[2] + d];
        if (kOnes && ones && kv0 + key < Lk && d == Ev) bits = 0x3c00u;  // the sum column
        Vr[key * VRP + d] = bits;
      }
    }
  };

  floatx16 acc[DVBP];
#pragma unroll
  for (int i = 0; i < DVBP; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float sl2 = fabsf(a.scale) * kLog2e;  // not KSHIFT: >= 0, the sign went into Q
  bool m_big = false;  // KSHIFT: |m| > 2^15, subtracted by the lane (dim KSD carries 0)
  const bool qok = q < a.Lq;
  const int mask_kind = MASK >= 0 ? MASK : a.mask_kind;
  // This lane's mask row (query q of head `head`), addressed per key by one 32-bit multiply.
  const uint8_t* mrow_b = nullptr;
  const uint16_t* mrow_h = nullptr;
  const float* mrow_f = nullptr;
  const int mk = (int)a.ms[3];
  if (mask_kind != MTHIP_MASK_NONE && qok) {
    const int64_t off = b * a.ms[0] + head * a.ms[1] + q * a.ms[2];
    if (mask_kind == MTHIP_MASK_BOOL)
      mrow_b = reinterpret_cast<const uint8_t*>(a.mask) + off;
    else if (a.mask_dtype == MTHIP_F16)
      mrow_h = reinterpret_cast<const uint16_t*>(a.mask) + off;
    else
      mrow_f = reinterpret_cast<const float*>(a.mask) + off;
  }

  fetch(kb + grp * BKV);
  const int iters = (Lk - kb + BKV * KG - 1) / (BKV * KG);
  for (int it = 0; it < iters; ++it) {
    const int kv0 = kb + (it * KG + grp) * BKV;
    __syncthreads();  // every wave is done with the previous tile
    stage(kv0);
    __syncthreads();
    if (kv0 + KG * BKV < Lk) fetch(kv0 + KG * BKV);  // next tile's loads overlap this tile's math
    if (KG > 1 && kv0 >= Lk) continue;  // a key group past the last tile only keeps the barriers

    // Scores and their max: raw (unscaled) on tiles with every key valid and unmasked, scaled to
    // log2 units on the others, so that an additive mask enters as given whatever the scale
    // (zero included).  mult takes either to log2 units below.
    float s[2][16];
    float mx = -INFINITY;
    const bool checked = kv0 + BKV > Lk || a.causal || mask_kind != MTHIP_MASK_NONE;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      floatx16 t;
#pragma unroll
      for (int r = 0; r < 16; ++r) t[r] = 0.0f;
#pragma unroll
      for (int st = 0; st < NSTEP; ++st) {
        const halfx8 kf = *reinterpret_cast<const halfx8*>(&Ks[(sb * 32 + col) * KP + st * 16 + hh * 8]);
        t = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[st], t, 0, 0, 0);
      }
      if (!checked) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[sb][r] = t[r];
          mx = fmaxf(mx, t[r]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + sb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
          float v = KSHIFT ? t[r] : t[r] * sl2;
          if (key >= Lk) {
            v = -INFINITY;
          } else {
            if (a.causal && key > q) v = -INFINITY;
            if (mask_kind == MTHIP_MASK_BOOL) {
              if (qok && !mrow_b[key * mk]) v = -INFINITY;
            } else if (mask_kind == MTHIP_MASK_ADD && qok) {
              v = fmaf(mrow_h ? h2f_bits(mrow_h[key * mk]) : mrow_f[key * mk], kLog2e, v);
            }
          }
          s[sb][r] = v;
          mx = fmaxf(mx, v);
        }
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // Lazy rescaling: the running max (log2 units) moves only when a score exceeds it by more
    // than 8, so P <= 2^8 (exact in fp16 and in the fp32 sums) and most tiles skip the
    // accumulator rescale.  O = acc / l is unchanged by the choice of reference max.
    const float mult = KSHIFT || checked ? 1.0f : sl2;
    // KSHIFT: the scores are relative to the m the tile ran with (dim KSD's -m, 0 before any
    // key or when the lane subtracts m itself)
    const float m_tile = KSHIFT ? (m_run == -INFINITY || m_big ? 0.0f : m_run) : 0.0f;
    const float m_cand = KSHIFT ? fmaxf(m_run, m_tile + mx) : fmaxf(m_run, mx * mult);
    if (m_cand > m_run + 8.0f) {
      float m_new = m_cand;
      if constexpr (KSHIFT) {
        // kept representable in fp16 (a new max a fraction of an ulp below the tile's max
        // leaves P <= 2^(8 + ulp/2)); dim KSD carries -m from the next tile on
        m_big = fabsf(m_cand) > 32768.0f;
        const _Float16 mh = (_Float16)(m_big ? 0.0f : -m_cand);
        if (!m_big) m_new = -(float)mh;
        if (hh == 1) qf[KSD / 16][0] = mh;
      }
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 when m_run = -inf
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < DVBP; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] *= alpha;
      if constexpr (KSHIFT) {  // re-base this tile's scores on the new max
        const float d = (m_big ? 0.0f : m_new) - m_tile;
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[sb][r] -= d;
      }
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    if constexpr (KSHIFT) {  // lanes whose max dim KSD cannot carry subtract it here
      if (__builtin_amdgcn_ballot_w64(m_big)) {
        const float d = m_big ? m_use : 0.0f;
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[sb][r] -= d;
      }
    }
    // exp2 argument: KSHIFT the score as it stands, else score * mult - m_use
    auto p_of = [&](float x) {
      return KSHIFT ? __builtin_amdgcn_exp2f(x) : __builtin_amdgcn_exp2f(fmaf(x, mult, -m_use));
    };
    if (kOnes && ones) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[sb][r] = p_of(s[sb][r]);
    } else {
      float psum = 0.0f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[sb][r] = p_of(s[sb][r]);
          psum += s[sb][r];
        }
      psum += __shfl_xor(psum, 32, 64);
      l_run += psum;
    }

    // O^T += V^T . P^T, four 16-key steps.
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        halfx8 pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[j] = (_Float16)s[sb][st * 8 + j];
#pragma unroll
        for (int ii = 0; ii < DVBP; ++ii) {
          const int i = dp * DVBP + ii;  // output block (wave-uniform)
          if (DS > 1 && i >= DVB) break;
          // Lane l needs V[k][i*32 + l%32] for keys k = K0+0..3 and K0+8..11, K0 = sb*32 +
          // st*16 + 4*(l/32).  In each 16-lane group the transposing read hands lane j the
          // halves [j%4] of the rows read by lanes j/4, j/4+4, j/4+8, j/4+12; so lane r of
          // the group points at key K0 + r/4, dims 16*((l/16)%2) + 4*(r%4) .. +3.
          const uint16_t* v0 = &Vr[(sb * 32 + st * 16 + hh * 4 + ((lane & 15) >> 2)) * VRP + i * 32 +
                                   16 * ((lane >> 4) & 1) + 4 * (lane & 3)];
          const halfx4 lo = tr_read16(v0);
          const halfx4 hi = tr_read16(v0 + 8 * VRP);
          const halfx8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          acc[ii] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, acc[ii], 0, 0, 0);
        }
      }
    }
  }

  if (kOnes && ones) {
    // O^T[Ev][q] sits in register 4*(o/8) + o%4 of block Ev/32 (o = Ev % 32) in the lanes of
    // half (o/4) % 2; every lane takes its query's value from there.
    const int ib = Ev >> 5, o = Ev & 31, rr = 4 * (o >> 3) + (o & 3), half = (o >> 2) & 1;
    float v = 0.0f;
#pragma unroll
    for (int i = 0; i < DVBP; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) v = (i == ib && r == rr) ? acc[i][r] : v;
    l_run = __shfl(v, col + 32 * half, 64);
  }

  if constexpr (KG > 1) {
    // Fold group 1's (max, sum, accumulator) into group 0: the same lane of both groups holds
    // the same query and the same output dims.  A group that saw no key (or only masked ones)
    // has max -inf and contributes nothing; if neither saw one, the sum stays 0 (NaN output).
    float* xl = reinterpret_cast<float*>(smem) + tid * 17;
    __syncthreads();  // every wave is done with the last tile
    if (grp == 1) {
      xl[0] = m_run;
      xl[1] = l_run;
    }
    __syncthreads();
    float a0 = 1.0f, a1 = 0.0f;
    if (grp == 0) {
      const float m1 = xl[0], l1 = xl[1];
      const float m = fmaxf(m_run, m1);
      a0 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
      a1 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - m);
      l_run = l_run * a0 + l1 * a1;
      m_run = m;  // the merged sum and accumulator are relative to the merged max
    }
#pragma unroll
    for (int i = 0; i < DVB; ++i) {
      __syncthreads();
      if (grp == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) xl[r] = acc[i][r];
      }
      __syncthreads();
      if (grp == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = acc[i][r] * a0 + xl[r] * a1;
      }
    }
    if (grp != 0) return;
  }

  if (!qok) return;
  if (gridDim.z > 1) {
    // one key split: the unnormalised accumulator and (max, sum) for flash_combine_kernel
    float* row = a.part + (((int64_t)blockIdx.z * gridDim.y + bh) * a.Lq + q) * a.part_pitch;
#pragma unroll
    for (int i = 0; i < DVBP; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = (dp * DVBP + i) * 32 + 8 * g + 4 * hh;
        if (d0 < DVB * 32)
          *reinterpret_cast<float4*>(row + d0) = make_float4(acc[i][4 * g], acc[i][4 * g + 1], acc[i][4 * g + 2],
                                                             acc[i][4 * g + 3]);
      }
    if (dp == 0 && hh == 0) *reinterpret_cast<float2*>(row + DVB * 32) = make_float2(m_run, l_run);
    return;
  }
  uint16_t* O = reinterpret_cast<uint16_t*>(a.o) + b * a.os[0] + head * a.os[1] + q * a.os[2];
  // A fully masked row has l = 0 and, every P being 0, a zero accumulator: 0 * (1/0) = NaN, the
  // reference's 0/0.
  const float inv_l = 1.0f / l_run;
  if constexpr (VEC) {
    // Under VEC, Ev and the output strides are multiples of 8 and the base is 16-byte aligned,
    // so every 4-dim group below Ev is whole and 8-byte aligned.  All values are narrowed in one
    // branch-free block, where the 16*DVB independent conversion chains interleave, and the
    // stores follow, each behind its bounds test: converting inside the guarded store loop split
    // the block at every group and left each ~21-instruction chain to run at full latency with
    // one wave per SIMD (about 5 us of a 16x16-latent attention).  The narrowing is f2h_nonnan;
    // a wave in which some lane met a NaN (a fully masked row) converts again with f2h_generic.
    uint2 h[DVBP][4];
    auto convert = [&](auto narrow) {
#pragma unroll
      for (int i = 0; i < DVBP; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          h[i][g].x = narrow(acc[i][4 * g] * inv_l) | (narrow(acc[i][4 * g + 1] * inv_l) << 16);
          h[i][g].y = narrow(acc[i][4 * g + 2] * inv_l) | (narrow(acc[i][4 * g + 3] * inv_l) << 16);
        }
    };
    bool nan_seen = false;
    convert([&](float x) {
      nan_seen |= x != x;
      return f2h_nonnan(x);
    });
    if (__builtin_amdgcn_ballot_w64(nan_seen)) convert([](float x) { return (uint32_t)f2h_generic(x); });
#pragma unroll
    for (int i = 0; i < DVBP; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = (dp * DVBP + i) * 32 + 8 * g + 4 * hh;
        if (d0 < Ev) *reinterpret_cast<uint2*>(O + d0) = h[i][g];
      }
  } else {
#pragma unroll
    for (int i = 0; i < DVBP; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = (dp * DVBP + i) * 32 + 8 * g + 4 * hh;
        if (d0 >= Ev) continue;
        for (int t = 0; t < 4 && d0 + t < Ev; ++t) O[d0 + t] = f2h_generic(acc[i][4 * g + t] * inv_l);
      }
  }
}

// Merges the key splits of the flash kernel: per query, m = max_z m_z, l = sum_z l_z 2^(m_z - m),
// o = (sum_z acc_z 2^(m_z - m)) / l, narrowed once (a split that saw only masked keys has
// m_z = -inf and weight 0; with none left, l = 0 and 0/0 gives the reference's NaN).  One thread
// per 4 consecutive output dims of one query.
__global__ __launch_bounds__(256) void flash_combine_kernel(const FlashArgs a, int splits, int dvb32) {
  const int groups = (int)((a.Ev + 3) / 4);
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (query, 4-dim group) of head blockIdx.y
  if (t >= a.Lq * groups) return;
  const int64_t bh = blockIdx.y, BH = gridDim.y;
  const int64_t q = t / groups;
  const int d0 = (int)(t - q * groups) * 4;
  float m = -INFINITY;
  for (int z = 0; z < splits; ++z) m = fmaxf(m, a.part[((z * BH + bh) * a.Lq + q) * a.part_pitch + dvb32]);
  float l = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int z = 0; z < splits; ++z) {
    const float* row = a.part + ((z * BH + bh) * a.Lq + q) * a.part_pitch;
    const float2 ml = *reinterpret_cast<const float2*>(row + dvb32);
    const float w = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - m);
    const float4 v = *reinterpret_cast<const float4*>(row + d0);
    l += ml.y * w;
    o[0] += v.x * w;
    o[1] += v.y * w;
    o[2] += v.z * w;
    o[3] += v.w * w;
  }
  const float inv_l = 1.0f / l;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  uint16_t* O = reinterpret_cast<uint16_t*>(a.o) + b * a.os[0] + h * a.os[1] + q * a.os[2];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (d0 + j < a.Ev) O[d0 + j] = f2h_generic(o[j] * inv_l);
}

// One wave per query: lanes split the head dims; online softmax over keys in fp32 (scores and
// the output accumulate in fp32, values widened from the storage dtype).
template <typename T, int VPL>
__global__ __launch_bounds__(256) void attention_rowwise_kernel(const FlashArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t bh = blockIdx.y;
  const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= a.Lq) return;
  const int64_t b = bh / a.H, head = bh - b * a.H, kvh = head / (a.H / a.Hk);
  const T* Q = reinterpret_cast<const T*>(a.q) + b * a.qs[0] + head * a.qs[1] + q * a.qs[2];
  const T* K = reinterpret_cast<const T*>(a.k) + b * a.ks[0] + kvh * a.ks[1];
  const T* V = reinterpret_cast<const T*>(a.v) + b * a.vs[0] + kvh * a.vs[1];
  float qv[VPL], o[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t d = lane + 64 * j;
    qv[j] = d < a.E ? Elem<T>::load(Q, d) : 0.0f;
    o[j] = 0.0f;
  }
  float m_run = -INFINITY, l_run = 0.0f;
  for (int64_t key = 0; key < a.Lk; ++key) {
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int64_t d = lane + 64 * j;
      if (d < a.E) part += qv[j] * Elem<T>::load(K, key * a.ks[2] + d);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
    float sc = part * a.scale;
    if (a.causal && key > q) sc = -INFINITY;
    sc = mask_value(a, b, head, q, key, sc);
    const float m_new = fmaxf(m_run, sc);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = expf(m_run - m_use);
    const float p = expf(sc - m_use);
    l_run = l_run * alpha + p;
    m_run = m_new;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int64_t d = lane + 64 * j;
      o[j] = o[j] * alpha + (d < a.Ev ? p * Elem<T>::load(V, key * a.vs[2] + d) : 0.0f);
    }
  }
  T* O = reinterpret_cast<T*>(a.o) + b * a.os[0] + head * a.os[1] + q * a.os[2];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t d = lane + 64 * j;
    if (d < a.Ev) Elem<T>::store(O, d, o[j] / l_run);
  }
}

template <int DK, int WAVES, int KG, int DS = 1>
void launch_flash_w(const FlashArgs& a, int64_t bh, hipStream_t s, bool vec, unsigned splits) {
  const dim3 grid((unsigned)ceil_div(a.Lq, 32 * WAVES / DS), (unsigned)bh, splits);
  const dim3 block(64 * WAVES * KG);
  if (!vec) {
    hipLaunchKernelGGL((flash_fwd_f16_kernel<DK, false, -1, WAVES, KG>),
                       dim3((unsigned)ceil_div(a.Lq, 32 * WAVES), (unsigned)bh, splits), block, 0, s, a);
  } else if (a.mask_kind == MTHIP_MASK_NONE) {
    hipLaunchKernelGGL((flash_fwd_f16_kernel<DK, true, MTHIP_MASK_NONE, WAVES, KG, DS>), grid, block, 0, s, a);
  } else if (a.mask_kind == MTHIP_MASK_BOOL) {
    hipLaunchKernelGGL((flash_fwd_f16_kernel<DK, true, MTHIP_MASK_BOOL, WAVES, KG, DS>), grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL((flash_fwd_f16_kernel<DK, true, MTHIP_MASK_ADD, WAVES, KG, DS>), grid, block, 0, s, a);
  }
}

// Which flash instance serves a problem: waves per key group, key groups, dim parts and the
// query blocks of its grid (so that the key-split planner and the launch agree).
struct FlashShape {
  int waves, kg, ds;
  int64_t gx;  // workgroups along the queries
};

template <int DK>
FlashShape flash_shape(const FlashArgs& a, int64_t bh, bool vec) {
  // Two key groups (8 waves) for small heads over long key sequences, where the extra waves per
  // SIMD hide the score -> softmax -> PV chain (SD self-attention at 64x64: -6 %); with few
  // keys (cross-attention on 77 tokens) the merge costs more than it saves.
  if constexpr (DK <= 48) {
    if (a.Lk >= 1024 && vec && a.mask_kind == MTHIP_MASK_NONE) {
      // Eight waves per key group (256 queries per workgroup, one workgroup per CU) where that
      // still gives every CU a workgroup: each staged K/V tile then serves twice the queries
      // (SD 64x64 self-attention 92.8 -> 86.4 us; four waves per workgroup had 93, two 196).
      // MTHIP_FLASH_W=4 keeps four.
      const char* wenv = std::getenv("MTHIP_FLASH_W");
      const bool w8 = wenv ? wenv[0] == '8' : ceil_div(a.Lq, 256) * bh >= a.cus;
      return w8 ? FlashShape{8, 2, 1, ceil_div(a.Lq, 256)} : FlashShape{4, 2, 1, ceil_div(a.Lq, 128)};
    }
  }
  // Head dims above 80 (SD's 160 at the 16x16 and 8x8 latents): four dim parts, so a workgroup
  // serves 32 queries and each wave runs a quarter of the value product and of the epilogue.
  // Those grids are 16-32 workgroups of one wave per SIMD, whose issue slots bound them; the
  // parts quadruple the SIMDs in use at the cost of recomputing each block's scores (measured at
  // 16x16: one key tile 9.9 -> 7.0 us, 77 keys 12.1 -> 9.5 us, 256 keys 14.6 -> 12.5 us).  At
  // head dim 80 the recomputed scores cost as much as the parts save (32x32, 1024 keys: 25.5
  // against 27.3 us with two parts).
  if (DK > 80 && vec) return FlashShape{4, 1, 4, ceil_div(a.Lq, 32)};
  // 4 waves (128 queries) per workgroup.  Measured on every SD shape (self/cross attention at
  // 64x64, 32x32, 16x16 latents), 4 waves were at least as fast as 2 even where they leave CUs
  // idle: each wave then stages a quarter of the K/V tile, and the shared tile serves 128 queries.
  return FlashShape{4, 1, 1, ceil_div(a.Lq, 128)};
}

template <int DK>
void launch_flash(const FlashArgs& a, int64_t bh, hipStream_t s, bool vec, unsigned splits) {
  const FlashShape sh = flash_shape<DK>(a, bh, vec);
  if constexpr (DK <= 48) {
    if (sh.kg == 2) {
      if (sh.waves == 8)
        hipLaunchKernelGGL((flash_fwd_f16_kernel<DK, true, MTHIP_MASK_NONE, 8, 2>),
                           dim3((unsigned)sh.gx, (unsigned)bh, splits), dim3(1024), 0, s, a);
      else
        hipLaunchKernelGGL((flash_fwd_f16_kernel<DK, true, MTHIP_MASK_NONE, 4, 2>),
                           dim3((unsigned)sh.gx, (unsigned)bh, splits), dim3(512), 0, s, a);
      return;
    }
  }
  if constexpr (DK > 80) {
    if (sh.ds == 4) {
      launch_flash_w<DK, 4, 1, 4>(a, bh, s, vec, splits);
      return;
    }
  }
  launch_flash_w<DK, 4, 1>(a, bh, s, vec, splits);
}

// Key splits for a grid that leaves CUs idle (the 32x32 latent's 128 workgroups): enough splits
// of whole 128-key runs to give every CU a workgroup, each keeping >= 512 keys, at most 8; 1 =
// none.  A split's own pipeline start and the combine launch cost ~3 us, so short key ranges
// stay whole (SD 32x32 self-attention, 1024 keys: 25.1 -> 23.1 us with 2 splits; 16x16, 256
// keys: 11.0 -> 13.6 us with 2, so none).  MTHIP_FLASH_SPLIT=n forces n (1 turns it off).
template <int DK>
int flash_splits(const FlashArgs& a, int64_t bh, bool vec, int* chunk) {
  const FlashShape sh = flash_shape<DK>(a, bh, vec);
  const int64_t wgs = sh.gx * bh;
  const int64_t runs = ceil_div(a.Lk, 128);
  int64_t n = wgs < a.cus ? std::min<int64_t>(ceil_div((int64_t)a.cus, wgs), runs / 4) : 1;
  if (const char* e = std::getenv("MTHIP_FLASH_SPLIT")) n = std::max(1, std::atoi(e));
  n = std::max<int64_t>(1, std::min<int64_t>({n, runs, 8}));
  const int64_t c = ceil_div(runs, n) * 128;
  *chunk = (int)c;
  return (int)ceil_div(a.Lk, c);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace mthip

using namespace mthip;

extern "C" int mthip_sdpa(int device, int dtype, const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                          const void* v, const int64_t* vs, void* o, const int64_t* os, int64_t B, int64_t H,
                          int64_t Hk, int64_t Lq,
                          int64_t Lk, int64_t E, int64_t Ev, int mask_kind, int mask_dtype, const void* mask,
                          const int64_t* mask_strides, int is_causal, int has_scale, double scale) {
  MTHIP_REQUIRE(dtype == MTHIP_F16 || dtype == MTHIP_F32, "mthip_sdpa: dtype must be F16 or F32");
  MTHIP_REQUIRE(B >= 0 && H > 0 && Hk > 0 && H % Hk == 0, "mthip_sdpa: key heads must divide query heads");
  MTHIP_REQUIRE(Lq >= 0 && Lk >= 0 && E > 0 && Ev > 0, "mthip_sdpa: bad extents");
  MTHIP_REQUIRE(E <= 512 && Ev <= 512, "mthip_sdpa: head dims above 512 are not supported");
  MTHIP_REQUIRE(mask_kind >= MTHIP_MASK_NONE && mask_kind <= MTHIP_MASK_ADD, "mthip_sdpa: unknown mask kind");
  MTHIP_REQUIRE(mask_kind == MTHIP_MASK_NONE || (mask != nullptr && mask_strides != nullptr),
                "mthip_sdpa: mask pointer/strides missing");
  MTHIP_REQUIRE(mask_kind != MTHIP_MASK_ADD || mask_dtype == MTHIP_F32 || mask_dtype == MTHIP_F16,
                "mthip_sdpa: additive mask must be F32 or F16");
  if (B == 0 || Lq == 0) return MTHIP_OK;
  MTHIP_REQUIRE(B * H <= 65535, "mthip_sdpa: batch*heads must be <= 65535");
  hipStream_t s = stream_for(device);
  if (!s) return MTHIP_ERR_HIP;
  if (int rc = use_device(device)) return rc;
  FlashArgs a{};
  {
    static int cus_cached[64] = {0};
    int n = device >= 0 && device < 64 ? cus_cached[device] : 0;
    if (n == 0) {
      if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n < 1) n = 256;
      if (device >= 0 && device < 64) cus_cached[device] = n;
    }
    a.cus = n;
  }
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = qs[i];
    a.ks[i] = ks[i];
    a.vs[i] = vs[i];
  }
  if (os) {
    for (int i = 0; i < 3; ++i) a.os[i] = os[i];
  } else {  // contiguous [B, H, Lq, Ev]
    a.os[2] = Ev;
    a.os[1] = Lq * Ev;
    a.os[0] = H * Lq * Ev;
  }
  a.H = H;
  a.Hk = Hk;
  a.Lq = Lq;
  a.Lk = Lk;
  a.E = E;
  a.Ev = Ev;
  a.mask_kind = mask_kind;
  a.mask_dtype = mask_dtype;
  a.mask = mask;
  if (mask_kind != MTHIP_MASK_NONE)
    for (int i = 0; i < 4; ++i) a.ms[i] = mask_strides[i];
  a.causal = is_causal;
  // scale=None is 1/sqrt(E); a given scale is used as is (tensor.cpp:31019, 31182).
  a.scale = (float)(has_scale ? scale : 1.0 / std::sqrt((double)E));
  const int64_t bh = B * H;
  const int64_t dmax = std::max(E, Ev);
  // One head's K and V must be addressable by 32-bit buffer offsets.
  const bool small_heads = ((Lk > 0 ? Lk - 1 : 0) * std::max(ks[2], vs[2]) + dmax) * 2 < (int64_t(1) << 31);
  // The flash kernel needs a finite scale (its running max works in scaled units); an infinite
  // or NaN one takes the row-wise kernel, which multiplies each score by it as the reference does.
  if (dtype == MTHIP_F16 && Lk > 0 && dmax <= 160 && small_heads && std::isfinite(a.scale)) {
    // The 48-dim VEC instance pre-scales Q by scale * log2(e) in fp16 (KSHIFT): for |scale *
    // log2 e| outside [2^-10, 1] (but 0) that product could overflow or drop Q's low bits, and
    // the generic instance, which scales the fp32 scores, runs instead.
    const double sl2 = std::fabs((double)a.scale) * 1.4426950408889634;
    const bool prescale_ok = !(dmax <= 48 && E <= 40 && dmax > 32) || a.scale == 0.0f || (sl2 >= 1.0 / 1024.0 && sl2 <= 1.0);
    const bool vec = E % 8 == 0 && Ev % 8 == 0 && qs[2] % 8 == 0 && ks[2] % 8 == 0 && vs[2] % 8 == 0 &&
                     qs[0] % 8 == 0 && qs[1] % 8 == 0 && ks[0] % 8 == 0 && ks[1] % 8 == 0 && vs[0] % 8 == 0 &&
                     vs[1] % 8 == 0 && a.os[0] % 8 == 0 && a.os[1] % 8 == 0 && a.os[2] % 8 == 0 &&
                     aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && prescale_ok;
    // the instance's padded value dims (DVB * 32) and key splits
    auto run = [&](auto dk_c) -> int {
      constexpr int DK = decltype(dk_c)::value;
      int chunk = 0;
      const int splits = flash_splits<DK>(a, bh, vec, &chunk);
      void* ws = nullptr;
      a.kv_chunk = splits > 1 ? chunk : (int)Lk;
      if (splits > 1) {
        constexpr int dvb32 = (DK + 31) / 32 * 32;
        a.part_pitch = dvb32 + 4;
        if (int rc = mthip_malloc(device, (size_t)splits * (size_t)bh * (size_t)Lq * a.part_pitch * sizeof(float), &ws))
          return rc;
        a.part = static_cast<float*>(ws);
      }
      launch_flash<DK>(a, bh, s, vec, (unsigned)splits);
      int rc = check_launch("flash_fwd_f16_kernel");
      if (rc == MTHIP_OK && splits > 1) {
        constexpr int dvb32 = (DK + 31) / 32 * 32;
        const int64_t per_bh = Lq * ceil_div(Ev, 4);
        hipLaunchKernelGGL(flash_combine_kernel, dim3((unsigned)ceil_div(per_bh, 256), (unsigned)bh), dim3(256), 0, s,
                           a, splits, dvb32);
        rc = check_launch("flash_combine_kernel");
      }
      mthip_free(device, ws);
      return rc;
    };
    if (dmax <= 32) return run(std::integral_constant<int, 32>{});
    // the 48-dim instance keeps dim 40 free for its max shift (KSHIFT): E 41..48 take 64
    if (dmax <= 48 && E <= 40) return run(std::integral_constant<int, 48>{});
    if (dmax <= 64) return run(std::integral_constant<int, 64>{});
    if (dmax <= 80) return run(std::integral_constant<int, 80>{});
    if (dmax <= 128) return run(std::integral_constant<int, 128>{});
    return run(std::integral_constant<int, 160>{});
  }
  dim3 grid((unsigned)ceil_div(Lq, 4), (unsigned)bh);
  if (dtype == MTHIP_F16) {
    if (dmax <= 64)
      hipLaunchKernelGGL((attention_rowwise_kernel<uint16_t, 1>), grid, dim3(256), 0, s, a);
    else if (dmax <= 256)
      hipLaunchKernelGGL((attention_rowwise_kernel<uint16_t, 4>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((attention_rowwise_kernel<uint16_t, 8>), grid, dim3(256), 0, s, a);
  } else {
    if (dmax <= 64)
      hipLaunchKernelGGL((attention_rowwise_kernel<float, 1>), grid, dim3(256), 0, s, a);
    else if (dmax <= 256)
      hipLaunchKernelGGL((attention_rowwise_kernel<float, 4>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((attention_rowwise_kernel<float, 8>), grid, dim3(256), 0, s, a);
  }
  return check_launch("attention_rowwise_kernel");
}
