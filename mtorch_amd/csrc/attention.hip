// scaled_dot_product_attention: flash-style fused kernel on MFMA (fp16) and a wave-per-query
// kernel for fp32 and shapes outside the MFMA instances.
//
// MFMA kernel layout.  A workgroup is 4 wave64s; each wave owns 32 queries of one (batch, head).
// Per 32-key tile it computes the transposed score block S^T = K . Q^T with
// v_mfma_f32_32x32x16_f16, so lane l holds the scores of query (l % 32) against 16 keys in its
// accumulator: the online-softmax max/sum of a query is an in-register reduction plus one
// exchange with lane l^32.  Those same accumulator registers, converted to fp16, are exactly the
// B operand of O^T += V^T . P^T (register r <-> key 8*(r/4) + 4*(l/32) + r%4 in both products),
// so P never leaves registers.  K is staged in LDS row-major and V transposed (keys contiguous).
// Softmax statistics and the output accumulator are fp32; fully masked rows end as 0/0 = NaN,
// as the reference's softmax of an all -inf row does (tensor.cpp:30429-30442).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "common.h"

namespace mthip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

struct FlashArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t qs[3], ks[3], vs[3];  // element strides: batch, head, sequence (last dim contiguous)
  int64_t H, Hk, Lq, Lk, E, Ev;
  int mask_kind, mask_dtype;
  const void* mask;
  int64_t ms[4];  // mask strides: b, h, q, k
  int causal;
  float scale;
};

__device__ __forceinline__ float mask_value(const FlashArgs& a, int64_t b, int64_t h, int64_t q, int64_t k,
                                            float score) {
  if (a.mask_kind == MTHIP_MASK_NONE) return score;
  const int64_t off = b * a.ms[0] + h * a.ms[1] + q * a.ms[2] + k * a.ms[3];
  if (a.mask_kind == MTHIP_MASK_BOOL) return reinterpret_cast<const uint8_t*>(a.mask)[off] ? score : -INFINITY;
  if (a.mask_dtype == MTHIP_F16) return score + h2f_bits(reinterpret_cast<const uint16_t*>(a.mask)[off]);
  return score + reinterpret_cast<const float*>(a.mask)[off];
}

template <int DK>
__global__ __launch_bounds__(256) void flash_fwd_f16_kernel(const FlashArgs a) {
  constexpr int NSTEP = DK / 16;          // K-dim MFMA steps of the score product
  constexpr int DVB = (DK + 31) / 32;     // 32-row output blocks of O^T
  constexpr int KP = DK + 8;              // LDS pitch of the K tile (halves)
  constexpr int VP = 32 + 8;              // LDS pitch of the transposed V tile (halves)
  __shared__ __align__(16) uint16_t Ks[32 * KP];
  __shared__ __align__(16) uint16_t Vt[DVB * 32 * VP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hh = lane >> 5, col = lane & 31;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.H, head = bh - b * a.H;
  const int64_t kvh = head / (a.H / a.Hk);
  const int64_t q = (int64_t)blockIdx.x * 128 + wave * 32 + col;
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.q) + b * a.qs[0] + head * a.qs[1];
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.k) + b * a.ks[0] + kvh * a.ks[1];
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.v) + b * a.vs[0] + kvh * a.vs[1];

  // Q^T fragments (B operand of S^T): query q, dims step*16 + hh*8 + [0, 8).
  halfx8 qf[NSTEP];
#pragma unroll
  for (int st = 0; st < NSTEP; ++st) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t d = st * 16 + hh * 8 + j;
      uint16_t bits = 0;
      if (q < a.Lq && d < a.E) bits = Q[q * a.qs[2] + d];
      qf[st][j] = __builtin_bit_cast(_Float16, bits);
    }
  }

  floatx16 acc[DVB];
#pragma unroll
  for (int i = 0; i < DVB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float log2e = 1.4426950408889634f;

  for (int64_t kv0 = 0; kv0 < a.Lk; kv0 += 32) {
    __syncthreads();  // the previous tile has been consumed by every wave
    // Stage K[kv0 .. kv0+32) -> Ks[key][d] (zero beyond Lk / E).
    for (int idx = tid; idx < 32 * DK; idx += 256) {
      const int key = idx / DK, d = idx - key * DK;
      uint16_t bits = 0;
      if (kv0 + key < a.Lk && d < a.E) bits = K[(kv0 + key) * a.ks[2] + d];
      Ks[key * KP + d] = bits;
    }
    // Stage V transposed -> Vt[d][key].
    for (int idx = tid; idx < 32 * DVB * 32; idx += 256) {
      const int key = idx / (DVB * 32), d = idx - key * (DVB * 32);
      uint16_t bits = 0;
      if (kv0 + key < a.Lk && d < a.Ev) bits = V[(kv0 + key) * a.vs[2] + d];
      Vt[d * VP + key] = bits;
    }
    __syncthreads();

    floatx16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) {
      const halfx8 kf = *reinterpret_cast<const halfx8*>(&Ks[col * KP + st * 16 + hh * 8]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[st], s, 0, 0, 0);
    }

    // Scale, causal, mask, key bounds; tile max of this query.
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t key = kv0 + 8 * (r >> 2) + 4 * hh + (r & 3);
      float v = s[r] * a.scale;
      if (key >= a.Lk) {
        v = -INFINITY;
      } else {
        if (a.causal && key > q) v = -INFINITY;
        if (q < a.Lq) v = mask_value(a, b, head, q, key, v);
      }
      s[r] = v;
      mx = fmaxf(mx, v);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f((m_run - m_use) * log2e);
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = exp2f((s[r] - m_use) * log2e);
      psum += s[r];
    }
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < DVB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] *= alpha;

    // O^T += V^T . P^T over two 16-key steps.
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      halfx8 pf;
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[j] = (_Float16)s[st * 8 + j];
#pragma unroll
      for (int i = 0; i < DVB; ++i) {
        const uint16_t* vrow = &Vt[(i * 32 + col) * VP + st * 16 + hh * 4];
        const halfx4 lo = *reinterpret_cast<const halfx4*>(vrow);
        const halfx4 hi = *reinterpret_cast<const halfx4*>(vrow + 8);
        const halfx8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, acc[i], 0, 0, 0);
      }
    }
  }

  if (q >= a.Lq) return;
  uint16_t* O = reinterpret_cast<uint16_t*>(a.o) + (bh * a.Lq + q) * a.Ev;
  const float inv_l = 1.0f / l_run;
#pragma unroll
  for (int i = 0; i < DVB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t d = i * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
      if (d < a.Ev) O[d] = f2h_bits(l_run == 0.0f ? acc[i][r] / l_run : acc[i][r] * inv_l);
    }
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
  T* O = reinterpret_cast<T*>(a.o) + (bh * a.Lq + q) * a.Ev;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t d = lane + 64 * j;
    if (d < a.Ev) Elem<T>::store(O, d, o[j] / l_run);
  }
}

}  // namespace
}  // namespace mthip

using namespace mthip;

extern "C" int mthip_sdpa(int device, int dtype, const void* q, const int64_t* qs, const void* k, const int64_t* ks,
                          const void* v, const int64_t* vs, void* o, int64_t B, int64_t H, int64_t Hk, int64_t Lq,
                          int64_t Lk, int64_t E, int64_t Ev, int mask_kind, int mask_dtype, const void* mask,
                          const int64_t* mask_strides, int is_causal, double scale) {
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
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  for (int i = 0; i < 3; ++i) {
    a.qs[i] = qs[i];
    a.ks[i] = ks[i];
    a.vs[i] = vs[i];
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
  a.scale = (float)(scale > 0.0 ? scale : 1.0 / std::sqrt((double)E));
  const int64_t bh = B * H;
  if (dtype == MTHIP_F16 && Lk > 0) {
    const int64_t dmax = std::max(E, Ev);
    dim3 grid((unsigned)ceil_div(Lq, 128), (unsigned)bh);
    bool launched = true;
    if (dmax <= 32)
      hipLaunchKernelGGL(flash_fwd_f16_kernel<32>, grid, dim3(256), 0, s, a);
    else if (dmax <= 48)
      hipLaunchKernelGGL(flash_fwd_f16_kernel<48>, grid, dim3(256), 0, s, a);
    else if (dmax <= 64)
      hipLaunchKernelGGL(flash_fwd_f16_kernel<64>, grid, dim3(256), 0, s, a);
    else if (dmax <= 80)
      hipLaunchKernelGGL(flash_fwd_f16_kernel<80>, grid, dim3(256), 0, s, a);
    else if (dmax <= 128)
      hipLaunchKernelGGL(flash_fwd_f16_kernel<128>, grid, dim3(256), 0, s, a);
    else if (dmax <= 160)
      hipLaunchKernelGGL(flash_fwd_f16_kernel<160>, grid, dim3(256), 0, s, a);
    else
      launched = false;
    if (launched) return check_launch("flash_fwd_f16_kernel");
  }
  dim3 grid((unsigned)ceil_div(Lq, 4), (unsigned)bh);
  const int64_t dmax = std::max(E, Ev);
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
