/*
 * CPU oracle for mtorch's SD-UNet dense-inference hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of what kazhiramatsu/mtorch computes on x86-64 Linux, where every
 * MTORCH_USE_ACCELERATE / __ARM_NEON branch is compiled out and each op runs its portable
 * scalar path.  Citations are file:line into the reference tree.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker.  The product (mtorch_amd + libmthip) never links it.
 *
 * Conventions: every buffer is dense row-major (contiguous); fp16 data is IEEE binary16
 * bit patterns in uint16_t; sizes are int64_t.  Functions return 0 on success.
 */
#ifndef MTORCH_ORACLE_H
#define MTORCH_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 bit conversion: tensor.cpp:276-315 (float_to_half_bits), :317-344 (half_bits_to_float) */
uint16_t orc_f2h(float value);
float orc_h2f(uint16_t bits);
void orc_f2h_array(const float* src, uint16_t* dst, int64_t n);
void orc_h2f_array(const uint16_t* src, float* dst, int64_t n);
/* storage_set_unchecked for fp16 (tensor.cpp:593-597): double -> float (RNE) -> half (half-away) */
uint16_t orc_d2h(double value);

/* ---- RNG: module.cpp:47-183, 245-274, 335-365 */
typedef struct {
  uint64_t state;
  int has_spare_normal;
  double spare_normal;
} orc_rng;

void orc_rng_seed(orc_rng* rng, uint64_t seed);                  /* module.cpp:70-74 */
uint64_t orc_rng_next_u64(orc_rng* rng);                         /* module.cpp:76-82 */
double orc_rng_uniform_open(orc_rng* rng);                       /* module.cpp:84-88 */
void orc_rng_normal_pair(orc_rng* rng, double* first, double* second); /* module.cpp:90-102 */
double orc_rng_next_normal(orc_rng* rng);                        /* module.cpp:104-115 */
/* randn / normal_ on a contiguous fp32 tensor: fill_random_normal_contiguous module.cpp:117-144 */
void orc_fill_normal_f32(orc_rng* rng, float* dst, int64_t n, double mean, double std);
/* randn / normal_ on fp16: per element set_at_linear(mean + std*next_normal) module.cpp:173-177, 270-272 */
void orc_fill_normal_f16(orc_rng* rng, uint16_t* dst, int64_t n, double mean, double std);
/* uniform_ on fp32: fill_random_uniform_contiguous module.cpp:146-157 */
void orc_fill_uniform_f32(orc_rng* rng, float* dst, int64_t n, double from, double to);
/* uniform_ on fp16: set_at_linear(from + (to-from)*U) module.cpp:361-364 */
void orc_fill_uniform_f16(orc_rng* rng, uint16_t* dst, int64_t n, double from, double to);

/* ---- dtype codes shared with the device library: F16=0, F32=1 (tensor.h:13-20 order) */
enum { ORC_F16 = 0, ORC_F32 = 1 };

/* ---- linear: tensor.cpp:31653-31672.  y[M,N] = x[M,K] . w[N,K]^T (+ b[N]); double accumulate.
 * bias may be NULL. */
int orc_linear(int dtype, const void* x, const void* w, const void* b, void* y,
               int64_t M, int64_t N, int64_t K);

/* ---- matmul 2-D / batched (same-dtype operands): tensor.cpp:24983-24996 (fp32),
 * :25049-25063 (fp16, double accum k-outer), batched_matmul :24822-24845.
 * a[batch,M,K] . b[batch,K,N] -> c[batch,M,N]; a_bstride/b_bstride are 0 to broadcast. */
int orc_matmul(int dtype, const void* a, const void* b, void* c, int64_t batch,
               int64_t M, int64_t N, int64_t K, int64_t a_bstride, int64_t b_bstride);

/* ---- addmm: tensor.cpp:25253-25258 then :25320-25334.
 * out = narrow(narrow(beta*in_bcast) + alpha*sum); `in` given as a dense [M,N] expansion. */
int orc_addmm(int dtype, const void* in_mn, const void* a, const void* b, void* out,
              int64_t M, int64_t N, int64_t K, double beta, double alpha);

/* ---- conv2d NCHW, groups: fp32 generic tensor.cpp:27359-27400; fp16 branches :26561-27194.
 * x[B,C,H,W], w[O,C/groups,KH,KW], b[O] or NULL -> y[B,O,OH,OW]. */
int orc_conv2d(int dtype, const void* x, const void* w, const void* b, void* y,
               int64_t B, int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW,
               int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
               int64_t dil_h, int64_t dil_w, int64_t groups);
int64_t orc_conv2d_out_size(int64_t in, int64_t k, int64_t stride, int64_t pad, int64_t dil);

/* ---- scaled_dot_product_attention: generic path tensor.cpp:31158-31207; fp16 casts :30969-30982.
 * q[P,Lq,E], k[P,Lk,E], v[P,Lk,Ev] -> o[P,Lq,Ev].  mask_kind: 0 none, 1 bool (uint8), 2 additive
 * (float32); the mask is a dense [P,Lq,Lk] expansion.  has_scale = 0 selects 1/sqrt(E) (the
 * reference's scale=None); otherwise scale multiplies the scores as given, zero and negative too. */
int orc_sdpa(int dtype, const void* q, const void* k, const void* v, void* o,
             int64_t P, int64_t Lq, int64_t Lk, int64_t E, int64_t Ev,
             int mask_kind, const void* mask, int is_causal, int has_scale, double scale);

/* ---- group_norm on contiguous input: fp32 tensor.cpp:18797-18841; fp16 :18734-18783.
 * x[B, C, inner]; weight/bias [C] or NULL. */
int orc_group_norm(int dtype, const void* x, const void* weight, const void* bias, void* y,
                   int64_t B, int64_t C, int64_t inner, int64_t groups, double eps);

/* ---- layer_norm over the trailing N elements: fp32 one-pass tensor.cpp:17575-17604;
 * fp16 two-pass :17531-17562.  weight/bias [N] or NULL. */
int orc_layer_norm(int dtype, const void* x, const void* weight, const void* bias, void* y,
                   int64_t rows, int64_t N, double eps);

/* ---- softmax over the last dim of a contiguous tensor of rank `rank`:
 * fp32 rank>2 tensor.cpp:7540-7590 (multiply by 1/total); fp32 rank 2 dim 1 :7690-7711 and
 * rank 1 :7517-7539 (divide); fp16 :7743-7802 (multiply by 1/total). */
int orc_softmax_lastdim(int dtype, const void* x, void* y, int64_t rows, int64_t cols, int rank);

/* ---- softmax with an output dtype other than the input's: the generic double path,
 * tensor.cpp:15165-15207 (e stored at the output dtype, divided by the double total). */
int orc_softmax_generic(int in_dtype, const void* x, int out_dtype, void* y, int64_t rows, int64_t cols);

/* ---- gelu: fp32 contiguous tensor.cpp:17254-17273 (+ :17132-17154); fp16 :17225-17235.
 * approximate: 0 = "none" (erf), 1 = "tanh". */
int orc_gelu(int dtype, const void* x, void* y, int64_t n, int approximate);
float orc_fast_erf_float(float value);            /* tensor.cpp:17132-17144 */
float orc_gelu_unit_polynomial_float(float x);    /* tensor.cpp:17146-17154 */

/* ---- silu: fp32 tensor.cpp:16586-16590; fp16 :16482-16541 */
int orc_silu(int dtype, const void* x, void* y, int64_t n);

/* ---- elementwise add/mul on same-shape operands (op 0 add, 1 mul, 2 sub):
 * fp32 float op (tensor.cpp:5465-5481 and siblings); fp16 f2h(h2f(a) op h2f(b)) :5838-5895, :6251-6273.
 * Broadcasting is expanded by the caller (the double path :19077-19084 rounds the same way). */
int orc_binary(int dtype, int op, const void* a, const void* b, void* y, int64_t n);

/* ---- dtype cast fp32 <-> fp16 (tensor.cpp:2642-2649, 2764-2796) */
void orc_cast_f32_to_f16(const float* x, uint16_t* y, int64_t n);
void orc_cast_f16_to_f32(const uint16_t* x, float* y, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
