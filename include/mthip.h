/*
 * libmthip -- MI355X (gfx950) device backend for mtorch's SD-UNet dense-inference hot path.
 *
 * Plain C ABI: raw device pointers, int64 sizes/strides, dtype codes, scalars.  No C++ or
 * framework types cross it, so mtorch's C++ core (a dispatch hook at the top of each public
 * op), its CPython binding, ctypes or any other FFI can bind it directly.
 *
 * Every function returns 0 (MTHIP_OK) on success or a non-zero status; the message of the
 * last failure on the calling thread is returned by mthip_last_error().  Kernels are
 * enqueued asynchronously on one in-order HIP stream per device (mthip_stream); device-to-host
 * copies and mthip_synchronize wait for it.
 *
 * Citations are file:line into kazhiramatsu/mtorch; each names the reference interface the
 * entry point serves when a tensor lives on the GPU device.
 */
#ifndef MTHIP_H
#define MTHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: the order of mtorch::ScalarType (tensor.h:13-20). */
enum {
  MTHIP_F16 = 0,
  MTHIP_F32 = 1,
  MTHIP_F64 = 2,
  MTHIP_I32 = 3,
  MTHIP_I64 = 4,
  MTHIP_BOOL = 5
};

/* status codes */
enum {
  MTHIP_OK = 0,
  MTHIP_ERR_INVALID = 1,     /* bad argument, shape or dtype (caller bug) */
  MTHIP_ERR_HIP = 2,         /* a HIP runtime call failed */
  MTHIP_ERR_OOM = 3,         /* device allocation failed */
  MTHIP_ERR_UNSUPPORTED = 4  /* valid request this backend does not implement */
};

/* ===================================================================== runtime */

/* Thread-local message of the last failure ("" if none). */
const char* mthip_last_error(void);
/* Library build identifier (offload arch and version). */
const char* mthip_version(void);

/* Number of visible GPUs.  Backs mtorch.cuda.is_available/device_count, which the reference
 * stubs to False/0 (mtorch/__init__.py:2320-2321). */
int mthip_device_count(int* count);
/* Name and compute-unit count of a device (for reports). */
int mthip_device_info(int device, char* name, size_t name_len, int* cu_count, size_t* total_mem);

/* ---- memory: the device Allocator seam planned at docs/design/08-phase5-device-layer.md:660-695
 * (allocate / deallocate / copy_from_host / copy_to_host / copy_on_device).  Storage for a GPU
 * tensor (tensor.h:60-85 gains a device buffer) is obtained here.  Blocks are cached per device
 * and reused by size; MTHIP_DISABLE_CACHING=1 in the environment frees eagerly. */
int mthip_malloc(int device, size_t nbytes, void** ptr);
int mthip_free(int device, void* ptr);
int mthip_empty_cache(int device);
int mthip_memory_stats(int device, size_t* allocated_bytes, size_t* reserved_bytes);

/* Host<->device copies behind mtorch::to(input, dtype, device) (tensor.cpp:8479-8508) and
 * Tensor.cpu() (module.cpp:9257).  h2d returns once the host buffer may be reused; d2h
 * returns once the data is on the host. */
int mthip_memcpy_h2d(int device, void* dst, const void* src, size_t nbytes);
int mthip_memcpy_d2h(int device, void* dst, const void* src, size_t nbytes);
int mthip_memcpy_d2d(int device, void* dst, const void* src, size_t nbytes);
int mthip_synchronize(int device);
/* The device's stream as an opaque hipStream_t. */
void* mthip_stream(int device);

/* ---- stream capture into a replayable HIP graph (launch-bound inner loops).  While a
 * capture is open, freed blocks stay reserved for the graph until mthip_graph_destroy. */
int mthip_graph_begin(int device);
int mthip_graph_end(int device, void** graph);
int mthip_graph_launch(int device, void* graph);
int mthip_graph_destroy(int device, void* graph);

/* ---- events on the device stream, for timing. */
int mthip_event_create(void** event);
int mthip_event_record(int device, void* event);
int mthip_event_elapsed_ms(void* start, void* end, float* ms);
int mthip_event_destroy(void* event);

/* ===================================================================== data movement */

/* dtype conversion of n contiguous elements (F16/F32/F64/I32/I64/BOOL).  fp32->fp16 follows
 * float_to_half_bits (tensor.cpp:276-315, half-away-from-zero); fp64->fp16 narrows to fp32
 * first as storage_set_unchecked does (tensor.cpp:593-597).  Serves mtorch::to with a dtype
 * change (tensor.cpp:8479-8508, try_dense_cast :2764-2796, cast_dense_numeric_to_half :2642). */
int mthip_cast(int device, int src_dtype, const void* src, int dst_dtype, void* dst, int64_t n);

/* dst (contiguous, dtype) <- src viewed through sizes/strides (element units), rank <= 8.
 * Serves Tensor::contiguous() (tensor.cpp:8210-8226) for permuted/transposed/sliced views. */
int mthip_copy_strided(int device, int dtype, const void* src, int rank, const int64_t* sizes,
                       const int64_t* src_strides, void* dst);

/* dst viewed through dst_strides <- src viewed through src_strides (element units, same sizes,
 * rank <= 8, 0 strides broadcast the source).  The two views must not overlap.  Serves copy_ and
 * item assignment into a non-contiguous view (Tensor::copy_from, tensor.cpp:8292-8340;
 * Tensor.__setitem__ with a tensor value). */
int mthip_copy_strided_to(int device, int dtype, const void* src, const int64_t* src_strides, int rank,
                          const int64_t* sizes, void* dst, const int64_t* dst_strides);

/* dst[i] = value for n contiguous elements.  Serves full/zeros/ones/fill_ (tensor.h:143-149). */
int mthip_fill(int device, int dtype, void* dst, int64_t n, double value);

/* dst viewed through sizes/strides (element units), rank <= 8 <- value, narrowed as mthip_fill
 * narrows it.  Serves item assignment of a scalar into a non-contiguous view
 * (Tensor.__setitem__, mtorch/__init__.py Tensor.__setitem__ -> Tensor::fill_ on the view). */
int mthip_fill_strided(int device, int dtype, void* dst, int rank, const int64_t* sizes, const int64_t* strides,
                       double value);

/* out (contiguous, out_sizes, dtype) = mask != 0 ? value : x; x and the BOOL mask viewed through
 * strides (0 on broadcast axes), rank <= 8; value narrowed once as mthip_fill narrows it.
 * Serves masked_fill (tensor.cpp:13497-13610). */
int mthip_masked_fill(int device, int dtype, const void* x, const int64_t* x_strides, const void* mask,
                      const int64_t* mask_strides, double value, void* out, int rank, const int64_t* out_sizes);

/* y = !x over n contiguous BOOL bytes (nonzero is true).  Serves logical_not (tensor.cpp:14616)
 * and ~ on bool tensors. */
int mthip_logical_not(int device, const void* x, void* y, int64_t n);

/* Concatenation of `count` contiguous inputs along `dim` of an output of rank `rank` and
 * shape out_sizes (each input shares every other extent).  Serves mtorch::cat (tensor.cpp:32141). */
int mthip_cat(int device, int dtype, int count, const void* const* inputs, const int64_t* dim_sizes,
              int rank, const int64_t* out_sizes, int dim, void* out);

/* The SD timestep embedding [cos(t f), sin(t f)] of fp32 timesteps t[B] and frequencies
 * f[half], narrowed to fp16 out[B][2*half]: the reference benchmark's embedding
 * (tests/compat/benchmarking.py:6031-6032: a broadcast multiply, cos, sin and cat, tensor.cpp:32141)
 * followed by .half() (tensor.cpp:8479-8508) in one launch, each value computed as those ops
 * compute it on the device (fp32 product, sin/cos evaluated in double, the mtorch narrowing). */
int mthip_timestep_embedding_f16(int device, const void* t, const void* freqs, void* out, int64_t B,
                                 int64_t half);

/* Nearest-neighbour 2-D upsampling of x[B*C, H, W] by integer factors.  Serves
 * interpolate(mode="nearest") (tensor.cpp:10897) on the UNet decoder path. */
int mthip_upsample_nearest2d(int device, int dtype, const void* x, void* y, int64_t planes,
                             int64_t H, int64_t W, int64_t scale_h, int64_t scale_w);

/* ===================================================================== elementwise */

enum { MTHIP_BIN_ADD = 0, MTHIP_BIN_MUL = 1, MTHIP_BIN_SUB = 2, MTHIP_BIN_DIV = 3 };

/* out = a (op) b with broadcasting expressed through strides (0 on broadcast axes), rank <= 8,
 * out contiguous with shape out_sizes.  a, b and out share `dtype` (F16 or F32); the op is
 * evaluated in fp32 and narrowed once (fp16: float_to_half_bits).  Serves
 * binary_tensor_tensor (tensor.cpp:18965-19104) for add/sub/mul/div. */
int mthip_binary(int device, int op, int dtype, const void* a, const int64_t* a_strides,
                 const void* b, const int64_t* b_strides, void* out, int rank,
                 const int64_t* out_sizes);

/* out = x (op) scalar for n contiguous elements; scalar_first swaps the operands.
 * Serves binary_tensor_scalar (tensor.cpp:19106-19176). */
int mthip_binary_scalar(int device, int op, int dtype, const void* x, double scalar, int scalar_first,
                        void* out, int64_t n);

enum {
  MTHIP_UNARY_SILU = 0,      /* silu       tensor.cpp:16480-16613 */
  MTHIP_UNARY_GELU = 1,      /* gelu none  tensor.cpp:17207-17288 */
  MTHIP_UNARY_GELU_TANH = 2, /* gelu tanh  tensor.cpp:17275-17279 */
  MTHIP_UNARY_EXP = 3,
  MTHIP_UNARY_SIN = 4,
  MTHIP_UNARY_COS = 5,
  MTHIP_UNARY_NEG = 6,
  MTHIP_UNARY_SIGMOID = 7,
  MTHIP_UNARY_RELU = 8
};
/* y = f(x) for n contiguous elements (F16/F32). */
int mthip_unary(int device, int op, int dtype, const void* x, void* y, int64_t n);

/* GEGLU gating on a [rows, 2*D] tensor: y[r, d] = x[r, d] * gelu(x[r, D + d]) -- the
 * `chunk(2, -1)` + gelu + mul of the SD feed-forward, evaluated with the same per-op roundings
 * (gelu result narrowed, then the product narrowed). */
int mthip_geglu(int device, int dtype, const void* x, void* y, int64_t rows, int64_t D);

/* ===================================================================== contractions */

enum {
  MTHIP_ACT_NONE = 0,
  MTHIP_ACT_GELU = 1,
  MTHIP_ACT_GELU_TANH = 2,
  MTHIP_ACT_SILU = 3
};

/* y[M,N] = act(x[M,K] . w[N,K]^T + b[N]) (+ residual[M,N]) -- mtorch::linear
 * (tensor.cpp:31401-31694; binding py_linear module.cpp:6778-6804) with optional fused
 * activation and residual.  Fusions apply each op's own narrowing in order (linear result
 * narrowed to dtype, then the activation's, then the residual sum's), so a fused call equals
 * the unfused op sequence.  lda/ldw/ldy are row strides in elements; b, residual may be NULL.
 * x, w, b, y, residual share dtype (F16: fp16 MFMA, fp32 accumulate; F32: fp32 MFMA). */
int mthip_linear(int device, int dtype, const void* x, int64_t lda, const void* w, int64_t ldw,
                 const void* b, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int act,
                 const void* residual, int64_t ld_res);

/* Batched GEMM: c[bt] = alpha * a[bt] . op(b[bt]) (+ beta * c_in), op(b) = b (b_trans=0,
 * b is [K,N]) or b^T (b_trans=1, b is [N,K]).  Strides in elements; batch strides may be 0
 * to broadcast.  c_in (may be NULL) is read with its own strides (broadcast allowed) and is
 * narrowed as narrow(beta*c_in) before alpha*product is added, as addmm does
 * (tensor.cpp:25253-25258, 25320-25334); it is read at beta = 0 too (0 * inf gives NaN there),
 * and alpha = 0 skips the product, as the reference's loops do (tensor.cpp:25320, 25621).
 * Serves matmul (tensor.cpp:24896-25064),
 * batched_matmul (:24822-24894), bmm (:25066) and addmm (:25184-25366). */
/* The SD feed-forward's GEGLU input projection in one GEMM: for h = x . W^T + b with
 * W = [W_value; W_gate] ([2N, K]), y[M, N] = h[:, :N] * gelu(h[:, N:]) -- the reference's
 * linear (tensor.cpp:31401) -> chunk(2, -1) (:12519) -> gelu (:17207) -> mul (:18965)
 * sequence, each intermediate narrowed as it narrows them.  w/b must be given with their rows
 * interleaved in 32-row blocks: rows [64q, 64q+32) = W_value[32q, 32q+32) and rows
 * [64q+32, 64q+64) = W_gate[32q, 32q+32) (b likewise; N a multiple of 32); b may be NULL.
 * x, w 16-byte aligned, K a multiple of 8 (F16) / 4 (F32) elements. */
int mthip_linear_geglu(int device, int dtype, const void* x, int64_t lda, const void* w, const void* b,
                       void* y, int64_t ldy, int64_t M, int64_t N, int64_t K);

int mthip_gemm(int device, int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
               const void* a, int64_t lda, int64_t stride_a,
               const void* b, int64_t ldb, int64_t stride_b, int b_trans,
               void* c, int64_t ldc, int64_t stride_c,
               double alpha, double beta, const void* c_in, int64_t c_in_rs, int64_t c_in_cs,
               int64_t stride_c_in);

/* y[B,O,OH,OW] = conv2d(x[B,C,H,W], w[O,C/groups,KH,KW]) + b[O] (+ residual[B,O,OH,OW]),
 * NCHW contiguous in and out -- mtorch::conv2d (tensor.cpp:26490-27528; py_conv2d
 * module.cpp:6912-6961).  groups == 1 runs as an implicit GEMM on MFMA (fp16: fp32
 * accumulate); the residual, when given, is added after the conv result is narrowed.
 * Staging buffers come from the library's caching allocator. */
int mthip_conv2d(int device, int dtype, const void* x, const void* w, const void* b, void* y,
                 int64_t B, int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW,
                 int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                 int64_t dil_h, int64_t dil_w, int64_t groups, const void* residual);

/* Packed conv weight for the groups == 1 implicit GEMM: wp[O][KH][KW][Cp], Cp = C rounded up
 * to 8 (F16) or 4 (F32) channels, zero filled.  The packed copy plays the role of the
 * reference's per-Storage weight caches (tensor.h:65-78, filled by the CPU conv/linear fast
 * paths): the caller keeps it while the weight storage's version is unchanged and passes it
 * to mthip_conv2d_prepacked, which then skips the per-call repack.
 * mthip_conv2d_packed_bytes returns the size of wp in bytes (-1 for a bad dtype). */
int64_t mthip_conv2d_packed_bytes(int dtype, int64_t O, int64_t C, int64_t KH, int64_t KW);
int mthip_conv2d_pack_weight(int device, int dtype, const void* w, void* wp,
                             int64_t O, int64_t C, int64_t KH, int64_t KW);
/* mthip_conv2d (groups == 1) with a weight packed by mthip_conv2d_pack_weight. */
int mthip_conv2d_prepacked(int device, int dtype, const void* x, const void* wp, const void* b, void* y,
                           int64_t B, int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW,
                           int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                           int64_t dil_h, int64_t dil_w, const void* residual);
/* Nearest 2x upsampling of NCHW x[B][C][H][W] written channels-last with Cp >= C channels
 * (padding channels zero), xp[B][2H*2W][Cp]: interpolate(scale_factor=2, mode="nearest")
 * (tensor.cpp:10897) and the layout change ahead of mthip_conv2d_nhwc in one pass -- the SD
 * decoder's Upsample block (upsample, then conv2d 3x3, tensor.cpp:26490). */
int mthip_upsample2x_to_nhwc(int device, int dtype, const void* x, void* xp, int64_t B, int64_t C,
                             int64_t Cp, int64_t H, int64_t W);

/* The same conv with the input already channels-last: x_nhwc[B][H][W][Cp] (Cp as for the
 * packed weight, channels C..Cp-1 zero), e.g. as written by mthip_group_norm_nhwc; the output
 * (and residual) stay NCHW.  This is the GroupNorm -> SiLU -> conv hand-off of every SD ResNet
 * block: the normalised activation is written once, in the layout the conv reads, instead of
 * NCHW plus a transposing copy.  chan_add (optional, NULL for none) adds
 * chan_add[b * chan_add_ld + o] to every pixel of output plane (b, o) after the bias and before
 * the residual -- the `h + t[:, :, None, None]` time-embedding add of an SD ResNet block
 * (binary add, tensor.cpp:18965), narrowed as that separate add narrows.  Launches only the GEMM. */
int mthip_conv2d_nhwc(int device, int dtype, const void* x_nhwc, const void* wp, const void* b, void* y,
                      int64_t B, int64_t C, int64_t H, int64_t W, int64_t O, int64_t KH, int64_t KW,
                      int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                      int64_t dil_h, int64_t dil_w, const void* residual, const void* chan_add,
                      int64_t chan_add_ld);

/* ===================================================================== attention */

enum { MTHIP_MASK_NONE = 0, MTHIP_MASK_BOOL = 1, MTHIP_MASK_ADD = 2 };

/* o = softmax(q k^T * scale + mask) v over heads -- mtorch::scaled_dot_product_attention
 * (tensor.cpp:30930-31324; py_scaled_dot_product_attention module.cpp:7407-7459).
 * Layout: q[B,H,Lq,E], k[B,Hk,Lk,E], v[B,Hk,Lk,Ev] addressed by element strides
 * (qs/ks/vs = {batch, head, seq}; the last dim is contiguous); o likewise through os (NULL:
 * contiguous [B,H,Lq,Ev]) -- e.g. {Lq*H*Ev, Ev, H*Ev} writes the heads merged back into a
 * [B, Lq, H*Ev] token tensor, the layout the output projection reads.
 * Hk divides H (H/Hk query heads share a key head: enable_gqa).  mask: MTHIP_MASK_BOOL
 * (uint8, false -> -inf) or MTHIP_MASK_ADD (mask_dtype F32 or the query dtype, added to the
 * scaled score), read through 4 strides {b, h, q, k} with 0 on broadcast axes.  is_causal
 * masks keys after the query.  has_scale = 0 selects 1/sqrt(E) (the reference's scale=None,
 * tensor.cpp:31019); otherwise scale multiplies every score as given -- zero (softmax of the mask
 * alone: the mean of V over the unmasked keys) and negative values included.  q/k/v/o share
 * dtype F16 (fp16 MFMA, fp32 softmax) or F32.  Fully-masked rows give NaN, as the reference
 * does. */
int mthip_sdpa(int device, int dtype, const void* q, const int64_t* qs, const void* k,
               const int64_t* ks, const void* v, const int64_t* vs, void* o, const int64_t* os,
               int64_t B, int64_t H, int64_t Hk, int64_t Lq, int64_t Lk, int64_t E, int64_t Ev, int mask_kind,
               int mask_dtype, const void* mask, const int64_t* mask_strides, int is_causal,
               int has_scale, double scale);

/* ===================================================================== normalisation */

/* group_norm on contiguous x[B, C, inner] (tensor.cpp:18643-18963; py_group_norm
 * module.cpp:7646-7693); weight/bias [C] or NULL.  fuse_silu != 0 applies silu to the
 * narrowed result (the GroupNorm->SiLU pair of every SD ResBlock) with silu's own rounding.
 * param_dtype is the dtype of weight/bias and of the computation: equal to dtype, or F32 with
 * F16 data -- the upcast pattern group_norm(x.float(), w32, b32).half() of SD pipelines, run as
 * the reference's fp32 path (tensor.cpp:18797-18841) narrowed once. */
int mthip_group_norm(int device, int dtype, const void* x, const void* weight, const void* bias,
                     void* y, int64_t B, int64_t C, int64_t inner, int64_t groups, double eps,
                     int fuse_silu, int param_dtype);
/* mthip_group_norm without any device allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Arguments and results are mthip_group_norm's, bit for bit;
 * the statistics partials live in a static 1 MiB device array per GPU instead of a block from
 * the caching allocator, so B * groups * ceil(group_size / chunk) must stay <= 131072 (at most
 * 64 chunks of >= 2048 elements per group; an error status otherwise).  Calls that overlap on one
 * GPU (other streams, other host threads) share the array and race. */
int mthip_group_norm_noalloc(int device, int dtype, const void* x, const void* weight, const void* bias,
                             void* y, int64_t B, int64_t C, int64_t inner, int64_t groups, double eps,
                             int fuse_silu, int param_dtype);
/* The same values written channels-last for mthip_conv2d_nhwc: y_nhwc[B][HW][Cp], Cp = C
 * rounded up to 8 (F16) or 4 (F32) channels, the padding channels zero.  x stays NCHW. */
int mthip_group_norm_nhwc(int device, int dtype, const void* x, const void* weight, const void* bias,
                          void* y_nhwc, int64_t B, int64_t C, int64_t HW, int64_t groups, double eps,
                          int fuse_silu, int param_dtype);

/* group_norm(cat([x0, x1], dim=1)) written channels-last as mthip_group_norm_nhwc writes it,
 * reading the two NCHW inputs x0[B][C0][HW] and x1[B][C1][HW] in place instead of a
 * concatenated copy (mtorch's torch.cat, tensor.cpp:32141, followed by group_norm,
 * tensor.cpp:18643-18963: the input of every SD up-block ResBlock).  raw_nhwc (NULL to skip)
 * receives the concatenated input itself channels-last, [B][HW][C0+C1] -- the operand of the
 * block's 1x1 shortcut conv (mthip_conv2d_nhwc).  F16 data only; C0+C1 and HW multiples of 8,
 * C0 even; y_nhwc and raw_nhwc have C0+C1 channels (no padding). */
int mthip_group_norm_nhwc_cat(int device, int dtype, const void* x0, int64_t C0, const void* x1,
                              int64_t C1, const void* weight, const void* bias, void* y_nhwc,
                              void* raw_nhwc, int64_t B, int64_t HW, int64_t groups, double eps,
                              int fuse_silu, int param_dtype);

/* layer_norm over the trailing N elements of contiguous x[rows, N] (tensor.cpp:17386-17708;
 * py_layer_norm module.cpp:7461-7516); weight/bias [N] or NULL.  fp16 uses the two-pass
 * centred variance, fp32 the one-pass form, as the reference does.  param_dtype as for
 * mthip_group_norm (F32 over F16 data: layer_norm(x.float(), w32, b32).half()). */
int mthip_layer_norm(int device, int dtype, const void* x, const void* weight, const void* bias,
                     void* y, int64_t rows, int64_t N, double eps, int param_dtype);

/* softmax over the last dim of contiguous x[rows, cols] (tensor.cpp:15145-15221,
 * try_softmax_float32_kernel :7508-7741, try_softmax_float16_kernel :7743-7802).
 * divide != 0 divides by the row total (fp32 rank<=2), else multiplies by its reciprocal. */
int mthip_softmax_lastdim(int device, int dtype, const void* x, void* y, int64_t rows,
                          int64_t cols, int divide);

/* ===================================================================== RNG (host) */

/* mtorch's generator: splitmix64 + Marsaglia polar normals with a spare-normal cache
 * (module.cpp:47-183, 245-274, 335-365).  A generator is an opaque host object; fills write
 * host buffers of `dtype` (F16/F32) exactly as the reference's randn/normal_/uniform_ do. */
void* mthip_generator_create(uint64_t seed);
void mthip_generator_destroy(void* gen);
int mthip_generator_seed(void* gen, uint64_t seed);           /* manual_seed module.cpp:2626 */
int mthip_generator_get_state(void* gen, uint64_t* state, int* has_spare, double* spare);
int mthip_generator_set_state(void* gen, uint64_t state, int has_spare, double spare);
int mthip_rng_normal(void* gen, int dtype, void* host_dst, int64_t n, double mean, double std);
int mthip_rng_uniform(void* gen, int dtype, void* host_dst, int64_t n, double from, double to);

#ifdef __cplusplus
}
#endif
#endif /* MTHIP_H */
