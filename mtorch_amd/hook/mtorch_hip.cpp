// GPU backend entry points for mtorch's C++ core over libmthip (declarations and the hook
// convention in mtorch_hip.h).  Built inside kazhiramatsu/mtorch with
//   -I cpp -I <this repository>/include   and linked with   -lmthip.
//
// Argument checks repeat the reference op's own checks and messages (cited per function), so a
// caller sees the same exceptions on either device; the GPU work itself is one or a few libmthip
// calls.  Every op returns a new contiguous GPU tensor; views of GPU tensors made by the
// reference's metadata ops (transpose, permute, slicing, expand) are accepted anywhere through
// their strides.
#include "mtorch_hip.h"

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <stdexcept>
#include <tuple>
#include <utility>

#include "mthip.h"

namespace mtorch::hip {
namespace {

// libmthip dtype codes follow ScalarType's order (tensor.h:13-20).
int code(ScalarType dtype) { return static_cast<int>(dtype); }

void check(int status) {
  if (status == MTHIP_OK) return;
  std::string message = std::string("mtorch: ") + mthip_last_error();
  if (status == MTHIP_ERR_INVALID) throw std::invalid_argument(message);
  throw std::runtime_error(message);
}

std::string type_name(DeviceType type) { return type == kGpu ? "cuda" : device_type_name(type); }

// The fixed message of the reference's dispatch hooks (docs/design/08-phase5-device-layer.md
// section 4, rule 4).
[[noreturn]] void unsupported(const std::string& op, DeviceType type) {
  throw std::runtime_error("mtorch: operator '" + op + "' is not implemented for device '" + type_name(type) +
                           "'");
}

int64_t product(const std::vector<int64_t>& values) {
  int64_t n = 1;
  for (int64_t v : values) n *= v;
  return n;
}

// A GPU buffer behind the reference's Storage.  Storage's constructor builds only CPU storages
// (require_cpu_device, tensor.cpp:8071-8074), so the base is built empty on the CPU and then
// re-tagged; `bytes` stays empty, as the device plan specifies for non-CPU storages.  A
// shared_ptr<Storage> made from make_shared<GpuStorage> keeps GpuStorage's destructor.
struct GpuStorage final : Storage {
  void* data = nullptr;
  size_t nbytes = 0;
  // Packed conv weights (mthip_conv2d_pack_weight) keyed by (offset, O, C, KH, KW) and tagged
  // with the storage version, so an in-place write to the weight repacks it: the role of the
  // half_conv2d_nhwc_weight_cache fields of tensor.h:67-78.
  struct Pack {
    uint64_t version;
    void* data;
  };
  std::map<std::tuple<int64_t, int64_t, int64_t, int64_t, int64_t>, Pack> packs;
  std::mutex packs_mutex;

  GpuStorage(ScalarType dtype_, int64_t elements, int64_t index) : Storage(dtype_, 0, cpu_device(), false) {
    device = Device{kGpu, index};
    nbytes = static_cast<size_t>(elements) * static_cast<size_t>(element_size(dtype_));
    if (nbytes != 0) check(mthip_malloc(static_cast<int>(index), nbytes, &data));
  }
  ~GpuStorage() {
    for (auto& entry : packs) mthip_free(static_cast<int>(device.index), entry.second.data);
    if (data != nullptr) mthip_free(static_cast<int>(device.index), data);
  }
  GpuStorage(const GpuStorage&) = delete;
  GpuStorage& operator=(const GpuStorage&) = delete;
};

GpuStorage& gpu_storage(const Tensor& t) { return static_cast<GpuStorage&>(*t.storage); }
void* data(const Tensor& t) {
  return static_cast<char*>(gpu_storage(t).data) + t.offset * element_size(t.dtype);
}
const void* data_or_null(const TensorPtr& t) { return t ? data(*t) : nullptr; }
int index_of(const Tensor& t) { return static_cast<int>(t.device.index); }

TensorPtr view(const TensorPtr& base, std::vector<int64_t> sizes, std::vector<int64_t> strides, int64_t offset) {
  return std::make_shared<Tensor>(base->storage, std::move(sizes), std::move(strides), offset, base->dtype, false);
}

// Row-major dense (size-1 dimensions may carry any stride).
bool dense(const Tensor& t) {
  int64_t expect = 1;
  for (int64_t d = t.dim() - 1; d >= 0; --d) {
    const int64_t size = t.sizes[static_cast<size_t>(d)];
    if (size == 1) continue;
    if (t.strides[static_cast<size_t>(d)] != expect) return false;
    expect *= size;
  }
  return true;
}

// Guards every entry point runs first: all operands on one GPU (ensure_same_device,
// tensor.cpp:265-268), none tracked by autograd (guard G1 of the CUDA plan,
// docs/design/10-phase7-cuda-backend.md:328-330).  Returns the device index.
int guard(const std::string& op, std::initializer_list<TensorPtr> operands) {
  const Tensor* first = nullptr;
  for (const TensorPtr& t : operands) {
    if (!t) continue;
    if (first != nullptr && !devices_equal(first->device, t->device)) {
      throw std::invalid_argument("tensor devices must match");
    }
    if (first == nullptr) first = t.get();
  }
  if (first == nullptr || first->device.type != kGpu) unsupported(op, first ? first->device.type : DeviceType::CPU);
  if (is_grad_enabled()) {
    for (const TensorPtr& t : operands) {
      if (t && t->requires_grad) {
        throw std::runtime_error("mtorch: operator '" + op +
                                 "' is not implemented for device 'cuda' with autograd; run inference under "
                                 "mtorch.no_grad()");
      }
    }
  }
  return index_of(*first);
}

// The float16/float32 allowlist of the contraction, norm and attention families (G5,
// docs/design/10-phase7-cuda-backend.md:342-355).
void require_float(const std::string& op, ScalarType dtype) {
  if (dtype != ScalarType::Float16 && dtype != ScalarType::Float32) unsupported(op + "[" + dtype_name(dtype) + "]", kGpu);
}

void require_same_dtype(const std::string& what, std::initializer_list<TensorPtr> operands) {
  const Tensor* first = nullptr;
  for (const TensorPtr& t : operands) {
    if (!t) continue;
    if (first != nullptr && t->dtype != first->dtype) {
      throw std::invalid_argument("expected " + what + " to have the same dtype");
    }
    if (first == nullptr) first = t.get();
  }
}

TensorPtr dense_copy(const TensorPtr& t) {
  auto out = empty(t->sizes, t->dtype, t->device);
  if (out->numel() == 0) return out;
  if (dense(*t)) {
    check(mthip_memcpy_d2d(index_of(*t), data(*out), data(*t),
                           static_cast<size_t>(t->numel() * element_size(t->dtype))));
  } else {
    check(mthip_copy_strided(index_of(*t), code(t->dtype), data(*t), static_cast<int>(t->dim()), t->sizes.data(),
                             t->strides.data(), data(*out)));
  }
  return out;
}

TensorPtr as_dense(const TensorPtr& t) { return dense(*t) ? t : dense_copy(t); }

TensorPtr cast(const TensorPtr& t, ScalarType dtype) {
  if (t->dtype == dtype) return t;
  auto src = as_dense(t);
  auto out = empty(t->sizes, dtype, t->device);
  const int64_t n = out->numel();
  if (n != 0) check(mthip_cast(index_of(*t), code(src->dtype), data(*src), code(dtype), data(*out), n));
  return out;
}

// t's strides aligned to `shape` (right-aligned broadcasting), 0 on broadcast axes.
std::vector<int64_t> broadcast_strides(const Tensor& t, const std::vector<int64_t>& shape) {
  const size_t rank = shape.size();
  const size_t pad = rank - t.sizes.size();
  std::vector<int64_t> strides(rank, 0);
  for (size_t i = 0; i < t.sizes.size(); ++i) {
    strides[pad + i] = (t.sizes[i] == 1 && shape[pad + i] != 1) ? 0 : t.strides[i];
  }
  return strides;
}

TensorPtr broadcast_view(const TensorPtr& t, const std::vector<int64_t>& shape) {
  return view(t, shape, broadcast_strides(*t, shape), t->offset);
}

bool broadcasts_to(const std::vector<int64_t>& from, const std::vector<int64_t>& to) {
  if (from.size() > to.size()) return false;
  const size_t pad = to.size() - from.size();
  for (size_t i = 0; i < from.size(); ++i) {
    if (from[i] != 1 && from[i] != to[pad + i]) return false;
  }
  return true;
}

// One element stride for the first nb (batch) dims of t, when they collapse to one.
bool collapse_batch(const Tensor& t, size_t nb, int64_t& stride) {
  int64_t found = 0, expect = 0;
  bool have = false;
  for (size_t i = nb; i-- > 0;) {
    const int64_t size = t.sizes[i], st = t.strides[i];
    if (size == 1) continue;
    if (!have) {
      found = st;
      expect = st * size;
      have = true;
    } else if (st != expect) {
      return false;
    } else {
      expect = st * size;
    }
  }
  stride = have ? found : 0;
  return true;
}

// x[..., K] as M rows of K with one row stride lda, when its layout allows that.
bool rows_view(const Tensor& x, int64_t& M, int64_t& lda) {
  const int64_t K = x.sizes.back();
  if (x.dim() == 1) {
    M = 1;
    lda = K;
    return x.strides[0] == 1 || K <= 1;
  }
  if (x.strides.back() != 1 && K > 1) return false;
  std::vector<int64_t> outer(x.sizes.begin(), x.sizes.end() - 1);
  std::vector<int64_t> outer_strides(x.strides.begin(), x.strides.end() - 1);
  int64_t stride = 0, expect = 0;
  bool have = false;
  for (size_t i = outer.size(); i-- > 0;) {
    if (outer[i] == 1) continue;
    if (!have) {
      stride = outer_strides[i];
      expect = stride * outer[i];
      have = true;
    } else if (outer_strides[i] != expect) {
      return false;
    } else {
      expect = outer_strides[i] * outer[i];
    }
  }
  M = product(outer);
  lda = have ? stride : K;
  return lda >= K;
}

// c[batch, M, N] = alpha * a . b (+ beta * c_in) on [batch?, M, K] / [batch?, K, N] views with
// batch strides sa / sb; a needs unit stride along K, b is used as it lies ([K, N] rows or a
// transposed [N, K]) when either of its inner strides is 1.
void gemm(TensorPtr a, TensorPtr b, const Tensor& out, int64_t batch, int64_t M, int64_t N, int64_t K, int64_t sa,
          int64_t sb, double alpha, double beta, const TensorPtr& c_in, int64_t c_rs, int64_t c_cs, int64_t c_bs) {
  const size_t r = a->sizes.size();
  if (a->strides[r - 1] != 1 && K > 1) {
    a = dense_copy(a);
    sa = sa != 0 ? M * K : 0;
  }
  int64_t lda = M > 1 ? a->strides[r - 2] : K;
  if (lda < K) {
    a = dense_copy(a);
    lda = K;
    sa = sa != 0 ? M * K : 0;
  }
  const size_t rb = b->sizes.size();
  int b_trans = 0;
  int64_t ldb = N;
  if (b->strides[rb - 1] == 1 || N == 1) {
    ldb = K > 1 ? b->strides[rb - 2] : N;
    if (ldb < N) {
      b = dense_copy(b);
      ldb = N;
      sb = sb != 0 ? K * N : 0;
    }
  } else if (b->strides[rb - 2] == 1) {
    b_trans = 1;
    ldb = b->strides[rb - 1];
    if (ldb < K) {
      b = dense_copy(b);
      b_trans = 0;
      ldb = N;
      sb = sb != 0 ? K * N : 0;
    }
  } else {
    b = dense_copy(b);
    ldb = N;
    sb = sb != 0 ? K * N : 0;
  }
  check(mthip_gemm(index_of(out), code(out.dtype), batch, M, N, K, data(*a), lda, sa, data(*b), ldb, sb, b_trans,
                   data(out), N, M * N, alpha, beta, data_or_null(c_in), c_rs, c_cs, c_bs));
}

int binary_code(const std::string& op) {
  if (op == "add") return MTHIP_BIN_ADD;
  if (op == "mul") return MTHIP_BIN_MUL;
  if (op == "sub") return MTHIP_BIN_SUB;
  if (op == "div") return MTHIP_BIN_DIV;
  return -1;
}

TensorPtr scalar_op(const TensorPtr& t, double scalar, const std::string& op, bool scalar_first) {
  const int d = guard(op, {t});
  const int opcode = binary_code(op);
  if (opcode < 0) unsupported(op, kGpu);
  require_float(op, t->dtype);
  auto src = as_dense(t);
  auto out = empty(t->sizes, t->dtype, t->device);
  const int64_t n = out->numel();
  if (n != 0) {
    check(mthip_binary_scalar(d, opcode, code(t->dtype), data(*src), scalar, scalar_first ? 1 : 0, data(*out), n));
  }
  return out;
}

TensorPtr unary(const TensorPtr& t, const std::string& op, int opcode) {
  const int d = guard(op, {t});
  require_float(op, t->dtype);
  auto src = as_dense(t);
  auto out = empty(t->sizes, t->dtype, t->device);
  const int64_t n = out->numel();
  if (n != 0) check(mthip_unary(d, opcode, code(t->dtype), data(*src), data(*out), n));
  return out;
}

// conv2d's (stride, padding, dilation) pairs: normalize_conv2d_pair (tensor.cpp:25901-25920).
std::pair<int64_t, int64_t> conv_pair(const std::vector<int64_t>& value, const char* name, bool allow_zero) {
  int64_t a = 0, b = 0;
  if (value.size() == 1) {
    a = b = value[0];
  } else if (value.size() == 2) {
    a = value[0];
    b = value[1];
  } else {
    throw std::invalid_argument(std::string("conv2d ") + name + " must be an int or a pair");
  }
  for (int64_t item : {a, b}) {
    if (allow_zero ? item < 0 : item <= 0) {
      throw std::invalid_argument(std::string("conv2d ") + name + " has an invalid value");
    }
  }
  return {a, b};
}

const void* packed_conv_weight(const TensorPtr& w, int d, int64_t O, int64_t C, int64_t KH, int64_t KW) {
  GpuStorage& st = gpu_storage(*w);
  std::lock_guard<std::mutex> lock(st.packs_mutex);
  const auto key = std::make_tuple(w->offset, O, C, KH, KW);
  auto hit = st.packs.find(key);
  if (hit != st.packs.end() && hit->second.version == st.version) return hit->second.data;
  const int64_t nbytes = mthip_conv2d_packed_bytes(code(w->dtype), O, C, KH, KW);
  if (nbytes <= 0) throw std::invalid_argument("conv2d weight cannot be packed");
  void* packed = nullptr;
  check(mthip_malloc(d, static_cast<size_t>(nbytes), &packed));
  const int status = mthip_conv2d_pack_weight(d, code(w->dtype), data(*w), packed, O, C, KH, KW);
  if (status != MTHIP_OK) {
    mthip_free(d, packed);
    check(status);
  }
  if (hit != st.packs.end()) {
    mthip_free(d, hit->second.data);
    hit->second = GpuStorage::Pack{st.version, packed};
  } else {
    st.packs.emplace(key, GpuStorage::Pack{st.version, packed});
  }
  return packed;
}

}  // namespace

// ============================================================================ runtime

bool on_gpu(const TensorPtr& t) { return t && t->device.type == kGpu; }

Device gpu_device(int64_t index) { return Device{kGpu, index < 0 ? 0 : index}; }

std::string device_string(const Device& device) {
  const std::string name = type_name(device.type);
  return device.index < 0 ? name : name + ":" + std::to_string(device.index);
}

int64_t device_count() {
  int count = 0;
  check(mthip_device_count(&count));
  return count;
}

void synchronize(const Device& device) { check(mthip_synchronize(static_cast<int>(gpu_device(device.index).index))); }

TensorPtr empty(const std::vector<int64_t>& sizes, ScalarType dtype, const Device& device) {
  if (device.type != kGpu) throw std::invalid_argument("hip::empty expects a GPU device");
  const int64_t index = device.index < 0 ? 0 : device.index;
  std::shared_ptr<Storage> storage = std::make_shared<GpuStorage>(dtype, product(sizes), index);
  return std::make_shared<Tensor>(std::move(storage), sizes, contiguous_strides(sizes), 0, dtype, false);
}

// ============================================================================ data movement

// mtorch::to (tensor.cpp:8479-8508) when either side is a GPU.  Host data is staged through the
// reference's own Tensor::contiguous; dtype conversion runs on the GPU with the reference's
// rounding (mthip_cast).
TensorPtr to(const TensorPtr& input, ScalarType dtype, Device device, bool copy) {
  if (device.type == kGpu) device = gpu_device(device.index);
  const bool from_gpu = input->device.type == kGpu;
  if (!from_gpu && device.type != kGpu) return mtorch::to(input, dtype, device, copy);
  if (input->device.type == DeviceType::Metal || device.type == DeviceType::Metal) {
    throw std::runtime_error("Metal/MPS device execution is not implemented yet");  // require_cpu_device
  }
  if (!from_gpu) {
    auto host = input->contiguous();
    auto staged = empty(input->sizes, input->dtype, device);
    const size_t nbytes = static_cast<size_t>(input->numel() * element_size(input->dtype));
    if (nbytes != 0) {
      const uint8_t* src = host->storage->bytes.data() + host->offset * element_size(host->dtype);
      check(mthip_memcpy_h2d(static_cast<int>(device.index), data(*staged), src, nbytes));
    }
    auto out = cast(staged, dtype);
    out->requires_grad = input->requires_grad;
    return out;
  }
  if (device.type == kGpu) {
    if (device.index != input->device.index) {
      throw std::runtime_error("copies between two GPUs are not supported by this backend");
    }
    if (dtype == input->dtype) return copy ? dense_copy(input) : input;
    return cast(input, dtype);
  }
  auto src = as_dense(cast(input, dtype));
  const int64_t n = input->numel();
  auto storage = std::make_shared<Storage>(dtype, n, cpu_device(), false);
  if (n != 0) {
    check(mthip_memcpy_d2h(index_of(*src), storage->bytes.data(), data(*src),
                           static_cast<size_t>(n * element_size(dtype))));
  }
  return std::make_shared<Tensor>(std::move(storage), input->sizes, contiguous_strides(input->sizes), 0, dtype,
                                  input->requires_grad);
}

TensorPtr contiguous(const TensorPtr& input) {
  guard("contiguous", {input});
  return as_dense(input);
}

// Tensor::copy_from (tensor.cpp:8292-8340): source values, converted to the destination's dtype
// and broadcast to its shape, written through the destination's strides.
void copy_from(const TensorPtr& destination, const TensorPtr& source) {
  if (destination->device.type != kGpu) unsupported("copy_", destination->device.type);
  if (!broadcasts_to(source->sizes, destination->sizes)) {
    throw std::invalid_argument("copy_ source is not broadcastable to the destination shape");
  }
  const int d = index_of(*destination);
  TensorPtr src = source->device.type == kGpu ? source : hip::to(source, source->dtype, destination->device);
  if (src->device.index != destination->device.index) throw std::invalid_argument("tensor devices must match");
  src = cast(src, destination->dtype);
  if (src->storage == destination->storage) src = dense_copy(src);  // overlapping views: stage first
  ++destination->storage->version;
  if (destination->numel() == 0) return;
  const auto src_strides = broadcast_strides(*src, destination->sizes);
  const int rank = static_cast<int>(destination->dim());
  if (rank == 0) {
    check(mthip_memcpy_d2d(d, data(*destination), data(*src), static_cast<size_t>(element_size(src->dtype))));
    return;
  }
  check(mthip_copy_strided_to(d, code(destination->dtype), data(*src), src_strides.data(), rank,
                              destination->sizes.data(), data(*destination), destination->strides.data()));
}

void fill_inplace(const TensorPtr& tensor, double value) {
  const int d = guard("fill_", {tensor});
  ++tensor->storage->version;
  const int64_t n = tensor->numel();
  if (n == 0) return;
  if (dense(*tensor)) {
    check(mthip_fill(d, code(tensor->dtype), data(*tensor), n, value));
  } else {
    check(mthip_fill_strided(d, code(tensor->dtype), data(*tensor), static_cast<int>(tensor->dim()),
                             tensor->sizes.data(), tensor->strides.data(), value));
  }
}

// ============================================================================ elementwise

// binary_tensor_tensor (tensor.cpp:18965-19104) for add/sub/mul/div: promoted dtype, broadcast
// through zero strides, evaluated in fp32 and narrowed once.
TensorPtr binary_tensor_tensor(const TensorPtr& left, const TensorPtr& right, const std::string& op) {
  const int d = guard(op, {left, right});
  const int opcode = binary_code(op);
  if (opcode < 0) unsupported(op, kGpu);
  const ScalarType dtype = promote_dtype(left->dtype, right->dtype);
  require_float(op, dtype);
  auto a = cast(left, dtype);
  auto b = cast(right, dtype);
  std::vector<int64_t> shape = broadcast_shapes({a->sizes, b->sizes});
  auto out = empty(shape, dtype, left->device);
  if (out->numel() == 0) return out;
  std::vector<int64_t> sa = broadcast_strides(*a, shape), sb = broadcast_strides(*b, shape);
  if (shape.empty()) {  // rank-0 operands run as one element of rank 1
    shape = {1};
    sa = {0};
    sb = {0};
  }
  check(mthip_binary(d, opcode, code(dtype), data(*a), sa.data(), data(*b), sb.data(), data(*out),
                     static_cast<int>(shape.size()), shape.data()));
  return out;
}

// binary_tensor_scalar / binary_scalar_tensor (tensor.cpp:19106-19230) on floating tensors: the
// scalar does not change a floating tensor's dtype.
TensorPtr binary_tensor_scalar(const TensorPtr& left, double scalar, ScalarType, const std::string& op) {
  return scalar_op(left, scalar, op, false);
}

TensorPtr binary_scalar_tensor(double scalar, ScalarType, const TensorPtr& right, const std::string& op) {
  return scalar_op(right, scalar, op, true);
}

TensorPtr silu(const TensorPtr& input) { return unary(input, "silu", MTHIP_UNARY_SILU); }  // tensor.cpp:16480

TensorPtr gelu(const TensorPtr& input, const std::string& approximate) {  // tensor.cpp:17207-17288
  if (approximate == "none") return unary(input, "gelu", MTHIP_UNARY_GELU);
  if (approximate == "tanh") return unary(input, "gelu", MTHIP_UNARY_GELU_TANH);
  throw std::invalid_argument("gelu approximate must be 'none' or 'tanh'");
}

// ============================================================================ contractions

// mtorch::linear (tensor.cpp:31401-31694): y = input . weight^T + bias in the promoted dtype;
// input rows are read through their row stride, weight in place unless it is transposed.
TensorPtr linear(const TensorPtr& input, const TensorPtr& weight, const TensorPtr& bias) {
  const int d = guard("linear", {input, weight, bias});
  if (input->dim() < 1 || weight->dim() != 2) {
    throw std::invalid_argument("linear expects an input with at least 1 dimension and a 2-D weight");
  }
  const int64_t K = input->sizes.back();
  const int64_t N = weight->sizes[0];
  if (weight->sizes[1] != K) throw std::invalid_argument("linear input and weight shapes cannot be multiplied");
  ScalarType dtype = promote_dtype(input->dtype, weight->dtype);
  if (bias) dtype = promote_dtype(dtype, bias->dtype);
  std::vector<int64_t> out_shape(input->sizes.begin(), input->sizes.end() - 1);
  out_shape.push_back(N);
  if (bias && !broadcasts_to(bias->sizes, out_shape)) {
    throw std::invalid_argument("linear bias is not broadcastable to the output shape");
  }
  require_float("linear", dtype);
  TensorPtr x = cast(input, dtype), w = cast(weight, dtype), b = bias ? cast(bias, dtype) : nullptr;
  int64_t M = 0, lda = 0;
  if (!rows_view(*x, M, lda)) {
    x = dense_copy(x);
    rows_view(*x, M, lda);
  }
  int64_t ldw = K;
  if (!(w->strides[1] == 1 && (w->strides[0] >= K || N <= 1))) {
    w = dense_copy(w);
  } else if (N > 1) {
    ldw = w->strides[0];
  }
  TensorPtr bias_vector, post_bias;
  if (b) {
    bool leading_ones = true;
    for (size_t i = 0; i + 1 < b->sizes.size(); ++i) leading_ones = leading_ones && b->sizes[i] == 1;
    if (b->numel() == N && leading_ones) {
      bias_vector = as_dense(b);
    } else {
      post_bias = b;
    }
  }
  auto out = empty(out_shape, dtype, input->device);
  if (out->numel() != 0) {
    check(mthip_linear(d, code(dtype), data(*x), lda, data(*w), ldw, data_or_null(bias_vector), data(*out), N, M, N,
                       K, MTHIP_ACT_NONE, nullptr, 0));
  }
  return post_bias ? hip::binary_tensor_tensor(out, post_bias, "add") : out;
}

// mtorch::matmul (tensor.cpp:24896-25064) with batched_matmul's broadcasting (:24822-24894); 1-D
// operands gain and then lose a unit dimension as dot/mv/vector_matmul define them.
TensorPtr matmul(const TensorPtr& left, const TensorPtr& right) {
  guard("matmul", {left, right});
  if (left->dim() == 0 || right->dim() == 0) {
    throw std::invalid_argument("matmul expects both arguments to be at least 1-D");
  }
  const ScalarType dtype = promote_dtype(left->dtype, right->dtype);
  require_float("matmul", dtype);
  TensorPtr a = cast(left, dtype), b = cast(right, dtype);
  const bool squeeze_m = a->dim() == 1, squeeze_n = b->dim() == 1;
  if (squeeze_m) a = view(a, {1, a->sizes[0]}, {a->sizes[0] * a->strides[0], a->strides[0]}, a->offset);
  if (squeeze_n) b = view(b, {b->sizes[0], 1}, {b->strides[0], 1}, b->offset);
  const int64_t M = a->sizes[a->dim() - 2], K = a->sizes[a->dim() - 1];
  const int64_t K2 = b->sizes[b->dim() - 2], N = b->sizes[b->dim() - 1];
  if (K != K2) throw std::invalid_argument("matmul shape mismatch");
  std::vector<int64_t> a_batch(a->sizes.begin(), a->sizes.end() - 2), b_batch(b->sizes.begin(), b->sizes.end() - 2);
  std::vector<int64_t> batch = broadcast_shapes({a_batch, b_batch});
  std::vector<int64_t> out_shape = batch;
  out_shape.push_back(M);
  out_shape.push_back(N);
  auto out = empty(out_shape, dtype, left->device);
  if (out->numel() != 0) {
    std::vector<int64_t> a_shape = batch, b_shape = batch;
    a_shape.insert(a_shape.end(), {M, K});
    b_shape.insert(b_shape.end(), {K, N});
    TensorPtr ae = broadcast_view(a, a_shape), be = broadcast_view(b, b_shape);
    int64_t sa = 0, sb = 0;
    if (!collapse_batch(*ae, batch.size(), sa)) {
      ae = dense_copy(ae);
      sa = M * K;
    }
    if (!collapse_batch(*be, batch.size(), sb)) {
      be = dense_copy(be);
      sb = K * N;
    }
    gemm(ae, be, *out, product(batch), M, N, K, sa, sb, 1.0, 0.0, nullptr, 0, 0, 0);
  }
  std::vector<int64_t> result = out_shape;
  if (squeeze_n) result.erase(result.end() - 1);
  if (squeeze_m) result.erase(result.end() - (squeeze_n ? 1 : 2));
  if (result != out_shape) out = view(out, result, contiguous_strides(result), 0);
  return out;
}

TensorPtr bmm(const TensorPtr& left, const TensorPtr& right) {  // tensor.cpp:25066
  if (left->dim() != 3 || right->dim() != 3) throw std::invalid_argument("bmm expects 3-D tensors");
  if (left->sizes[0] != right->sizes[0]) throw std::invalid_argument("bmm batch sizes must match");
  return hip::matmul(left, right);
}

// addmm (tensor.cpp:25184-25366): beta * input (narrowed) + alpha * mat1 . mat2.
TensorPtr addmm(const TensorPtr& input, const TensorPtr& mat1, const TensorPtr& mat2, double beta, double alpha) {
  guard("addmm", {input, mat1, mat2});
  require_same_dtype("addmm operands", {input, mat1, mat2});
  require_float("addmm", mat1->dtype);
  if (mat1->dim() != 2 || mat2->dim() != 2) throw std::invalid_argument("addmm expects 2-D mat1 and mat2 tensors");
  const int64_t M = mat1->sizes[0], K = mat1->sizes[1], N = mat2->sizes[1];
  if (mat2->sizes[0] != K) throw std::invalid_argument("addmm matrix shapes cannot be multiplied");
  if (!broadcasts_to(input->sizes, {M, N})) {
    throw std::invalid_argument("addmm input is not broadcastable to the matrix product shape");
  }
  auto e = broadcast_view(input, {M, N});
  auto out = empty({M, N}, mat1->dtype, mat1->device);
  if (out->numel() != 0) {
    gemm(mat1, mat2, *out, 1, M, N, K, 0, 0, alpha, beta, e, e->strides[0], e->strides[1], 0);
  }
  return out;
}

// baddbmm (tensor.cpp:25557): out[i] = beta * input[i] + alpha * batch1[i] . batch2[i].
TensorPtr baddbmm(const TensorPtr& input, const TensorPtr& batch1, const TensorPtr& batch2, double beta,
                  double alpha) {
  guard("baddbmm", {input, batch1, batch2});
  require_same_dtype("baddbmm operands", {input, batch1, batch2});
  require_float("baddbmm", batch1->dtype);
  if (batch1->dim() != 3 || batch2->dim() != 3 || batch1->sizes[0] != batch2->sizes[0] ||
      batch1->sizes[2] != batch2->sizes[1]) {
    throw std::invalid_argument("baddbmm expects batch1 [B,M,K] and batch2 [B,K,N]");
  }
  const int64_t B = batch1->sizes[0], M = batch1->sizes[1], K = batch1->sizes[2], N = batch2->sizes[2];
  if (!broadcasts_to(input->sizes, {B, M, N})) {
    throw std::invalid_argument("baddbmm input is not broadcastable to the batch product shape");
  }
  auto e = broadcast_view(input, {B, M, N});
  auto out = empty({B, M, N}, batch1->dtype, batch1->device);
  if (out->numel() != 0) {
    int64_t sa = 0, sb = 0;
    collapse_batch(*batch1, 1, sa);
    collapse_batch(*batch2, 1, sb);
    gemm(batch1, batch2, *out, B, M, N, K, sa, sb, alpha, beta, e, e->strides[1], e->strides[2], e->strides[0]);
  }
  return out;
}

// mtorch::conv2d (tensor.cpp:26490-27528): checks and output size as conv2d_output_size
// (:25941); groups == 1 runs the implicit GEMM on a packed weight cached on the weight's storage.
TensorPtr conv2d(const TensorPtr& input, const TensorPtr& weight, const TensorPtr& bias,
                 const std::vector<int64_t>& stride, const std::vector<int64_t>& padding,
                 const std::vector<int64_t>& dilation, int64_t groups) {
  const int d = guard("conv2d", {input, weight, bias});
  if (input->dim() != 3 && input->dim() != 4) throw std::invalid_argument("conv2d expects a 3-D or 4-D input tensor");
  if (weight->dim() != 4) throw std::invalid_argument("conv2d expects a 4-D weight tensor");
  if (groups <= 0) throw std::invalid_argument("conv2d groups must be positive");
  require_same_dtype("conv2d tensors", {input, weight, bias});
  require_float("conv2d", input->dtype);
  const auto [sh, sw] = conv_pair(stride, "stride", false);
  const auto [ph, pw] = conv_pair(padding, "padding", true);
  const auto [dh, dw] = conv_pair(dilation, "dilation", false);
  const bool unbatched = input->dim() == 3;
  const size_t o = unbatched ? 0 : 1;
  const int64_t B = unbatched ? 1 : input->sizes[0];
  const int64_t C = input->sizes[o], H = input->sizes[o + 1], W = input->sizes[o + 2];
  const int64_t O = weight->sizes[0], KH = weight->sizes[2], KW = weight->sizes[3];
  if (C != weight->sizes[1] * groups) {
    throw std::invalid_argument("conv2d input channels must equal weight channels times groups");
  }
  if (O % groups != 0) throw std::invalid_argument("conv2d output channels must be divisible by groups");
  if (bias && !(bias->dim() == 1 && bias->sizes[0] == O)) {
    throw std::invalid_argument("conv2d bias must be 1-D with out_channels elements");
  }
  const int64_t OH = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
  const int64_t OW = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
  if (OH <= 0 || OW <= 0) throw std::invalid_argument("conv2d output size must be positive");
  auto x = as_dense(input);
  auto w = as_dense(weight);
  auto b = bias ? as_dense(bias) : nullptr;
  auto out = empty({B, O, OH, OW}, input->dtype, input->device);
  if (out->numel() != 0) {
    if (groups == 1) {
      const void* packed = packed_conv_weight(w, d, O, C, KH, KW);
      check(mthip_conv2d_prepacked(d, code(input->dtype), data(*x), packed, data_or_null(b), data(*out), B, C, H, W,
                                   O, KH, KW, sh, sw, ph, pw, dh, dw, nullptr));
    } else {
      check(mthip_conv2d(d, code(input->dtype), data(*x), data(*w), data_or_null(b), data(*out), B, C, H, W, O, KH, KW,
                         sh, sw, ph, pw, dh, dw, groups, nullptr));
    }
  }
  if (unbatched) out = view(out, {O, OH, OW}, {OH * OW, OW, 1}, 0);
  return out;
}

// mtorch::scaled_dot_product_attention (tensor.cpp:30930-31324; sdpa_prefix_plan :30318-30391).
// q/k/v/mask are read through their strides: head splits made by view/transpose stay views.
TensorPtr scaled_dot_product_attention(const TensorPtr& query, const TensorPtr& key, const TensorPtr& value,
                                       const TensorPtr& attn_mask, double dropout_p, bool is_causal,
                                       std::optional<double> scale, bool enable_gqa) {
  const std::string op = "scaled_dot_product_attention";
  for (const TensorPtr& t : {query, key, value}) {
    if (t->dtype != ScalarType::Float16 && t->dtype != ScalarType::Float32 && t->dtype != ScalarType::Float64) {
      throw std::invalid_argument(op + " expects floating point query, key, and value");
    }
  }
  if (query->dtype != key->dtype || query->dtype != value->dtype) {
    throw std::invalid_argument(op + " query, key, and value must have the same dtype");
  }
  if (attn_mask && attn_mask->dtype != ScalarType::Bool && attn_mask->dtype != ScalarType::Float32 &&
      attn_mask->dtype != query->dtype) {
    throw std::invalid_argument(op + " attn_mask must be bool, float32, or match query dtype");
  }
  if (dropout_p < 0.0 || dropout_p > 1.0) throw std::invalid_argument(op + " dropout_p must be between 0 and 1");
  const int d = guard(op, {query, key, value, attn_mask});
  require_float(op, query->dtype);
  if (query->dim() < 2 || key->dim() < 2 || value->dim() < 2) {
    throw std::invalid_argument(op + " expects tensors with rank >= 2");
  }
  if (query->dim() != key->dim() || query->dim() != value->dim()) {
    throw std::invalid_argument(op + " query, key, and value ranks must match");
  }
  const size_t rank = query->sizes.size();
  const int64_t E = query->sizes[rank - 1];
  if (key->sizes[rank - 1] != E) throw std::invalid_argument(op + " query and key embedding dimensions must match");
  const int64_t Lk = key->sizes[rank - 2];
  if (value->sizes[rank - 2] != Lk) throw std::invalid_argument(op + " key and value sequence lengths must match");
  const int64_t Lq = query->sizes[rank - 2], Ev = value->sizes[rank - 1];
  const std::vector<int64_t> prefix(query->sizes.begin(), query->sizes.end() - 2);
  int64_t ratio = 1;
  if (!enable_gqa) {
    if (std::vector<int64_t>(key->sizes.begin(), key->sizes.end() - 2) != prefix ||
        std::vector<int64_t>(value->sizes.begin(), value->sizes.end() - 2) != prefix) {
      throw std::invalid_argument(op + " leading dimensions must match");
    }
  } else {
    if (rank < 3) throw std::invalid_argument(op + " enable_gqa requires a head dimension");
    const std::vector<int64_t> outer(prefix.begin(), prefix.end() - 1);
    if (std::vector<int64_t>(key->sizes.begin(), key->sizes.end() - 3) != outer ||
        std::vector<int64_t>(value->sizes.begin(), value->sizes.end() - 3) != outer) {
      throw std::invalid_argument(op + " leading dimensions must match for enable_gqa");
    }
    if (key->sizes[rank - 3] != value->sizes[rank - 3]) {
      throw std::invalid_argument(op + " key and value heads must match for enable_gqa");
    }
    if (key->sizes[rank - 3] <= 0 || query->sizes[rank - 3] % key->sizes[rank - 3] != 0) {
      throw std::invalid_argument(op + " query heads must be divisible by key/value heads for enable_gqa");
    }
    ratio = query->sizes[rank - 3] / key->sizes[rank - 3];
  }
  std::vector<int64_t> attn_shape = prefix;
  attn_shape.insert(attn_shape.end(), {Lq, Lk});
  if (attn_mask && !broadcasts_to(attn_mask->sizes, attn_shape)) {
    throw std::invalid_argument(op + " attn_mask is not broadcastable to attention weights");
  }
  std::vector<int64_t> out_shape = prefix;
  out_shape.insert(out_shape.end(), {Lq, Ev});
  auto out = empty(out_shape, query->dtype, query->device);
  if (out->numel() == 0) return out;
  if (dropout_p == 1.0) {
    fill_inplace(out, 0.0);
    return out;
  }
  if (dropout_p != 0.0) throw std::invalid_argument(op + " dropout_p is only supported when it is 0 or 1");
  const size_t npre = prefix.size();
  const int64_t H = npre ? prefix.back() : 1;
  const int64_t B = npre ? product(std::vector<int64_t>(prefix.begin(), prefix.end() - 1)) : 1;
  const int64_t Hk = H / ratio;
  // {batch, head, row} element strides of a q/k/v operand whose last dim is unit-stride.
  auto strides3 = [&](TensorPtr t, std::vector<int64_t>& s) {
    if (t->strides[rank - 1] != 1) t = dense_copy(t);
    int64_t bs = 0;
    if (npre >= 2 && !collapse_batch(*t, npre - 1, bs)) {
      t = dense_copy(t);
      collapse_batch(*t, npre - 1, bs);
    }
    const int64_t hs = npre >= 1 && t->sizes[npre - 1] > 1 ? t->strides[npre - 1] : 0;
    s = {bs, hs, t->strides[rank - 2]};
    return t;
  };
  std::vector<int64_t> qs, ks, vs, ms;
  TensorPtr q = strides3(query, qs), k = strides3(key, ks), v = strides3(value, vs);
  int mask_kind = MTHIP_MASK_NONE, mask_dtype = MTHIP_F32;
  TensorPtr m;
  if (attn_mask) {
    m = broadcast_view(attn_mask, attn_shape);
    int64_t bs = 0;
    if (npre >= 2 && !collapse_batch(*m, npre - 1, bs)) {
      m = dense_copy(m);
      collapse_batch(*m, npre - 1, bs);
    }
    const int64_t hs = npre >= 1 ? m->strides[npre - 1] : 0;
    ms = {bs, hs, m->strides[attn_shape.size() - 2], m->strides[attn_shape.size() - 1]};
    mask_kind = m->dtype == ScalarType::Bool ? MTHIP_MASK_BOOL : MTHIP_MASK_ADD;
    mask_dtype = code(m->dtype);
  }
  check(mthip_sdpa(d, code(query->dtype), data(*q), qs.data(), data(*k), ks.data(), data(*v), vs.data(), data(*out),
                   nullptr, B, H, Hk, Lq, Lk, E, Ev, mask_kind, mask_dtype, m ? data(*m) : nullptr,
                   m ? ms.data() : nullptr, is_causal ? 1 : 0, scale ? 1 : 0, scale ? *scale : 0.0));
  return out;
}

// ============================================================================ normalisation

// mtorch::group_norm (tensor.cpp:18643-18963): statistics per (batch, group) over C/G * inner.
TensorPtr group_norm(const TensorPtr& input, int64_t num_groups, const TensorPtr& weight, const TensorPtr& bias,
                     double eps) {
  if (input->dtype != ScalarType::Float16 && input->dtype != ScalarType::Float32 &&
      input->dtype != ScalarType::Float64) {
    throw std::invalid_argument("group_norm expects a floating point input");
  }
  if (input->dim() < 2) throw std::invalid_argument("group_norm expected input rank of at least 2");
  if (num_groups <= 0) throw std::invalid_argument("group_norm num_groups must be positive");
  const int64_t B = input->sizes[0], C = input->sizes[1];
  if (C % num_groups != 0) throw std::invalid_argument("group_norm num_channels must be divisible by num_groups");
  const int64_t inner = product(std::vector<int64_t>(input->sizes.begin() + 2, input->sizes.end()));
  if ((C / num_groups) * inner <= 1) throw std::invalid_argument("group_norm expected more than 1 value per group");
  const int d = guard("group_norm", {input, weight, bias});
  if (weight && weight->sizes != std::vector<int64_t>{C}) {
    throw std::invalid_argument("group_norm weight must have shape [C]");
  }
  if (bias && bias->sizes != std::vector<int64_t>{C}) throw std::invalid_argument("group_norm bias must have shape [C]");
  require_same_dtype("group_norm tensors", {input, weight, bias});
  require_float("group_norm", input->dtype);
  auto x = as_dense(input);
  auto w = weight ? as_dense(weight) : nullptr;
  auto b = bias ? as_dense(bias) : nullptr;
  auto out = empty(input->sizes, input->dtype, input->device);
  if (out->numel() != 0) {
    check(mthip_group_norm(d, code(input->dtype), data(*x), data_or_null(w), data_or_null(b), data(*out), B, C, inner,
                           num_groups, eps, 0, code(input->dtype)));
  }
  return out;
}

// mtorch::layer_norm (tensor.cpp:17386-17708) over the trailing normalized_shape elements.
TensorPtr layer_norm(const TensorPtr& input, const std::vector<int64_t>& normalized_shape, const TensorPtr& weight,
                     const TensorPtr& bias, double eps) {
  if (normalized_shape.empty()) throw std::invalid_argument("layer_norm normalized_shape must not be empty");
  if (input->dtype != ScalarType::Float16 && input->dtype != ScalarType::Float32 &&
      input->dtype != ScalarType::Float64) {
    throw std::invalid_argument("layer_norm expects a floating point input");
  }
  if (static_cast<int64_t>(normalized_shape.size()) > input->dim()) {
    throw std::invalid_argument("layer_norm normalized_shape exceeds input rank");
  }
  if (!std::equal(normalized_shape.begin(), normalized_shape.end(), input->sizes.end() - normalized_shape.size())) {
    throw std::invalid_argument("layer_norm normalized_shape must match the input tail dimensions");
  }
  const int d = guard("layer_norm", {input, weight, bias});
  if (weight && weight->sizes != normalized_shape) {
    throw std::invalid_argument("layer_norm weight shape must match normalized_shape");
  }
  if (bias && bias->sizes != normalized_shape) {
    throw std::invalid_argument("layer_norm bias shape must match normalized_shape");
  }
  require_same_dtype("layer_norm tensors", {input, weight, bias});
  require_float("layer_norm", input->dtype);
  const int64_t N = product(normalized_shape);
  const int64_t rows = N == 0 ? 0 : input->numel() / N;
  auto x = as_dense(input);
  auto w = weight ? as_dense(weight) : nullptr;
  auto b = bias ? as_dense(bias) : nullptr;
  auto out = empty(input->sizes, input->dtype, input->device);
  if (out->numel() != 0) {
    check(mthip_layer_norm(d, code(input->dtype), data(*x), data_or_null(w), data_or_null(b), data(*out), rows, N, eps,
                           code(input->dtype)));
  }
  return out;
}

// softmax_impl (tensor.cpp:15145-15221).  The reference's float32 kernel divides by the row
// total for rank <= 2 and multiplies by its reciprocal otherwise; its float16 kernel multiplies
// (:7535-7537, 7581-7588, 7708-7710, 7789-7796); a dtype other than the input's takes the
// generic path, which reads the input at its own precision, divides, and narrows only the
// result (:15165-15207).  A dim other than the last runs on a permuted dense copy.
TensorPtr softmax(const TensorPtr& input, int64_t dim, ScalarType dtype) {
  const int d = guard("softmax", {input});
  const int64_t rank = input->dim();
  const int64_t axis = rank == 0 ? 0 : (dim < 0 ? dim + rank : dim);
  if (rank != 0 && (axis < 0 || axis >= rank)) throw std::out_of_range("dimension out of range");
  if (!(input->dtype == ScalarType::Float16 || input->dtype == ScalarType::Float32 ||
        input->dtype == ScalarType::Float64) ||
      !(dtype == ScalarType::Float16 || dtype == ScalarType::Float32 || dtype == ScalarType::Float64)) {
    throw std::runtime_error("softmax(): input dtype must be floating point");
  }
  require_float("softmax", dtype);
  const bool narrowing = input->dtype == ScalarType::Float32 && dtype == ScalarType::Float16;
  TensorPtr src = (dtype == input->dtype || narrowing) ? input : cast(input, dtype);
  if (rank == 0) src = view(src, {1}, {1}, src->offset);
  const int64_t r = src->dim();
  const bool last = axis == r - 1;
  const bool divide = (dtype == ScalarType::Float32 && r <= 2) || !last || dtype != input->dtype;
  std::vector<int64_t> perm;
  for (int64_t i = 0; i < r; ++i) {
    if (i != axis) perm.push_back(i);
  }
  perm.push_back(axis);
  std::vector<int64_t> moved_sizes, moved_strides;
  for (int64_t p : perm) {
    moved_sizes.push_back(src->sizes[static_cast<size_t>(p)]);
    moved_strides.push_back(src->strides[static_cast<size_t>(p)]);
  }
  auto moved = as_dense(view(src, moved_sizes, moved_strides, src->offset));
  auto res = empty(moved_sizes, src->dtype, input->device);
  const int64_t cols = moved_sizes.back();
  const int64_t rows = cols == 0 ? 0 : moved->numel() / cols;
  if (res->numel() != 0) {
    check(mthip_softmax_lastdim(d, code(src->dtype), data(*moved), data(*res), rows, cols, divide ? 1 : 0));
  }
  TensorPtr out = res;
  if (!last) {
    std::vector<int64_t> back_sizes(static_cast<size_t>(r)), back_strides(static_cast<size_t>(r));
    const auto res_strides = res->strides;
    for (int64_t i = 0; i < r; ++i) {
      back_sizes[static_cast<size_t>(perm[static_cast<size_t>(i)])] = moved_sizes[static_cast<size_t>(i)];
      back_strides[static_cast<size_t>(perm[static_cast<size_t>(i)])] = res_strides[static_cast<size_t>(i)];
    }
    out = dense_copy(view(res, back_sizes, back_strides, 0));
  }
  if (narrowing) out = cast(out, dtype);
  if (rank == 0) out = view(out, {}, {}, 0);
  return out;
}

}  // namespace mtorch::hip
