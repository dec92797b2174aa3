// GPU backend entry points for mtorch's C++ core, over libmthip's C ABI (include/mthip.h).
//
// This translation unit is compiled inside kazhiramatsu/mtorch, next to cpp/mtorch/core: it
// includes the reference's own tensor.h unchanged.  Each function mirrors the public op of the
// same name in tensor.h and is what the dispatch check at the top of that op calls when an
// operand lives on the GPU (the hook-point convention of docs/design/08-phase5-device-layer.md
// section 4: "route to the backend namespace function ... backend entry points mirror the public
// signature"; CUDA never falls back silently).  A call such as
//
//   TensorPtr linear(const TensorPtr& input, const TensorPtr& weight, const TensorPtr& bias) {
//     if (hip::on_gpu(input) || hip::on_gpu(weight) || hip::on_gpu(bias))
//       return hip::linear(input, weight, bias);
//     ...existing CPU path...
//
// is the whole change to tensor.cpp per op; py_linear (module.cpp:6778-6804) and every other
// binding in module.cpp stay as they are.
#pragma once

#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "mtorch/core/tensor.h"

namespace mtorch::hip {

// Device tag of GPU storages.  tensor.h:22-25 names CPU (0) and Metal (1); the reference's
// device plan appends DeviceType::CUDA = 2 (docs/design/08-phase5-device-layer.md:497-535).
// Until tensor.h carries that member, GPU storages are tagged with the same value here.
inline constexpr DeviceType kGpu = static_cast<DeviceType>(2);

// True when t is non-null and its storage lives on a GPU.
bool on_gpu(const TensorPtr& t);
// The GPU device with the given index (index -1, "unindexed", means device 0).
Device gpu_device(int64_t index = 0);
// "cpu", "mps" or "cuda[:i]" -- device_name (tensor.h:54) extended with the GPU tag.
std::string device_string(const Device& device);
// Number of visible GPUs (mtorch.cuda.device_count; mtorch/__init__.py:2320-2321).
int64_t device_count();
// Waits until every op enqueued on the device has finished.
void synchronize(const Device& device);

// Uninitialised contiguous GPU tensor (empty_strided, tensor.h:150-155, for the GPU).
TensorPtr empty(const std::vector<int64_t>& sizes, ScalarType dtype, const Device& device);

// ---------------------------------------------------------------- data movement
TensorPtr to(const TensorPtr& input, ScalarType dtype, Device device, bool copy = false);  // tensor.h:157
TensorPtr contiguous(const TensorPtr& input);                                             // Tensor::contiguous
void copy_from(const TensorPtr& destination, const TensorPtr& source);                    // Tensor::copy_from
void fill_inplace(const TensorPtr& tensor, double value);                                 // Tensor::fill_inplace

// ---------------------------------------------------------------- elementwise
TensorPtr binary_tensor_tensor(const TensorPtr& left, const TensorPtr& right, const std::string& op);
TensorPtr binary_tensor_scalar(const TensorPtr& left, double scalar, ScalarType scalar_dtype, const std::string& op);
TensorPtr binary_scalar_tensor(double scalar, ScalarType scalar_dtype, const TensorPtr& right, const std::string& op);
TensorPtr silu(const TensorPtr& input);
TensorPtr gelu(const TensorPtr& input, const std::string& approximate = "none");

// ---------------------------------------------------------------- contractions
TensorPtr linear(const TensorPtr& input, const TensorPtr& weight, const TensorPtr& bias = nullptr);
TensorPtr matmul(const TensorPtr& left, const TensorPtr& right);
TensorPtr bmm(const TensorPtr& left, const TensorPtr& right);
TensorPtr addmm(const TensorPtr& input, const TensorPtr& mat1, const TensorPtr& mat2, double beta = 1.0,
                double alpha = 1.0);
TensorPtr baddbmm(const TensorPtr& input, const TensorPtr& batch1, const TensorPtr& batch2, double beta = 1.0,
                  double alpha = 1.0);
TensorPtr conv2d(const TensorPtr& input, const TensorPtr& weight, const TensorPtr& bias = nullptr,
                 const std::vector<int64_t>& stride = {1, 1}, const std::vector<int64_t>& padding = {0, 0},
                 const std::vector<int64_t>& dilation = {1, 1}, int64_t groups = 1);
TensorPtr scaled_dot_product_attention(const TensorPtr& query, const TensorPtr& key, const TensorPtr& value,
                                       const TensorPtr& attn_mask = nullptr, double dropout_p = 0.0,
                                       bool is_causal = false, std::optional<double> scale = std::nullopt,
                                       bool enable_gqa = false);

// ---------------------------------------------------------------- normalisation
TensorPtr group_norm(const TensorPtr& input, int64_t num_groups, const TensorPtr& weight = nullptr,
                     const TensorPtr& bias = nullptr, double eps = 1e-5);
TensorPtr layer_norm(const TensorPtr& input, const std::vector<int64_t>& normalized_shape,
                     const TensorPtr& weight = nullptr, const TensorPtr& bias = nullptr, double eps = 1e-5);
TensorPtr softmax(const TensorPtr& input, int64_t dim, ScalarType dtype);

}  // namespace mtorch::hip
