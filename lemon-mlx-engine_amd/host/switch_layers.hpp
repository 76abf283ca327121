// switch_layers.hpp -- C++ host classes over the MI355X MoE C ABI
// (include/moe_mi355x.h) with the reference's module interface:
//
//   SwitchLinear, SwitchGLU, gather_sort, scatter_unsort
//       include/mlx-lm/common/switch_layers.h:15-108
//   QuantizationInfo, QuantizedWeightRegistry
//       include/mlx-lm/common/quantized_linear.h:16-61
//   moe_route
//       include/mlx-lm/common/gated_delta.h:111-119
//
// Same class names, constructor arguments, weight_map keys, call signatures and
// output shapes as the reference; `array` stands where the reference has
// mlx::core::array: a contiguous device tensor (bf16, fp32, uint32 or int32)
// owning a HIP allocation.  Work is enqueued on the calling thread's default
// stream (set_default_stream; the reference keeps a thread-local stream,
// src/common/generate.cpp:44-56) and is asynchronous, as MLX evaluation is
// lazy; array::to_host waits for it.  Status codes from the ABI become
// std::invalid_argument (bad shapes, unsupported sizes, bad indices) or
// std::runtime_error (HIP failures), as MLX's op validation and the engine's
// loaders throw (src/llm/llm_factory.cpp:346).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <string>
#include <tuple>
#include <unordered_map>
#include <utility>
#include <vector>

#include "moe_mi355x.h"

namespace mlx_lm {
namespace mi355x {

enum class Dtype { bfloat16, float32, uint32, int32 };
size_t itemsize(Dtype d);
const char* dtype_name(Dtype d);

using Shape = std::vector<int32_t>;  // as mlx::core::Shape

// The stream every call of this layer enqueues on (thread-local; default: the
// null stream).
hipStream_t default_stream();
void set_default_stream(hipStream_t stream);

// Throws the exception the reference would for an ABI status (no-op for MOE_OK).
void check_status(int status, const char* where);

class array {
 public:
  array() = default;                      // no data (an unloaded weight)
  array(Shape shape, Dtype dtype);        // uninitialised device memory
  static array from_host(const void* data, Shape shape, Dtype dtype);  // synchronous upload
  void to_host(void* dst) const;          // waits for the default stream, then copies

  const Shape& shape() const { return shape_; }
  int32_t shape(int axis) const;          // negative axes count from the end
  int ndim() const { return static_cast<int>(shape_.size()); }
  size_t size() const;
  size_t nbytes() const { return size() * itemsize(dtype_); }
  Dtype dtype() const { return dtype_; }
  bool has_data() const { return static_cast<bool>(buf_); }

  void* raw() { return buf_.get(); }
  const void* raw() const { return buf_.get(); }
  template <class T>
  T* data() { return static_cast<T*>(raw()); }
  template <class T>
  const T* data() const { return static_cast<const T*>(raw()); }

  // Same buffer, new shape of equal size.
  array reshape(Shape shape) const;

 private:
  std::shared_ptr<void> buf_;
  Shape shape_;
  Dtype dtype_ = Dtype::float32;
};

// ---- quantized weights (quantized_linear.h:16-61) ----------------------------
struct QuantizationInfo {
  array scales;
  std::optional<array> biases;
  int group_size;
  int bits;
};

class QuantizedWeightRegistry {
 public:
  static QuantizedWeightRegistry& instance();
  void register_weight(const array* weight_ptr, array scales, std::optional<array> biases, int group_size,
                       int bits);
  const QuantizationInfo* find(const array* weight_ptr) const;
  void unregister(const array* weight_ptr);
  void clear() { registry_.clear(); }
  size_t size() const { return registry_.size(); }

 private:
  QuantizedWeightRegistry() = default;
  std::unordered_map<const array*, QuantizationInfo> registry_;
};

// ---- gather_sort / scatter_unsort (switch_layers.cpp:17-46) ------------------
// (sorted_x, sorted_indices, inverse_order): x [..., M, K] flattened to
// [rows, M, K] over its leading axes; indices [..., m] with m indices per row;
// sorted_x [P, M, K] = x rows order // m, sorted_indices [P] ascending (stable),
// inverse_order [P].  num_experts bounds the index values (the bucket
// histogram's size); indices at or above it are an error in the reference and
// sort last here.
std::tuple<array, array, array> gather_sort(const array& x, const array& indices,
                                            int num_experts = 1024);
array scatter_unsort(const array& x, const array& inv_order, const Shape* shape = nullptr);

// ---- moe_route (gated_delta.h:111-119) --------------------------------------
// Top-k of the router logits [..., E] (bf16) with the softmax over the k
// selected: (indices [..., k] uint32 in descending logit order, lower expert
// first on ties; scores [..., k] float32 holding bf16 values).
std::pair<array, array> moe_route(const array& logits, int k);

// Device scratch that grows on demand (one per layer object).
class Workspace {
 public:
  void* get(size_t bytes);
  size_t capacity() const { return bytes_; }

 private:
  std::shared_ptr<void> buf_;
  size_t bytes_ = 0;
};

// ---- SwitchLinear (switch_layers.h:26-93) ------------------------------------
class SwitchLinear {
 public:
  SwitchLinear(int input_dims, int output_dims, int num_experts, bool bias = false);

  // x [..., M, input_dims] bf16, indices (uint32 or int32) broadcastable with
  // x's batch axes -> [broadcast batch..., M, output_dims] bf16.  The weight
  // must be registered quantized (gather_qmm); sorted_indices asserts that the
  // indices ascend.
  array operator()(const array& x, const array& indices, bool sorted_indices = false);

  std::unordered_map<std::string, array*> weight_map();

  const array& weight() const { return weight_; }
  int output_dims() const { return output_dims_; }
  int num_experts() const { return num_experts_; }

  void adopt_fused_weight(array w, array scales, std::optional<array> biases, int group_size, int bits);
  void release_weight();

 private:
  array weight_;               // [num_experts, output_dims, input_dims * bits / 32] uint32 when quantized
  std::optional<array> bias_;  // [num_experts, output_dims] bf16
  int input_dims_;
  int output_dims_;
  int num_experts_;
  // broadcast index maps, cached per (x batch shape, indices shape) like the
  // reference's default_lhs_indices cache (switch_layers.cpp:60-77)
  Shape cache_xb_, cache_ib_;
  std::optional<array> lhs_map_, rhs_map_;
  Workspace ws_;
};

// ---- GPT-OSS's clipped SwiGLU -------------------------------------------------
// swiglu(x_linear, x_glu) of src/llm/models/gptoss.cpp:50-58 (alpha 1.702,
// limit 7), bf16 in and out (moe_gptoss_swiglu); GPT-OSS's MoE MLP calls it as
// gptoss_swiglu(x_gate, x_up) (:158).
array gptoss_swiglu(const array& x_linear, const array& x_glu);

// ---- SwitchGLU (switch_layers.h:95-108) --------------------------------------
class SwitchGLU {
 public:
  // activation: the moe_activation between gate|up and down (the reference's
  // SwitchGLU always applies SwiGLU; MOE_ACT_GPTOSS runs GPT-OSS's expert MLP,
  // gptoss.cpp:141-167, through the same class)
  SwitchGLU(int input_dims, int hidden_dims, int num_experts, bool bias = false,
            int activation = MOE_ACT_SWIGLU);

  // x [..., input_dims] bf16, indices [..., k] -> [..., k, input_dims] bf16.
  array operator()(const array& x, const array& indices);

  std::unordered_map<std::string, array*> weight_map();

 private:
  // true when gate, up and down are quantized alike and carry no linear bias:
  // then one fused call runs the whole expert MLP (moe_switch_glu)
  bool fused_ready() const;

  SwitchLinear gate_proj_;
  SwitchLinear up_proj_;
  SwitchLinear down_proj_;
  int input_dims_;
  int hidden_dims_;
  int num_experts_;
  int activation_;
  Workspace ws_;
};

}  // namespace mi355x
}  // namespace mlx_lm
