// quantize_utils.hpp -- the loader steps between a checkpoint's tensors and
// the host classes' weights:
//
//   PerLayerQuantization, parse_quantization
//       include/mlx-lm/common/base_config.h:22-55, src/common/base_config.cpp:28-73
//   sanitize_moe_experts
//       the per-expert -> stacked step of the MoE models' sanitize:
//       src/llm/models/qwen3_moe.cpp:291-318, qwen3_next.cpp:700-748,
//       deepseek_v3.cpp:531-555, phimoe.cpp:208-235
//   register_quantized_weights
//       src/common/quantize_utils.cpp:14-104
//   load_weights
//       src/common/safetensors.cpp:79-90 (assign by weight_map name)
//
// The reference runs them as load -> sanitize -> register -> load_weights
// (src/llm/llm_factory.cpp:106-119, 350); here sanitize runs on host tensors before
// the upload, so stacked experts reach the device once.
#pragma once

#include <optional>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "json.hpp"
#include "safetensors.hpp"
#include "switch_layers.hpp"

namespace mlx_lm {
namespace mi355x {

struct Quantization {
  int group_size = 64;
  int bits = 4;
};

// config.json's "quantization" entry: defaults plus per-prefix entries (an
// object: its own group_size/bits; false: skip).
struct PerLayerQuantization {
  std::optional<Quantization> default_quantization;
  std::unordered_map<std::string, std::optional<Quantization>> per_layer;  // nullopt = skip

  // The prefix's entry when it has one (nullopt for a skip), else the default.
  std::optional<Quantization> quantization_for(const std::string& prefix) const;
};

// nullopt when the config has no "quantization" entry.  Keys with the VLM
// prefix "language_model." are stored without it; the keys group_size, bits,
// mode, quant_method, linear_class and quantization_mode are not prefixes.
std::optional<PerLayerQuantization> parse_quantization(const Json& config);

Json read_json_file(const std::string& path);

// Where a model family keeps its MoE experts.
struct MoeNaming {
  std::string block;          // module under model.layers.{l}: "mlp" or "block_sparse_moe"
  std::string experts_key;    // config key of the routed expert count
  int experts_default;        // its value when the key is absent or null (-1: required)
  std::string intermediate_key;  // config key of the experts' hidden width
  int intermediate_default;      // (-1: required)
  // (per-expert projection name, switch_mlp projection name)
  std::vector<std::pair<std::string, std::string>> projs;
};

// qwen3_moe, qwen3_next, deepseek_v3, phimoe; throws std::invalid_argument
// for another model_type.
const MoeNaming& moe_naming(const std::string& model_type);

// Stacks model.layers.{l}.<block>.experts.{e}.<proj>.{weight,scales,biases}
// (e = 0 .. E-1) into model.layers.{l}.<block>.switch_mlp.<proj'>.{...} of
// shape [E, ...] and removes the per-expert tensors, for every layer that
// holds experts.0.  A layer with some of its E experts missing, or with
// experts of different dtype or shape, throws std::invalid_argument.
// Returns the number of stacked tensors.  (Qwen3-MoE's own sanitize stacks
// only .weight; stacking scales and biases too is what its load_weights,
// Qwen3-Next's and DeepSeek-V3's do, and what a per-expert quantized
// checkpoint needs.)
int sanitize_moe_experts(HostTensors& weights, const Json& config);

// For every "<p>.scales" with a "<p>.weight" in `weights`: registers the
// module member weight_map["<p>.weight"] as quantized with those scales, the
// optional "<p>.biases", and the prefix's bits and group size; then removes
// scales and biases from `weights`.  Prefixes absent from weight_map are
// skipped and keep their scales and biases.  Embedding prefixes, which the
// reference dequantizes at load, are left untouched: no MoE block reads them.
// Without a quantization config nothing is registered.
void register_quantized_weights(std::unordered_map<std::string, array>& weights,
                                const std::optional<PerLayerQuantization>& quantization,
                                const std::unordered_map<std::string, array*>& weight_map);

// Assigns weights[name] to *weight_map[name] for every name in both; returns
// how many were assigned.
int load_weights(const std::unordered_map<std::string, array>& weights,
                 const std::unordered_map<std::string, array*>& weight_map);

}  // namespace mi355x
}  // namespace mlx_lm
