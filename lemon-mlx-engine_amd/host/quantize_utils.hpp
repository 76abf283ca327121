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
  std::string stacked = "switch_mlp";  // module of the stacked experts (GPT-OSS: "experts")
  // a fused experts.gate_up_proj: "" none, "halves" (Qwen3.5-MoE, split at
  // the middle row), "interleaved" (GPT-OSS, even rows gate, odd rows up)
  std::string fused = "";
  bool vlm = false;          // config under text_config, language_model. names (Qwen3.5)
  bool linear_bias = false;  // SwitchLinear biases on the experts (GPT-OSS)
  int activation = MOE_ACT_SWIGLU;
};

// qwen3_moe, qwen3_next, qwen3_5_moe (and qwen3_5), deepseek_v3, phimoe,
// gpt_oss; throws std::invalid_argument for another model_type.
const MoeNaming& moe_naming(const std::string& model_type);

// The text model's config: config["text_config"] for a VLM naming that nests
// it there (qwen35_moe.cpp:31-32), else config itself.
const Json& text_config(const Json& config);

// The MoE part of the models' sanitize, on host tensors, for every layer:
//  * (Qwen3.5) VLM names: "language_model." stripped, "model.language_model."
//    -> "model.", vision tensors dropped (qwen35_moe.cpp:1046-1078);
//  * a fused model.layers.{l}.<block>.experts.gate_up_proj [E, 2I, H] (the bare
//    tensor the reference splits, or its .weight/.scales/.biases quantized
//    form, split row for row alike) into <stacked>.gate_proj / up_proj:
//    halves for Qwen3.5 (qwen35_moe.cpp:1080-1107), even / odd rows for
//    GPT-OSS, whose experts.gate_up_proj_bias [E, 2I] splits the same way into
//    gate_proj.bias / up_proj.bias (gptoss.cpp:305-350); experts.down_proj
//    becomes <stacked>.down_proj.weight and (GPT-OSS) experts.down_proj_bias
//    down_proj.bias.  GPT-OSS checkpoints that already hold gate_proj.weight
//    are left alone, as the reference's early return does;
//  * model.layers.{l}.<block>.experts.{e}.<proj>.{weight,scales,biases}
//    (e = 0 .. E-1) stacked into model.layers.{l}.<block>.switch_mlp.<proj'>.{...}
//    of shape [E, ...], the per-expert tensors removed, for every layer that
//    holds experts.0.  A layer with some of its E experts missing, or with
//    experts of different dtype or shape, throws std::invalid_argument.
// Returns the number of tensors written (stacked or split).  (Qwen3-MoE's own
// sanitize stacks only .weight; stacking scales and biases too is what its
// load_weights, Qwen3-Next's and DeepSeek-V3's do, and what a per-expert
// quantized checkpoint needs.)
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
