// quantize_utils.cpp -- the loader steps declared in quantize_utils.hpp.
#include "quantize_utils.hpp"

#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>

namespace mlx_lm {
namespace mi355x {

std::optional<Quantization> PerLayerQuantization::quantization_for(const std::string& prefix) const {
  const auto it = per_layer.find(prefix);
  if (it != per_layer.end()) return it->second;
  return default_quantization;
}

std::optional<PerLayerQuantization> parse_quantization(const Json& config) {
  if (!config.contains("quantization")) return std::nullopt;
  const Json& q = config.at("quantization");
  PerLayerQuantization plq;
  Quantization dq;
  dq.group_size = static_cast<int>(q.value("group_size", int64_t{64}));
  dq.bits = static_cast<int>(q.value("bits", int64_t{4}));
  plq.default_quantization = dq;
  static const std::set<std::string> skip = {"group_size", "bits",         "mode",
                                             "quant_method", "linear_class", "quantization_mode"};
  static const std::string vlm = "language_model.";
  for (const auto& [key, v] : q.fields()) {
    if (skip.count(key)) continue;
    const std::string k = key.compare(0, vlm.size(), vlm) == 0 ? key.substr(vlm.size()) : key;
    if (v.type() == Json::Type::boolean) {
      if (!v.boolean()) plq.per_layer[k] = std::nullopt;
    } else if (v.is_object()) {
      Quantization lq;
      lq.group_size = static_cast<int>(v.value("group_size", int64_t{dq.group_size}));
      lq.bits = static_cast<int>(v.value("bits", int64_t{dq.bits}));
      plq.per_layer[k] = lq;
    }
  }
  return plq;
}

Json read_json_file(const std::string& path) {
  std::ifstream f(path);
  if (!f) throw std::runtime_error("cannot open " + path);
  std::stringstream ss;
  ss << f.rdbuf();
  return parse_json(ss.str());
}

const MoeNaming& moe_naming(const std::string& model_type) {
  static const std::vector<std::pair<std::string, std::string>> same = {
      {"gate_proj", "gate_proj"}, {"up_proj", "up_proj"}, {"down_proj", "down_proj"}};
  static const std::map<std::string, MoeNaming> names = {
      // qwen3_moe.cpp:17-47, qwen3_next.cpp:21-70, deepseek_v3.cpp:21-62, phimoe.cpp:11-30
      {"qwen3_moe", {"mlp", "num_experts", -1, "moe_intermediate_size", -1, same}},
      {"qwen3_next", {"mlp", "num_experts", -1, "moe_intermediate_size", -1, same}},
      {"deepseek_v3", {"mlp", "n_routed_experts", 1, "moe_intermediate_size", -1, same}},
      {"phimoe", {"block_sparse_moe", "num_local_experts", 16, "intermediate_size", 6400,
                  {{"w1", "gate_proj"}, {"w3", "up_proj"}, {"w2", "down_proj"}}}},
      // qwen35_moe.cpp:25-70 (text_config), 1046-1160 (sanitize); llm_factory.cpp:143-145
      {"qwen3_5_moe", {"mlp", "num_experts", -1, "moe_intermediate_size", -1, same, "switch_mlp", "halves", true}},
      {"qwen3_5", {"mlp", "num_experts", -1, "moe_intermediate_size", -1, same, "switch_mlp", "halves", true}},
      // gptoss.cpp:11-38 (config), 118-178 (mlp.experts SwitchLinear(bias) x3, router), 305-350 (sanitize)
      {"gpt_oss", {"mlp", "num_local_experts", -1, "intermediate_size", -1, same, "experts", "interleaved", false,
                   true, MOE_ACT_GPTOSS}},
  };
  const auto it = names.find(model_type);
  if (it == names.end()) throw std::invalid_argument("model_type '" + model_type + "': MoE naming not supported");
  return it->second;
}

const Json& text_config(const Json& config) {
  if (config.contains("model_type") && moe_naming(config.at("model_type").str()).vlm &&
      config.contains("text_config"))
    return config.at("text_config");
  return config;
}

namespace {

// rows of a fused gate|up tensor along `axis` (E x 2I x rest) -> (gate, up):
// the first and second half, or the even and odd rows
std::pair<HostTensor, HostTensor> split_rows(const HostTensor& t, size_t axis, bool interleaved,
                                             const std::string& what) {
  if (axis >= t.shape.size() || t.shape[axis] % 2 != 0)
    throw std::invalid_argument(what + ": a fused gate|up tensor needs an even row count");
  const size_t n = t.numel();
  const size_t item = n ? t.nbytes / n : 0;
  size_t outer = 1, inner = item;
  for (size_t i = 0; i < axis; ++i) outer *= static_cast<size_t>(t.shape[i]);
  for (size_t i = axis + 1; i < t.shape.size(); ++i) inner *= static_cast<size_t>(t.shape[i]);
  const size_t rows = static_cast<size_t>(t.shape[axis]), half = rows / 2;
  HostTensor parts[2];
  for (int h = 0; h < 2; ++h) {
    HostTensor& o = parts[h];
    o.dtype = t.dtype;
    o.shape = t.shape;
    o.shape[axis] = static_cast<int32_t>(half);
    o.nbytes = t.nbytes / 2;
    std::shared_ptr<uint8_t> buf(new uint8_t[o.nbytes > 0 ? o.nbytes : 1], std::default_delete<uint8_t[]>());
    for (size_t a = 0; a < outer; ++a)
      for (size_t r = 0; r < half; ++r) {
        const size_t src = interleaved ? 2 * r + h : h * half + r;
        std::memcpy(buf.get() + (a * half + r) * inner, t.data + (a * rows + src) * inner, inner);
      }
    o.data = buf.get();
    o.owner = std::shared_ptr<const void>(buf, buf.get());
  }
  return {parts[0], parts[1]};
}

bool ends_with(const std::string& s, const std::string& suffix) {
  return s.size() >= suffix.size() && s.compare(s.size() - suffix.size(), suffix.size(), suffix) == 0;
}

// The fused-tensor and VLM-name steps of sanitize_moe_experts.
int sanitize_fused(HostTensors& weights, const MoeNaming& nm) {
  int written = 0;
  if (nm.vlm) {  // qwen35_moe.cpp:1046-1078
    HostTensors renamed;
    for (auto& [key, t] : weights) {
      if (key.rfind("vision_tower", 0) == 0 || key.rfind("model.visual", 0) == 0) continue;
      std::string k = key;
      if (k.rfind("language_model.", 0) == 0) k = k.substr(15);
      if (k.rfind("model.language_model.", 0) == 0) k = "model." + k.substr(21);
      renamed.insert_or_assign(k, std::move(t));
    }
    weights = std::move(renamed);
  }
  if (nm.fused.empty()) return 0;
  const bool interleaved = nm.fused == "interleaved";
  if (interleaved)  // gptoss.cpp:307-312: already split, nothing to do
    for (const auto& [k, t] : weights)
      if (k.find("gate_proj.weight") != std::string::npos) return 0;
  const std::string fused = ".experts.gate_up_proj";
  std::vector<std::string> keys;
  for (const auto& [k, t] : weights) keys.push_back(k);
  for (const std::string& k : keys) {
    const size_t pos = k.find(fused);
    if (pos == std::string::npos || k.rfind("model.layers.", 0) != 0) continue;
    const std::string block = k.substr(0, pos);  // model.layers.<l>.<block>
    const std::string rest = k.substr(pos + fused.size());
    const std::string dst = block + "." + nm.stacked + ".";
    auto it = weights.find(k);
    if (rest.empty() || rest == ".weight" || rest == ".scales" || rest == ".biases") {
      const std::string suffix = rest.empty() ? ".weight" : rest;
      auto [g, u] = split_rows(it->second, it->second.shape.size() - 2, interleaved, k);
      weights.erase(it);
      weights.insert_or_assign(dst + "gate_proj" + suffix, std::move(g));
      weights.insert_or_assign(dst + "up_proj" + suffix, std::move(u));
      written += 2;
    } else if (rest == "_bias" && interleaved) {  // gptoss.cpp:322-333
      auto [g, u] = split_rows(it->second, it->second.shape.size() - 1, true, k);
      weights.erase(it);
      weights.insert_or_assign(dst + "gate_proj.bias", std::move(g));
      weights.insert_or_assign(dst + "up_proj.bias", std::move(u));
      written += 2;
    }
  }
  // experts.down_proj -> <stacked>.down_proj.weight (its quantized form's
  // .weight / .scales / .biases alike), experts.down_proj_bias -> .bias
  keys.clear();
  for (const auto& [k, t] : weights) keys.push_back(k);
  static const std::pair<const char*, const char*> kDown[] = {
      {".experts.down_proj", ".weight"},         {".experts.down_proj.weight", ".weight"},
      {".experts.down_proj.scales", ".scales"}, {".experts.down_proj.biases", ".biases"},
      {".experts.down_proj_bias", ".bias"}};
  for (const std::string& k : keys) {
    if (k.rfind("model.layers.", 0) != 0) continue;
    for (const auto& [from, to] : kDown) {
      if (!ends_with(k, from)) continue;
      if (std::string(to) == ".bias" && !interleaved) continue;
      const std::string dst = k.substr(0, k.size() - std::strlen(from)) + "." + nm.stacked + ".down_proj" + to;
      if (dst == k) continue;  // (GPT-OSS: already the stacked name)
      auto it = weights.find(k);
      HostTensor t = std::move(it->second);
      weights.erase(it);
      weights.insert_or_assign(dst, std::move(t));
      ++written;
    }
  }
  return written;
}

HostTensor stack(const std::vector<const HostTensor*>& parts, const std::string& what) {
  const HostTensor& first = *parts.front();
  HostTensor out;
  out.dtype = first.dtype;
  out.shape.push_back(static_cast<int32_t>(parts.size()));
  out.shape.insert(out.shape.end(), first.shape.begin(), first.shape.end());
  out.nbytes = first.nbytes * parts.size();
  std::shared_ptr<uint8_t> buf(new uint8_t[out.nbytes > 0 ? out.nbytes : 1], std::default_delete<uint8_t[]>());
  for (size_t e = 0; e < parts.size(); ++e) {
    if (parts[e]->dtype != first.dtype || parts[e]->shape != first.shape)
      throw std::invalid_argument(what + ": expert " + std::to_string(e) + " differs in dtype or shape");
    if (first.nbytes) std::memcpy(buf.get() + e * first.nbytes, parts[e]->data, first.nbytes);
  }
  out.data = buf.get();
  out.owner = std::shared_ptr<const void>(buf, buf.get());
  return out;
}

}  // namespace

int sanitize_moe_experts(HostTensors& weights, const Json& config) {
  const MoeNaming& nm = moe_naming(config.at("model_type").str());
  const int64_t E = text_config(config).value(nm.experts_key, int64_t{nm.experts_default});
  if (E <= 0) throw std::invalid_argument("config: " + nm.experts_key + " is missing or not positive");
  const int split = sanitize_fused(weights, nm);
  // layers that hold per-expert tensors: "model.layers.<l>.<block>.experts.0.<proj>.<suffix>"
  const std::string head = "model.layers.", mid = "." + nm.block + ".experts.0.";
  std::set<std::string> layer_prefixes;  // "model.layers.<l>.<block>."
  for (const auto& [name, t] : weights) {
    if (name.compare(0, head.size(), head) != 0) continue;
    const size_t pos = name.find(mid);
    if (pos == std::string::npos) continue;
    const std::string layer = name.substr(head.size(), pos - head.size());
    if (layer.empty() || layer.find_first_not_of("0123456789") != std::string::npos) continue;
    layer_prefixes.insert(name.substr(0, pos + 1 + nm.block.size() + 1));
  }
  int stacked = 0;
  for (const std::string& pre : layer_prefixes) {
    for (const auto& [src, dst] : nm.projs) {
      for (const char* suffix : {"weight", "scales", "biases"}) {
        const std::string key0 = pre + "experts.0." + src + "." + suffix;
        if (!weights.count(key0)) continue;
        std::vector<const HostTensor*> parts;
        std::vector<std::string> keys;
        for (int64_t e = 0; e < E; ++e) {
          const std::string k = pre + "experts." + std::to_string(e) + "." + src + "." + suffix;
          const auto it = weights.find(k);
          if (it == weights.end()) throw std::invalid_argument("sanitize: missing " + k);
          parts.push_back(&it->second);
          keys.push_back(k);
        }
        HostTensor s = stack(parts, pre + "switch_mlp." + dst + "." + suffix);
        for (const std::string& k : keys) weights.erase(k);
        weights.insert_or_assign(pre + "switch_mlp." + dst + "." + suffix, std::move(s));
        ++stacked;
      }
    }
  }
  return stacked + split;
}

void register_quantized_weights(std::unordered_map<std::string, array>& weights,
                                const std::optional<PerLayerQuantization>& quantization,
                                const std::unordered_map<std::string, array*>& weight_map) {
  if (!quantization || !quantization->default_quantization) return;
  const Quantization dq = *quantization->default_quantization;
  static const std::string suffix = ".scales";
  std::vector<std::string> prefixes;
  for (const auto& [key, v] : weights) {
    if (key.size() > suffix.size() && key.compare(key.size() - suffix.size(), suffix.size(), suffix) == 0) {
      const std::string p = key.substr(0, key.size() - suffix.size());
      if (weights.count(p + ".weight")) prefixes.push_back(p);
    }
  }
  auto& reg = QuantizedWeightRegistry::instance();
  for (const std::string& p : prefixes) {
    if (p.find("embed") != std::string::npos) continue;  // dequantized at load by the reference
    // a skip entry leaves the defaults, as quantize_utils.cpp:54-60 does
    const std::optional<Quantization> lq = quantization->quantization_for(p);
    const Quantization q = lq ? *lq : dq;
    const auto wm = weight_map.find(p + ".weight");
    if (wm == weight_map.end()) continue;  // no member to register: scales stay, as in the reference
    const auto bit = weights.find(p + ".biases");
    std::optional<array> biases;
    if (bit != weights.end()) {
      biases = bit->second;
      weights.erase(bit);
    }
    reg.register_weight(wm->second, weights.at(p + ".scales"), biases, q.group_size, q.bits);
    weights.erase(p + ".scales");
  }
}

int load_weights(const std::unordered_map<std::string, array>& weights,
                 const std::unordered_map<std::string, array*>& weight_map) {
  int n = 0;
  for (const auto& [name, target] : weight_map) {
    const auto it = weights.find(name);
    if (it != weights.end()) {
      *target = it->second;
      ++n;
    }
  }
  return n;
}

}  // namespace mi355x
}  // namespace mlx_lm
