// test_switch_layers.cpp -- tests of the C++ host classes (SwitchLinear,
// SwitchGLU, gather_sort, scatter_unsort, moe_route, QuantizedWeightRegistry)
// in lemon-mlx-engine_amd/host/switch_layers.hpp.
//
//   test_switch_layers cpu   interface checks that touch no device: weight_map
//                            keys, registry semantics, status -> exception
//                            mapping, argument validation
//   test_switch_layers gpu   forward passes on the MI355X against the CPU
//                            checker (oracle/moe_oracle.h) on the same host
//                            buffers: routing and bucketing bit-exact, products
//                            within |a - b| <= 2e-2 + 1e-2 |b|
//   test_switch_layers dump DIR [sanitize]
//                            one line per tensor of the checkpoint directory
//                            (name, dtype, shape, CRC-32 of the bytes), after the
//                            MoE sanitize when asked; compared with the
//                            safetensors package by tests/test_host_cpp.py
//   test_switch_layers load-glu DIR LAYER IN OUT
//                            loads LAYER's experts from DIR into a SwitchGLU
//                            (read, sanitize, upload, register, load_weights),
//                            runs it on IN (int32 T, k; bf16 x [T, H]; uint32
//                            indices [T, k]) and writes y [T, k, H] bf16 to OUT
//
// The checker is test infrastructure; this program only compares against it.
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <numeric>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"
#include "moe_oracle.h"
#include "quantize_utils.hpp"
#include "safetensors.hpp"
#include "switch_layers.hpp"

using namespace mlx_lm::mi355x;

namespace {

struct Case {
  const char* name;
  const char* group;
  std::function<void()> fn;
};
std::vector<Case>& cases() {
  static std::vector<Case> c;
  return c;
}
struct Reg {
  Reg(const char* n, const char* g, std::function<void()> f) { cases().push_back({n, g, std::move(f)}); }
};
#define TEST_CASE(name, group)                     \
  static void name();                              \
  static Reg reg_##name(#name, group, name);       \
  static void name()

struct Failure : std::runtime_error {
  using std::runtime_error::runtime_error;
};
#define REQUIRE(cond)                                                                              \
  do {                                                                                             \
    if (!(cond)) throw Failure(std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond); \
  } while (0)
#define REQUIRE_THROWS_AS(expr, type)  \
  do {                                 \
    bool thrown_ = false;              \
    try {                              \
      expr;                            \
    } catch (const type&) {            \
      thrown_ = true;                  \
    }                                  \
    REQUIRE(thrown_ && #type);         \
  } while (0)

float bf2f(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Benchmark tolerance, elementwise.
void require_close(const std::vector<uint16_t>& got, const std::vector<uint16_t>& ref, const char* what) {
  REQUIRE(got.size() == ref.size());
  size_t bad = 0;
  double worst = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double g = bf2f(got[i]), r = bf2f(ref[i]);
    const double err = std::fabs(g - r);
    worst = std::max(worst, err);
    if (!(err <= 2e-2 + 1e-2 * std::fabs(r))) ++bad;
  }
  if (bad) {
    std::printf("  %s: %zu of %zu values outside tolerance (max abs err %.4g)\n", what, bad, got.size(), worst);
    REQUIRE(bad == 0);
  }
}

template <class T>
std::vector<T> download(const array& a) {
  std::vector<T> v(a.size());
  a.to_host(v.data());
  return v;
}

// ---- synthetic quantized expert weights (the library's seeded generator and MLX affine quantizer)
struct HostQ {
  int E, N, K, gs, bits;
  std::vector<uint32_t> w;
  std::vector<uint16_t> s, b;
  oracle_qweight o() const { return {w.data(), s.data(), b.data(), E, N, K, gs, bits, nullptr}; }
};

HostQ make_q(uint64_t seed, uint64_t tid, int E, int N, int K, int bits, int gs = 64) {
  HostQ q{E, N, K, gs, bits, {}, {}, {}};
  std::vector<uint16_t> dense(static_cast<size_t>(E) * N * K);
  REQUIRE(moe_synth_normal_bf16(seed, tid, 0.0f, 0.02f, 0, static_cast<int64_t>(dense.size()), dense.data()) == 0);
  q.w.resize(static_cast<size_t>(E) * N * K * bits / 32);
  q.s.resize(static_cast<size_t>(E) * N * K / gs);
  q.b.resize(q.s.size());
  REQUIRE(moe_quantize_affine(dense.data(), static_cast<int64_t>(E) * N, K, gs, bits, q.w.data(), q.s.data(),
                              q.b.data()) == 0);
  return q;
}

std::vector<uint16_t> make_x(uint64_t seed, size_t n) {
  std::vector<uint16_t> x(n);
  REQUIRE(moe_synth_normal_bf16(seed, 100, 0.0f, 1.0f, 0, static_cast<int64_t>(n), x.data()) == 0);
  return x;
}

// distinct experts per token, deterministic
std::vector<uint32_t> make_inds(int T, int k, int E, uint32_t seed) {
  std::vector<uint32_t> inds(static_cast<size_t>(T) * k);
  uint64_t st = seed * 0x9E3779B97F4A7C15ull + 1;
  for (int t = 0; t < T; ++t) {
    std::set<uint32_t> used;
    for (int j = 0; j < k; ++j) {
      uint32_t e;
      do {
        st = st * 6364136223846793005ull + 1442695040888963407ull;
        e = static_cast<uint32_t>((st >> 33) % static_cast<uint64_t>(E));
      } while (used.count(e));
      used.insert(e);
      inds[static_cast<size_t>(t) * k + j] = e;
    }
  }
  return inds;
}

void load(SwitchLinear& lin, const HostQ& q) {
  array w = array::from_host(q.w.data(), {q.E, q.N, q.K * q.bits / 32}, Dtype::uint32);
  array s = array::from_host(q.s.data(), {q.E, q.N, q.K / q.gs}, Dtype::bfloat16);
  array b = array::from_host(q.b.data(), {q.E, q.N, q.K / q.gs}, Dtype::bfloat16);
  lin.adopt_fused_weight(w, s, b, q.gs, q.bits);
}

// The loader's path: assign through weight_map, then register the quant metadata.
void load_glu(SwitchGLU& glu, const HostQ& g, const HostQ& u, const HostQ& d) {
  auto map = glu.weight_map();
  const std::pair<const char*, const HostQ*> parts[3] = {{"gate_proj", &g}, {"up_proj", &u}, {"down_proj", &d}};
  for (const auto& [name, q] : parts) {
    array* w = map.at(std::string(name) + ".weight");
    *w = array::from_host(q->w.data(), {q->E, q->N, q->K * q->bits / 32}, Dtype::uint32);
    QuantizedWeightRegistry::instance().register_weight(
        w, array::from_host(q->s.data(), {q->E, q->N, q->K / q->gs}, Dtype::bfloat16),
        array::from_host(q->b.data(), {q->E, q->N, q->K / q->gs}, Dtype::bfloat16), q->gs, q->bits);
  }
}

std::vector<uint16_t> ref_gather_qmm(const std::vector<uint16_t>& x, const HostQ& q, const uint32_t* lhs,
                                     const std::vector<uint32_t>& rhs, int M = 1) {
  std::vector<uint16_t> out(rhs.size() * M * q.N);
  const oracle_qweight o = q.o();
  REQUIRE(oracle_gather_qmm(x.data(), &o, lhs, rhs.data(), static_cast<int64_t>(rhs.size()), M, out.data()) == 0);
  return out;
}

std::vector<uint16_t> add_bias(std::vector<uint16_t> y, const std::vector<uint16_t>& bias,
                               const std::vector<uint32_t>& rhs, int N) {
  for (size_t r = 0; r < rhs.size(); ++r)
    for (int c = 0; c < N; ++c) {
      uint16_t& v = y[r * N + c];
      v = f2bf(bf2f(v) + bf2f(bias[static_cast<size_t>(rhs[r]) * N + c]));
    }
  return y;
}

// ============================================================ cpu
TEST_CASE(weight_map_keys, "cpu") {
  SwitchLinear a(64, 32, 4);
  auto m = a.weight_map();
  REQUIRE(m.size() == 1 && m.count("weight"));
  SwitchLinear b(64, 32, 4, true);
  m = b.weight_map();
  REQUIRE(m.size() == 2 && m.count("weight") && m.count("bias"));
  SwitchGLU g(64, 128, 4);
  auto gm = g.weight_map();
  REQUIRE(gm.size() == 3);
  for (const char* k : {"gate_proj.weight", "up_proj.weight", "down_proj.weight"}) REQUIRE(gm.count(k));
  SwitchGLU gb(64, 128, 4, true);
  REQUIRE(gb.weight_map().size() == 6 && gb.weight_map().count("down_proj.bias"));
  REQUIRE(a.output_dims() == 32 && a.num_experts() == 4);
}

TEST_CASE(registry_semantics, "cpu") {
  auto& reg = QuantizedWeightRegistry::instance();
  reg.clear();
  SwitchLinear a(64, 32, 4);
  const array* key = &a.weight();
  REQUIRE(reg.find(key) == nullptr);
  reg.register_weight(key, array(), std::nullopt, 64, 4);
  REQUIRE(reg.size() == 1 && reg.find(key) && reg.find(key)->bits == 4 && !reg.find(key)->biases);
  reg.register_weight(key, array(), array(), 128, 8);  // insert_or_assign
  REQUIRE(reg.size() == 1 && reg.find(key)->group_size == 128 && reg.find(key)->biases.has_value());
  a.release_weight();
  REQUIRE(reg.find(key) == nullptr && reg.size() == 0);
  reg.clear();
}

TEST_CASE(status_to_exception, "cpu") {
  check_status(MOE_OK, "ok");
  REQUIRE_THROWS_AS(check_status(MOE_E_INVALID_ARG, "x"), std::invalid_argument);
  REQUIRE_THROWS_AS(check_status(MOE_E_UNSUPPORTED, "x"), std::invalid_argument);
  REQUIRE_THROWS_AS(check_status(MOE_E_INDEX, "x"), std::invalid_argument);
  REQUIRE_THROWS_AS(check_status(MOE_E_WORKSPACE, "x"), std::runtime_error);
  REQUIRE_THROWS_AS(check_status(MOE_E_HIP, "x"), std::runtime_error);
  bool logic = false;
  try {
    check_status(MOE_E_HIP, "x");
  } catch (const std::invalid_argument&) {
    logic = true;
  } catch (const std::runtime_error&) {
  }
  REQUIRE(!logic);
}

TEST_CASE(validation_before_device, "cpu") {
  // zero-sized arrays hold no device memory: every check below runs on the host
  SwitchLinear lin(64, 32, 4);
  array x({0, 1, 64}, Dtype::bfloat16), idx({0}, Dtype::uint32);
  REQUIRE_THROWS_AS(lin(x, idx), std::invalid_argument);  // neither quantized nor a loaded bf16 [E, N, K] weight
  QuantizedWeightRegistry::instance().register_weight(&lin.weight(), array(), std::nullopt, 64, 4);
  REQUIRE_THROWS_AS(lin(x, idx), std::invalid_argument);  // weight not loaded
  QuantizedWeightRegistry::instance().clear();
  SwitchGLU glu(64, 128, 4);
  REQUIRE_THROWS_AS(glu(array({0, 63}, Dtype::bfloat16), array({0, 2}, Dtype::uint32)), std::invalid_argument);
  REQUIRE_THROWS_AS(glu(array({0, 64}, Dtype::float32), array({0, 2}, Dtype::uint32)), std::invalid_argument);
  REQUIRE_THROWS_AS(glu(array({0, 64}, Dtype::bfloat16), array({1, 0, 2}, Dtype::uint32)), std::invalid_argument);
  REQUIRE_THROWS_AS(gather_sort(array({0, 1, 64}, Dtype::bfloat16), array({0, 2}, Dtype::float32)),
                    std::invalid_argument);
  REQUIRE_THROWS_AS(moe_route(array({0, 8}, Dtype::float32), 2), std::invalid_argument);
  REQUIRE_THROWS_AS(array({0, 4}, Dtype::bfloat16).reshape({5}), std::invalid_argument);
  REQUIRE_THROWS_AS(SwitchLinear(0, 32, 4), std::invalid_argument);
}

// ---- checkpoint reading (json.hpp, safetensors.hpp, quantize_utils.hpp) -----------
TEST_CASE(json_reader, "cpu") {
  const Json j = parse_json(
      " {\"a\": [1, -2.5e-1, true, false, null, \"x\\u00e9\\n\\\"\"], \"b\": {\"c\": 3, \"d\": {}}, \"e\": []} ");
  REQUIRE(j.is_object() && j.fields().size() == 3);
  const auto& a = j.at("a").items();
  REQUIRE(a.size() == 6 && a[0].integer() == 1 && a[1].num() == -0.25 && a[2].boolean() && !a[3].boolean());
  REQUIRE(a[4].is_null() && a[5].str() == "x\xc3\xa9\n\"");
  REQUIRE(j.at("b").value("c", int64_t{0}) == 3 && j.at("b").value("zz", int64_t{7}) == 7);
  REQUIRE(j.at("b").at("d").fields().empty() && j.at("e").items().empty());
  REQUIRE(parse_json("\"\\ud83d\\ude00\"").str() == "\xf0\x9f\x98\x80");  // surrogate pair
  REQUIRE_THROWS_AS(a[1].integer(), std::invalid_argument);
  REQUIRE_THROWS_AS(j.at("missing"), std::invalid_argument);
  REQUIRE_THROWS_AS(j.at("a").str(), std::invalid_argument);
  for (const char* badj : {"{\"a\":}", "[1, 2", "\"abc", "{} x", "{\"a\" 1}", "[1,]", "tru", "\"\\q\"", ""})
    REQUIRE_THROWS_AS(parse_json(badj), std::invalid_argument);
  REQUIRE_THROWS_AS(parse_json(std::string(100, '[') + std::string(100, ']')), std::invalid_argument);
}

TEST_CASE(quantization_config, "cpu") {
  // base_config.cpp:28-73: defaults, per-prefix objects, false = skip, the VLM prefix stripped
  const Json c = parse_json(R"({"quantization": {"group_size": 32, "bits": 4, "mode": "affine",
      "language_model.model.layers.0.mlp.gate": {"group_size": 64, "bits": 8},
      "model.layers.1.mlp.gate": false, "model.layers.2.mlp.gate": {"bits": 6}}})");
  const auto q = parse_quantization(c);
  REQUIRE(q && q->default_quantization && q->default_quantization->group_size == 32);
  REQUIRE(q->per_layer.size() == 3 && !q->per_layer.count("mode"));
  const auto q0 = q->quantization_for("model.layers.0.mlp.gate");
  REQUIRE(q0 && q0->bits == 8 && q0->group_size == 64);
  REQUIRE(!q->quantization_for("model.layers.1.mlp.gate"));  // skip
  const auto q2 = q->quantization_for("model.layers.2.mlp.gate");
  REQUIRE(q2 && q2->bits == 6 && q2->group_size == 32);  // group size from the defaults
  REQUIRE(q->quantization_for("model.layers.5.mlp.switch_mlp.up_proj")->bits == 4);
  REQUIRE(!parse_quantization(parse_json("{\"model_type\": \"qwen3_moe\"}")));
}

HostTensor host_tensor(const std::string& dt, Shape shape, size_t bytes, uint8_t fill) {
  auto buf = std::make_shared<std::vector<uint8_t>>(bytes);
  for (size_t i = 0; i < bytes; ++i) (*buf)[i] = static_cast<uint8_t>(fill + i);
  HostTensor t;
  t.dtype = dt;
  t.shape = std::move(shape);
  t.data = buf->data();
  t.nbytes = bytes;
  t.owner = buf;
  return t;
}

TEST_CASE(sanitize_stacks_experts, "cpu") {
  // deepseek_v3.cpp:531-555: experts.{e}.<proj>.{weight,scales,biases} -> switch_mlp.<proj> [E, ...]
  const int E = 3;
  HostTensors w;
  for (int l : {1, 3})
    for (int e = 0; e < E; ++e)
      for (const char* proj : {"gate_proj", "up_proj", "down_proj"}) {
        const std::string p = "model.layers." + std::to_string(l) + ".mlp.experts." + std::to_string(e) + "." + proj;
        w[p + ".weight"] = host_tensor("U32", {4, 2}, 32, static_cast<uint8_t>(16 * e + l));
        w[p + ".scales"] = host_tensor("BF16", {4, 1}, 8, static_cast<uint8_t>(100 + e));
      }
  w["model.layers.1.mlp.gate.weight"] = host_tensor("BF16", {E, 16}, 96, 0);
  w["model.layers.1.mlp.shared_experts.gate_proj.weight"] = host_tensor("U32", {8, 2}, 64, 0);
  const Json cfg = parse_json(R"({"model_type": "deepseek_v3", "n_routed_experts": 3})");
  REQUIRE(sanitize_moe_experts(w, cfg) == 12);
  REQUIRE(w.size() == 14);
  const HostTensor& g = w.at("model.layers.3.mlp.switch_mlp.gate_proj.weight");
  REQUIRE((g.shape == Shape{E, 4, 2}) && g.dtype == "U32" && g.nbytes == 96);
  for (int e = 0; e < E; ++e) REQUIRE(g.data[32 * e] == static_cast<uint8_t>(16 * e + 3) && g.data[32 * e + 31] == static_cast<uint8_t>(16 * e + 3 + 31));
  REQUIRE((w.at("model.layers.1.mlp.switch_mlp.down_proj.scales").shape == Shape{E, 4, 1}));
  REQUIRE(!w.count("model.layers.1.mlp.experts.0.up_proj.weight") && w.count("model.layers.1.mlp.gate.weight"));
  // a missing expert, and experts of different shapes, are errors
  HostTensors m;
  m["model.layers.0.mlp.experts.0.up_proj.weight"] = host_tensor("U32", {4, 2}, 32, 0);
  m["model.layers.0.mlp.experts.2.up_proj.weight"] = host_tensor("U32", {4, 2}, 32, 0);
  REQUIRE_THROWS_AS(sanitize_moe_experts(m, cfg), std::invalid_argument);
  m["model.layers.0.mlp.experts.1.up_proj.weight"] = host_tensor("U32", {2, 4}, 32, 0);
  REQUIRE_THROWS_AS(sanitize_moe_experts(m, cfg), std::invalid_argument);
  // phimoe.cpp:208-235: block_sparse_moe, w1/w3/w2 -> gate/up/down
  HostTensors ph;
  for (int e = 0; e < 2; ++e)
    for (const char* n : {"w1", "w2", "w3"})
      ph["model.layers.0.block_sparse_moe.experts." + std::to_string(e) + "." + n + ".weight"] =
          host_tensor("U32", {2, 2}, 16, static_cast<uint8_t>(n[1]));
  REQUIRE(sanitize_moe_experts(ph, parse_json(R"({"model_type": "phimoe", "num_local_experts": 2})")) == 3);
  REQUIRE(ph.at("model.layers.0.block_sparse_moe.switch_mlp.down_proj.weight").data[0] == '2');
  REQUIRE(ph.at("model.layers.0.block_sparse_moe.switch_mlp.up_proj.weight").data[0] == '3');
  REQUIRE_THROWS_AS(sanitize_moe_experts(ph, parse_json(R"({"model_type": "llama"})")), std::invalid_argument);
}

TEST_CASE(sanitize_fused_gate_up, "cpu") {
  // fused [E, 2I, H] gate_up_proj: BF16 E = 2, 2I = 4, H = 2 -> byte (e, r, c, b) = fill + ((e*4+r)*2+c)*2+b
  auto first_byte = [](const HostTensor& t, int e, int r) { return t.data[(static_cast<size_t>(e) * t.shape[1] + r) * 4]; };
  // GPT-OSS (gptoss.cpp:305-350): even rows -> gate, odd -> up; the bias [E, 2I] alike; down renamed
  {
    HostTensors w;
    const std::string p = "model.layers.0.mlp.experts.";
    w[p + "gate_up_proj"] = host_tensor("BF16", {2, 4, 2}, 32, 0);
    w[p + "gate_up_proj_bias"] = host_tensor("BF16", {2, 4}, 16, 100);
    w[p + "down_proj"] = host_tensor("BF16", {2, 2, 2}, 16, 50);
    w[p + "down_proj_bias"] = host_tensor("BF16", {2, 2}, 8, 70);
    w["model.layers.0.mlp.router.weight"] = host_tensor("BF16", {2, 2}, 8, 0);
    const Json cfg = parse_json(R"({"model_type": "gpt_oss", "num_local_experts": 2})");
    REQUIRE(sanitize_moe_experts(w, cfg) == 6);
    const HostTensor& g = w.at(p + "gate_proj.weight");
    const HostTensor& u = w.at(p + "up_proj.weight");
    REQUIRE((g.shape == Shape{2, 2, 2}) && (u.shape == Shape{2, 2, 2}) && g.nbytes == 16);
    for (int e = 0; e < 2; ++e)
      for (int r = 0; r < 2; ++r) {
        REQUIRE(first_byte(g, e, r) == static_cast<uint8_t>(((e * 4 + 2 * r) * 2) * 2));
        REQUIRE(first_byte(u, e, r) == static_cast<uint8_t>(((e * 4 + 2 * r + 1) * 2) * 2));
      }
    const HostTensor& gb = w.at(p + "gate_proj.bias");
    const HostTensor& ub = w.at(p + "up_proj.bias");
    REQUIRE((gb.shape == Shape{2, 2}) && gb.data[2] == 100 + 4 && ub.data[0] == 100 + 2 && ub.data[6] == 100 + 14);
    REQUIRE(w.at(p + "down_proj.weight").data[0] == 50 && w.at(p + "down_proj.bias").data[0] == 70);
    REQUIRE(!w.count(p + "gate_up_proj") && !w.count(p + "down_proj") && w.size() == 7);
    // a checkpoint that already holds gate_proj.weight is left alone (gptoss.cpp:307-312)
    HostTensors done;
    done[p + "gate_proj.weight"] = host_tensor("U32", {2, 2, 1}, 16, 0);
    done[p + "gate_up_proj"] = host_tensor("BF16", {2, 4, 2}, 32, 0);
    REQUIRE(sanitize_moe_experts(done, cfg) == 0 && done.count(p + "gate_up_proj"));
  }
  // Qwen3.5-MoE (qwen35_moe.cpp:1046-1107): VLM names, halves, down_proj -> switch_mlp; the
  // quantized form (.weight / .scales / .biases) split alike
  {
    HostTensors w;
    w["language_model.model.layers.1.mlp.experts.gate_up_proj"] = host_tensor("BF16", {2, 4, 2}, 32, 0);
    w["model.language_model.layers.2.mlp.experts.gate_up_proj.weight"] = host_tensor("U32", {2, 4, 1}, 32, 0);
    w["model.language_model.layers.2.mlp.experts.gate_up_proj.scales"] = host_tensor("BF16", {2, 4, 1}, 16, 9);
    w["language_model.model.layers.1.mlp.experts.down_proj"] = host_tensor("BF16", {2, 2, 2}, 16, 50);
    w["vision_tower.blocks.0.weight"] = host_tensor("BF16", {2}, 4, 0);
    w["language_model.model.layers.1.mlp.shared_expert_gate.weight"] = host_tensor("BF16", {1, 2}, 4, 0);
    const Json cfg = parse_json(R"({"model_type": "qwen3_5_moe", "text_config": {"num_experts": 2}})");
    REQUIRE(sanitize_moe_experts(w, cfg) == 7);
    const HostTensor& g = w.at("model.layers.1.mlp.switch_mlp.gate_proj.weight");
    const HostTensor& u = w.at("model.layers.1.mlp.switch_mlp.up_proj.weight");
    for (int e = 0; e < 2; ++e)
      for (int r = 0; r < 2; ++r) {
        REQUIRE(first_byte(g, e, r) == static_cast<uint8_t>(((e * 4 + r) * 2) * 2));
        REQUIRE(first_byte(u, e, r) == static_cast<uint8_t>(((e * 4 + 2 + r) * 2) * 2));
      }
    const HostTensor& us = w.at("model.layers.2.mlp.switch_mlp.up_proj.scales");
    REQUIRE((us.shape == Shape{2, 2, 1}) && us.data[0] == 9 + 4 && us.data[4] == 9 + 12);
    REQUIRE(w.count("model.layers.2.mlp.switch_mlp.gate_proj.weight") && w.count("model.layers.1.mlp.switch_mlp.down_proj.weight"));
    REQUIRE(w.count("model.layers.1.mlp.shared_expert_gate.weight") && !w.count("vision_tower.blocks.0.weight"));
    REQUIRE(w.size() == 8);
    REQUIRE(text_config(cfg).value("num_experts", int64_t{0}) == 2);
  }
}

TEST_CASE(register_quantized_weights_semantics, "cpu") {
  // quantize_utils.cpp:14-104 on arrays without device data
  auto& reg = QuantizedWeightRegistry::instance();
  reg.clear();
  SwitchGLU glu(64, 128, 4);
  std::unordered_map<std::string, array*> wm;
  for (auto& [k, v] : glu.weight_map()) wm["model.layers.0.mlp.switch_mlp." + k] = v;
  std::unordered_map<std::string, array> w;
  const std::string p = "model.layers.0.mlp.switch_mlp.";
  for (const char* n : {"gate_proj", "up_proj", "down_proj"}) {
    w[p + n + ".weight"] = array();
    w[p + n + ".scales"] = array();
  }
  w[p + "gate_proj.biases"] = array();
  w["model.layers.0.mlp.gate.weight"] = array();  // not quantized
  w["model.layers.0.mlp.shared_experts.up_proj.weight"] = array();  // quantized, not a member
  w["model.layers.0.mlp.shared_experts.up_proj.scales"] = array();
  w["model.embed_tokens.weight"] = array();
  w["model.embed_tokens.scales"] = array();
  const Json cfg = parse_json(R"({"quantization": {"group_size": 64, "bits": 4,
      "model.layers.0.mlp.switch_mlp.down_proj": {"group_size": 32, "bits": 8}}})");
  register_quantized_weights(w, parse_quantization(cfg), wm);
  REQUIRE(reg.size() == 3);
  const QuantizationInfo* g = reg.find(wm.at(p + "gate_proj.weight"));
  REQUIRE(g && g->bits == 4 && g->group_size == 64 && g->biases.has_value());
  const QuantizationInfo* d = reg.find(wm.at(p + "down_proj.weight"));
  REQUIRE(d && d->bits == 8 && d->group_size == 32 && !d->biases.has_value());
  REQUIRE(!w.count(p + "gate_proj.scales") && !w.count(p + "gate_proj.biases") && w.count(p + "gate_proj.weight"));
  REQUIRE(w.count("model.layers.0.mlp.shared_experts.up_proj.scales"));  // no member: kept
  REQUIRE(w.count("model.embed_tokens.scales"));
  REQUIRE(load_weights(w, wm) == 3);
  reg.clear();
  std::unordered_map<std::string, array> w2 = {{p + "up_proj.weight", array()}, {p + "up_proj.scales", array()}};
  register_quantized_weights(w2, std::nullopt, wm);  // no quantization entry: nothing registered
  REQUIRE(reg.size() == 0 && w2.size() == 2);
}

struct TempDir {
  std::filesystem::path path;
  TempDir() {
    path = std::filesystem::temp_directory_path() / ("moe_ckpt_" + std::to_string(::getpid()));
    std::filesystem::remove_all(path);
    std::filesystem::create_directories(path);
  }
  ~TempDir() { std::filesystem::remove_all(path); }
  std::string file(const std::string& name, const std::string& bytes) const {
    const std::string p = (path / name).string();
    std::ofstream(p, std::ios::binary) << bytes;
    return p;
  }
};

std::string st_file(const std::string& header, const std::string& data, int64_t len_override = -1) {
  std::string out(8, '\0');
  const uint64_t n = len_override >= 0 ? static_cast<uint64_t>(len_override) : header.size();
  for (int i = 0; i < 8; ++i) out[i] = static_cast<char>((n >> (8 * i)) & 0xff);
  return out + header + data;
}

TEST_CASE(safetensors_reader_and_resolution, "cpu") {
  TempDir d;
  const std::string data(24, 'x');
  const std::string good = d.file(
      "a.safetensors", st_file(R"({"__metadata__": {"format": "mlx"}, "w": {"dtype": "U32", "shape": [2, 2],
          "data_offsets": [0, 16]}, "s": {"dtype": "BF16", "shape": [], "data_offsets": [16, 18]},
          "z": {"dtype": "F32", "shape": [0, 3], "data_offsets": [18, 18]}})", data));
  const HostTensors t = read_safetensors(good);
  REQUIRE(t.size() == 3 && (t.at("w").shape == Shape{2, 2}) && t.at("w").nbytes == 16 && t.at("s").shape.empty());
  REQUIRE(t.at("z").nbytes == 0 && t.at("s").numel() == 1);
  REQUIRE(crc32("123456789", 9) == 0xCBF43926u);  // the CRC-32 check value
  const std::string hdr = R"({"w": {"dtype": "U32", "shape": [2, 2], "data_offsets": [0, 16]}})";
  const std::vector<std::string> bad = {
      st_file(hdr, data, 1 << 20),                                                                // length past EOF
      st_file(R"({"w": {"dtype": "U32", "shape": [2, 2], "data_offsets": [0, 32]}})", data),   // past the data
      st_file(R"({"w": {"dtype": "U32", "shape": [2, 3], "data_offsets": [0, 16]}})", data),   // size mismatch
      st_file(R"({"w": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 2]}})", data),        // unknown dtype
      st_file(R"({"w": {"dtype": "U32", "shape": [-1], "data_offsets": [0, 0]}})", data),      // negative dim
      // element count past 2^64, and 2^62 four-byte elements (bytes wrap to 0 = the offsets' span)
      st_file(R"({"w": {"dtype": "U8", "shape": [2147483647, 2147483647, 2147483647], "data_offsets": [0, 0]}})",
              data),
      st_file(R"({"w": {"dtype": "U32", "shape": [1073741824, 1073741824, 4], "data_offsets": [0, 0]}})", data),
      st_file(R"({"w": {"shape": [2], "data_offsets": [0, 8]}})", data),                       // no dtype
      st_file(R"({"w": )", data),                                                                 // bad JSON
      std::string("abc")};                                                                        // too short
  for (size_t i = 0; i < bad.size(); ++i)
    REQUIRE_THROWS_AS(read_safetensors(d.file("bad" + std::to_string(i) + ".bin", bad[i])), std::invalid_argument);
  REQUIRE_THROWS_AS(read_safetensors((d.path / "nope.safetensors").string()), std::runtime_error);
  // resolution: *.safetensors fallback (a small model.safetensors stub does not count)
  d.file("model.safetensors", st_file("{}", ""));
  const std::string b = d.file("b.safetensors", st_file(hdr, data));
  auto files = safetensors_files(d.path.string());
  REQUIRE(files.size() == 3 && files[0] == good && files[1] == b);  // sorted; the stub is a *.safetensors too
  // an index wins and names the shards; a missing shard is an error
  d.file("model.safetensors.index.json", R"({"weight_map": {"w": "b.safetensors", "s": "a.safetensors"}})");
  files = safetensors_files(d.path.string());
  REQUIRE(files.size() == 2 && files[0] == good && files[1] == b);
  const HostTensors all = read_safetensors_from_directory(d.path.string());
  REQUIRE(all.size() == 3 && all.count("z") && all.at("w").nbytes == 16);
  REQUIRE(std::memcmp(all.at("w").data, data.data(), 16) == 0);
  d.file("model.safetensors.index.json", R"({"weight_map": {"w": "c.safetensors"}})");
  bool missing = false;
  try {
    safetensors_files(d.path.string());
  } catch (const std::runtime_error& e) {
    missing = std::string(e.what()).find("Missing shard file") != std::string::npos;
  }
  REQUIRE(missing);
  std::filesystem::remove(d.path / "model.safetensors.index.json");
  std::filesystem::remove(d.path / "a.safetensors");
  std::filesystem::remove(d.path / "b.safetensors");
  std::filesystem::remove(d.path / "model.safetensors");
  REQUIRE_THROWS_AS(safetensors_files(d.path.string()), std::runtime_error);
}

// ============================================================ gpu
// Qwen3-MoE style: SwitchGLU over quantized experts (fused path), tiny config and
// the Qwen3-30B-A3B shape at decode.
void glu_case(int T, int k, int E, int H, int I, int bits) {
  QuantizedWeightRegistry::instance().clear();
  const HostQ g = make_q(T + 1, 2, E, I, H, bits), u = make_q(T + 1, 3, E, I, H, bits),
              d = make_q(T + 1, 4, E, H, I, bits);
  SwitchGLU glu(H, I, E);
  load_glu(glu, g, u, d);
  const std::vector<uint16_t> x = make_x(T, static_cast<size_t>(T) * H);
  const std::vector<uint32_t> inds = make_inds(T, k, E, T + k);
  array xd = array::from_host(x.data(), {1, T, H}, Dtype::bfloat16);
  array id = array::from_host(inds.data(), {1, T, k}, Dtype::uint32);
  array y = glu(xd, id);
  REQUIRE((y.shape() == Shape{1, T, k, H}));
  std::vector<uint32_t> lhs(static_cast<size_t>(T) * k);
  for (size_t i = 0; i < lhs.size(); ++i) lhs[i] = static_cast<uint32_t>(i / k);
  const auto gg = ref_gather_qmm(x, g, lhs.data(), inds), uu = ref_gather_qmm(x, u, lhs.data(), inds);
  std::vector<uint16_t> h(gg.size());
  oracle_swiglu(gg.data(), uu.data(), static_cast<int64_t>(h.size()), h.data());
  require_close(download<uint16_t>(y), ref_gather_qmm(h, d, nullptr, inds), "SwitchGLU");
}

TEST_CASE(switch_glu_tiny, "gpu") { glu_case(16, 2, 8, 512, 1024, 4); }
TEST_CASE(switch_glu_qwen3_decode, "gpu") { glu_case(8, 8, 128, 2048, 768, 4); }
TEST_CASE(switch_glu_8bit, "gpu") { glu_case(40, 4, 6, 256, 512, 8); }
TEST_CASE(switch_glu_6bit, "gpu") { glu_case(40, 4, 6, 256, 512, 6); }  // examples/convert.cpp:10 --bits 6

// GPT-OSS style (gptoss.cpp:129-168): SwitchLinear with linear biases called
// directly, with gather_sort / scatter_unsort when there are >= 64 pairs, and
// GPT-OSS's clipped SwiGLU called as swiglu(x_gate, x_up) (:158).  The gate
// and up biases are N(0, 4), so the activation's inputs straddle -7 and +7.
void gptoss_case(int T, int k) {
  QuantizedWeightRegistry::instance().clear();
  const int E = 8, H = 256, I = 512;
  const HostQ g = make_q(7, 2, E, I, H, 4), u = make_q(7, 3, E, I, H, 4), d = make_q(7, 4, E, H, I, 4);
  SwitchLinear gate(H, I, E, true), up(H, I, E, true), down(I, H, E, true);
  load(gate, g);
  load(up, u);
  load(down, d);
  std::vector<uint16_t> bg(E * I), bu(E * I), bd(E * H);
  REQUIRE(moe_synth_normal_bf16(7, 10, 0.0f, 4.0f, 0, E * I, bg.data()) == 0);
  REQUIRE(moe_synth_normal_bf16(7, 11, 0.0f, 4.0f, 0, E * I, bu.data()) == 0);
  REQUIRE(moe_synth_normal_bf16(7, 12, 0.0f, 0.1f, 0, E * H, bd.data()) == 0);
  *gate.weight_map().at("bias") = array::from_host(bg.data(), {E, I}, Dtype::bfloat16);
  *up.weight_map().at("bias") = array::from_host(bu.data(), {E, I}, Dtype::bfloat16);
  *down.weight_map().at("bias") = array::from_host(bd.data(), {E, H}, Dtype::bfloat16);

  const std::vector<uint16_t> x = make_x(T + 50, static_cast<size_t>(T) * H);
  const std::vector<uint32_t> inds = make_inds(T, k, E, T);
  array x_exp = array::from_host(x.data(), {1, T, 1, 1, H}, Dtype::bfloat16);
  array stop_inds = array::from_host(inds.data(), {1, T, k}, Dtype::uint32);
  const bool do_sort = static_cast<int>(inds.size()) >= 64;
  array idx = stop_inds, inverse_order;
  if (do_sort) {
    auto [sx, si, io] = gather_sort(x_exp, stop_inds, E);
    x_exp = sx;
    idx = si;
    inverse_order = io;
  }
  array x_up = up(x_exp, idx, do_sort);
  array x_gate = gate(x_exp, idx, do_sort);
  array act = gptoss_swiglu(x_gate, x_up);
  array result = down(act, idx, do_sort);
  if (do_sort) {
    Shape s = stop_inds.shape();
    result = scatter_unsort(result, inverse_order, &s);
  }
  REQUIRE((result.shape() == Shape{1, T, k, 1, H}));

  std::vector<uint32_t> lhs(inds.size());
  for (size_t i = 0; i < lhs.size(); ++i) lhs[i] = static_cast<uint32_t>(i / k);
  const auto gg = add_bias(ref_gather_qmm(x, g, lhs.data(), inds), bg, inds, I);
  const auto uu = add_bias(ref_gather_qmm(x, u, lhs.data(), inds), bu, inds, I);
  size_t clipped = 0;
  for (size_t i = 0; i < gg.size(); ++i) clipped += std::fabs(bf2f(gg[i])) > 7.0f || bf2f(uu[i]) > 7.0f;
  REQUIRE(clipped > gg.size() / 50);  // the clip limits are exercised
  std::vector<uint16_t> h(gg.size());
  oracle_gptoss_swiglu(gg.data(), uu.data(), static_cast<int64_t>(h.size()), h.data(), nullptr);
  if (!do_sort) require_close(download<uint16_t>(act), h, "GPT-OSS swiglu");  // (sorted: in bucket order)
  require_close(download<uint16_t>(result), add_bias(ref_gather_qmm(h, d, nullptr, inds), bd, inds, H),
                "GPT-OSS experts");
}

// Dense (bf16) experts: a weight that is not registered as quantized takes
// SwitchLinear's gather_mm branch (switch_layers.cpp:103-109), with its bias.
void dense_case(int T, int k) {
  QuantizedWeightRegistry::instance().clear();
  const int E = 8, H = 256, I = 512;
  std::vector<uint16_t> wg(static_cast<size_t>(E) * I * H), wu(wg.size()), wd(static_cast<size_t>(E) * H * I);
  REQUIRE(moe_synth_normal_bf16(9, 2, 0.0f, 0.02f, 0, static_cast<int64_t>(wg.size()), wg.data()) == 0);
  REQUIRE(moe_synth_normal_bf16(9, 3, 0.0f, 0.02f, 0, static_cast<int64_t>(wu.size()), wu.data()) == 0);
  REQUIRE(moe_synth_normal_bf16(9, 4, 0.0f, 0.02f, 0, static_cast<int64_t>(wd.size()), wd.data()) == 0);
  std::vector<uint16_t> bd(static_cast<size_t>(E) * H);
  REQUIRE(moe_synth_normal_bf16(9, 12, 0.0f, 0.1f, 0, E * H, bd.data()) == 0);
  SwitchLinear gate(H, I, E), up(H, I, E), down(I, H, E, true);
  *gate.weight_map().at("weight") = array::from_host(wg.data(), {E, I, H}, Dtype::bfloat16);
  *up.weight_map().at("weight") = array::from_host(wu.data(), {E, I, H}, Dtype::bfloat16);
  *down.weight_map().at("weight") = array::from_host(wd.data(), {E, H, I}, Dtype::bfloat16);
  *down.weight_map().at("bias") = array::from_host(bd.data(), {E, H}, Dtype::bfloat16);

  const std::vector<uint16_t> x = make_x(T + 60, static_cast<size_t>(T) * H);
  const std::vector<uint32_t> inds = make_inds(T, k, E, T + 1);
  array x_exp = array::from_host(x.data(), {T, 1, 1, H}, Dtype::bfloat16);
  array idx = array::from_host(inds.data(), {T, k}, Dtype::uint32);
  array x_gate = gate(x_exp, idx), x_up = up(x_exp, idx);
  array act(x_gate.shape(), Dtype::bfloat16);
  check_status(moe_swiglu(x_gate.data<uint16_t>(), x_up.data<uint16_t>(), static_cast<int64_t>(act.size()),
                          act.data<uint16_t>(), nullptr),
               "swiglu");
  array result = down(act, idx);
  REQUIRE((result.shape() == Shape{T, k, 1, H}));

  std::vector<uint32_t> lhs(inds.size());
  for (size_t i = 0; i < lhs.size(); ++i) lhs[i] = static_cast<uint32_t>(i / k);
  const int64_t P = static_cast<int64_t>(inds.size());
  std::vector<uint16_t> gg(P * I), uu(P * I), h(P * I), ref(P * H);
  REQUIRE(oracle_gather_mm(x.data(), wg.data(), nullptr, E, I, H, lhs.data(), inds.data(), P, 1, gg.data()) == 0);
  REQUIRE(oracle_gather_mm(x.data(), wu.data(), nullptr, E, I, H, lhs.data(), inds.data(), P, 1, uu.data()) == 0);
  oracle_swiglu(gg.data(), uu.data(), P * I, h.data());
  REQUIRE(oracle_gather_mm(h.data(), wd.data(), bd.data(), E, H, I, nullptr, inds.data(), P, 1, ref.data()) == 0);
  require_close(download<uint16_t>(result), ref, "dense experts");
}

TEST_CASE(switch_linear_dense, "gpu") { dense_case(16, 2); }
TEST_CASE(switch_linear_dense_many_pairs, "gpu") { dense_case(300, 4); }

TEST_CASE(switch_linear_bias_unsorted, "gpu") { gptoss_case(16, 2); }   // 32 pairs: broadcast lhs
TEST_CASE(switch_linear_bias_sorted, "gpu") { gptoss_case(100, 4); }    // 400 pairs: gather_sort path

TEST_CASE(switch_glu_with_linear_bias, "gpu") {
  // SwitchGLU(bias=true) takes the per-projection path; biases of zero make it
  // equal to the fused path on the same experts
  QuantizedWeightRegistry::instance().clear();
  const int T = 24, k = 4, E = 8, H = 256, I = 512;
  const HostQ g = make_q(3, 2, E, I, H, 4), u = make_q(3, 3, E, I, H, 4), d = make_q(3, 4, E, H, I, 4);
  SwitchGLU fused(H, I, E), biased(H, I, E, true);
  load_glu(fused, g, u, d);
  load_glu(biased, g, u, d);
  std::vector<uint16_t> zi(E * I, 0), zh(E * H, 0);
  auto bm = biased.weight_map();
  *bm.at("gate_proj.bias") = array::from_host(zi.data(), {E, I}, Dtype::bfloat16);
  *bm.at("up_proj.bias") = array::from_host(zi.data(), {E, I}, Dtype::bfloat16);
  *bm.at("down_proj.bias") = array::from_host(zh.data(), {E, H}, Dtype::bfloat16);
  const auto x = make_x(5, static_cast<size_t>(T) * H);
  const auto inds = make_inds(T, k, E, 5);
  array xd = array::from_host(x.data(), {2, T / 2, H}, Dtype::bfloat16);
  array id = array::from_host(inds.data(), {2, T / 2, k}, Dtype::uint32);
  const auto a = download<uint16_t>(fused(xd, id));
  const auto b = download<uint16_t>(biased(xd, id));
  require_close(b, a, "SwitchGLU per-projection vs fused");
}

TEST_CASE(sorted_equals_unsorted, "gpu") {
  // gather_qmm invariance: sorting the pairs does not change any product
  QuantizedWeightRegistry::instance().clear();
  const int T = 50, k = 4, E = 16, H = 512, N = 256;
  const HostQ q = make_q(9, 2, E, N, H, 4);
  SwitchLinear lin(H, N, E);
  load(lin, q);
  const auto x = make_x(9, static_cast<size_t>(T) * H);
  const auto inds = make_inds(T, k, E, 9);
  array xe = array::from_host(x.data(), {T, 1, 1, H}, Dtype::bfloat16);
  array id = array::from_host(inds.data(), {T, k}, Dtype::uint32);
  const auto direct = download<uint16_t>(lin(xe, id, false));
  auto [sx, si, io] = gather_sort(xe, id, E);
  Shape s = id.shape();
  const auto via_sort = download<uint16_t>(scatter_unsort(lin(sx, si, true), io, &s));
  REQUIRE(direct == via_sort);
}

TEST_CASE(gather_sort_matches_checker, "gpu") {
  const int T = 300, k = 8, E = 128, H = 64;
  const auto x = make_x(11, static_cast<size_t>(T) * H);
  const auto inds = make_inds(T, k, E, 11);
  array xe = array::from_host(x.data(), {T, 1, 1, H}, Dtype::bfloat16);
  array id = array::from_host(inds.data(), {T, k}, Dtype::uint32);
  auto [sx, si, io] = gather_sort(xe, id, E);
  REQUIRE((sx.shape() == Shape{T * k, 1, H}));
  const size_t P = inds.size();
  std::vector<int32_t> perm(P), inv(P), offs(E + 1);
  std::vector<uint32_t> se(P);
  REQUIRE(oracle_bucket(inds.data(), T, k, E, perm.data(), inv.data(), se.data(), offs.data()) == 0);
  REQUIRE(download<uint32_t>(si) == se);
  const auto gi = download<uint32_t>(io);
  for (size_t i = 0; i < P; ++i) REQUIRE(gi[i] == static_cast<uint32_t>(inv[i]));
  const auto gx = download<uint16_t>(sx);
  for (size_t p = 0; p < P; ++p)
    REQUIRE(std::memcmp(&gx[p * H], &x[static_cast<size_t>(perm[p] / k) * H], H * 2) == 0);
}

TEST_CASE(moe_route_matches_checker, "gpu") {
  // gated_delta.h:117-119: top-k + softmax over the k selected (R4), bit-exact
  const int T = 33, E = 512, k = 10;
  std::vector<uint16_t> lg(static_cast<size_t>(T) * E);
  REQUIRE(moe_synth_normal_bf16(13, 1, 0.0f, 1.0f, 0, static_cast<int64_t>(lg.size()), lg.data()) == 0);
  for (int t = 0; t < T; ++t) lg[static_cast<size_t>(t) * E + 7] = lg[static_cast<size_t>(t) * E + 300];  // ties
  array ld = array::from_host(lg.data(), {1, T, E}, Dtype::bfloat16);
  auto [inds, scores] = moe_route(ld, k);
  REQUIRE((inds.shape() == Shape{1, T, k}) && (scores.shape() == Shape{1, T, k}));
  std::vector<uint32_t> ri(static_cast<size_t>(T) * k);
  std::vector<float> rs(ri.size());
  const oracle_router_params p{ORACLE_ROUTE_SOFTMAX_TOPK, E, k, 1, 1, 1, 1.0f};
  REQUIRE(oracle_route(lg.data(), nullptr, T, &p, ri.data(), rs.data(), nullptr) == 0);
  REQUIRE(download<uint32_t>(inds) == ri);
  const auto gs = download<float>(scores);
  REQUIRE(std::memcmp(gs.data(), rs.data(), rs.size() * 4) == 0);
}

// ---- subcommands over a checkpoint directory -----------------------------------------
int dump(const std::string& dir, bool sanitize) {
  HostTensors t = read_safetensors_from_directory(dir);
  if (sanitize) sanitize_moe_experts(t, read_json_file(dir + "/config.json"));
  std::vector<std::string> names;
  for (const auto& [n, v] : t) names.push_back(n);
  std::sort(names.begin(), names.end());
  for (const std::string& n : names) {
    const HostTensor& v = t.at(n);
    std::string shape;
    for (size_t i = 0; i < v.shape.size(); ++i) shape += (i ? "," : "") + std::to_string(v.shape[i]);
    std::printf("%s\t%s\t%s\t%08x\n", n.c_str(), v.dtype.c_str(), shape.c_str(), crc32(v.data, v.nbytes));
  }
  return 0;
}

template <class T>
void read_exact(std::ifstream& f, T* p, size_t n) {
  f.read(reinterpret_cast<char*>(p), static_cast<std::streamsize>(n * sizeof(T)));
  if (!f) throw std::runtime_error("short input file");
}

// The reference's loader sequence (llm_factory.cpp:106-119) for one layer's experts.
int load_glu(const std::string& dir, int layer, const std::string& in, const std::string& out) {
  const Json cfg = read_json_file(dir + "/config.json");
  const MoeNaming& nm = moe_naming(cfg.at("model_type").str());
  const Json& tc = text_config(cfg);
  const int H = static_cast<int>(tc.at("hidden_size").integer());
  const int I = static_cast<int>(tc.value(nm.intermediate_key, int64_t{nm.intermediate_default}));
  const int E = static_cast<int>(tc.value(nm.experts_key, int64_t{nm.experts_default}));
  HostTensors host = read_safetensors_from_directory(dir);
  const int stacked = sanitize_moe_experts(host, cfg);
  const std::string prefix = "model.layers." + std::to_string(layer) + "." + nm.block + "." + nm.stacked + ".";
  std::unordered_map<std::string, array> weights;
  for (const auto& [n, t] : host)
    if (n.rfind(prefix, 0) == 0) weights.emplace(n, to_device(t));
  QuantizedWeightRegistry::instance().clear();
  // GPT-OSS: SwitchLinear(bias=true) x3 and its clipped SwiGLU (gptoss.cpp:122-124, 158)
  SwitchGLU glu(H, I, E, nm.linear_bias, nm.activation);
  std::unordered_map<std::string, array*> wm;
  for (auto& [k, v] : glu.weight_map()) wm[prefix + k] = v;
  register_quantized_weights(weights, parse_quantization(cfg), wm);
  const int loaded = load_weights(weights, wm);
  std::printf("load-glu: %zu tensors, %d stacked, %zu under %s, %d loaded, %zu registered\n", host.size(), stacked,
              weights.size(), prefix.c_str(), loaded, QuantizedWeightRegistry::instance().size());
  const int want = nm.linear_bias ? 6 : 3;
  if (loaded != want || QuantizedWeightRegistry::instance().size() != 3) throw std::runtime_error("layer not loaded");
  std::ifstream f(in, std::ios::binary);
  int32_t tk[2];
  read_exact(f, tk, 2);
  const int T = tk[0], k = tk[1];
  std::vector<uint16_t> x(static_cast<size_t>(T) * H);
  std::vector<uint32_t> inds(static_cast<size_t>(T) * k);
  read_exact(f, x.data(), x.size());
  read_exact(f, inds.data(), inds.size());
  array y = glu(array::from_host(x.data(), {1, T, H}, Dtype::bfloat16),
                array::from_host(inds.data(), {1, T, k}, Dtype::uint32));
  if (y.shape() != Shape{1, T, k, H}) throw std::runtime_error("unexpected output shape");
  const auto yh = download<uint16_t>(y);
  std::ofstream(out, std::ios::binary).write(reinterpret_cast<const char*>(yh.data()),
                                             static_cast<std::streamsize>(yh.size() * 2));
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  const std::string group = argc > 1 ? argv[1] : "cpu";
  try {
    if (group == "dump" && argc >= 3) return dump(argv[2], argc > 3 && std::string(argv[3]) == "sanitize");
    if (group == "load-glu" && argc == 6) return load_glu(argv[2], std::atoi(argv[3]), argv[4], argv[5]);
  } catch (const std::exception& e) {
    std::printf("%s failed: %s\n", group.c_str(), e.what());
    return 1;
  }
  int failed = 0, run = 0;
  for (const Case& c : cases()) {
    if (group != c.group) continue;
    ++run;
    std::printf("[%s] %s ...\n", c.group, c.name);
    std::fflush(stdout);
    try {
      c.fn();
      std::printf("  ok\n");
    } catch (const std::exception& e) {
      ++failed;
      std::printf("  FAILED: %s\n", e.what());
    }
    std::fflush(stdout);
  }
  std::printf("%d of %d %s tests passed\n", run - failed, run, group.c_str());
  return failed == 0 && run > 0 ? 0 : 1;
}
