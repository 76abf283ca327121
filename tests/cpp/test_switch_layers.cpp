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
//
// The checker is test infrastructure; this program only compares against it.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <numeric>
#include <set>
#include <stdexcept>
#include <string>
#include <vector>

#include "moe_oracle.h"
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

// GPT-OSS style (gptoss.cpp:129-168): SwitchLinear with linear biases called
// directly, with gather_sort / scatter_unsort when there are >= 64 pairs.
void gptoss_case(int T, int k) {
  QuantizedWeightRegistry::instance().clear();
  const int E = 8, H = 256, I = 512;
  const HostQ g = make_q(7, 2, E, I, H, 4), u = make_q(7, 3, E, I, H, 4), d = make_q(7, 4, E, H, I, 4);
  SwitchLinear gate(H, I, E, true), up(H, I, E, true), down(I, H, E, true);
  load(gate, g);
  load(up, u);
  load(down, d);
  std::vector<uint16_t> bg(E * I), bu(E * I), bd(E * H);
  REQUIRE(moe_synth_normal_bf16(7, 10, 0.0f, 0.1f, 0, E * I, bg.data()) == 0);
  REQUIRE(moe_synth_normal_bf16(7, 11, 0.0f, 0.1f, 0, E * I, bu.data()) == 0);
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
  array act(x_gate.shape(), Dtype::bfloat16);
  check_status(moe_swiglu(x_gate.data<uint16_t>(), x_up.data<uint16_t>(), static_cast<int64_t>(act.size()),
                          act.data<uint16_t>(), nullptr),
               "swiglu");
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
  std::vector<uint16_t> h(gg.size());
  oracle_swiglu(gg.data(), uu.data(), static_cast<int64_t>(h.size()), h.data());
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

}  // namespace

int main(int argc, char** argv) {
  const std::string group = argc > 1 ? argv[1] : "cpu";
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
