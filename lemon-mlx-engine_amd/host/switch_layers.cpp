// switch_layers.cpp -- the C++ host classes of switch_layers.hpp.  Every
// device operation is one call of the C ABI in include/moe_mi355x.h; this file
// does shape logic, broadcasting, weight bookkeeping and error mapping only.
#include "switch_layers.hpp"

#include <cstdlib>
#include <stdexcept>
#include <string>

namespace mlx_lm {
namespace mi355x {

namespace {

thread_local hipStream_t t_stream = nullptr;

moe_stream_t abi_stream() { return reinterpret_cast<moe_stream_t>(default_stream()); }

void hip_check(hipError_t e, const char* where) {
  if (e != hipSuccess) throw std::runtime_error(std::string(where) + ": " + hipGetErrorString(e));
}

std::shared_ptr<void> device_alloc(size_t bytes) {
  void* p = nullptr;
  hip_check(hipMalloc(&p, bytes), "hipMalloc");
  return std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
}

[[noreturn]] void bad(const std::string& msg) { throw std::invalid_argument(msg); }

std::string shape_str(const Shape& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

int64_t numel(const Shape& s, size_t begin = 0, size_t end = static_cast<size_t>(-1)) {
  int64_t n = 1;
  for (size_t i = begin; i < s.size() && i < end; ++i) n *= s[i];
  return n;
}

// numpy broadcasting of two shapes (right-aligned; 1 stretches)
Shape broadcast_shapes(const Shape& a, const Shape& b, const char* where) {
  const size_t n = std::max(a.size(), b.size());
  Shape r(n);
  for (size_t i = 0; i < n; ++i) {
    const int32_t da = i < n - a.size() ? 1 : a[i - (n - a.size())];
    const int32_t db = i < n - b.size() ? 1 : b[i - (n - b.size())];
    if (da != db && da != 1 && db != 1)
      bad(std::string(where) + ": shapes " + shape_str(a) + " and " + shape_str(b) + " do not broadcast");
    r[i] = da == 1 ? db : da;
  }
  return r;
}

// For every element of the broadcast shape `out`, the flat index of the
// element of `src` it reads.
std::vector<int32_t> broadcast_map(const Shape& src, const Shape& out) {
  const size_t n = out.size(), off = n - src.size();
  std::vector<int64_t> stride(n, 0);
  int64_t s = 1;
  for (size_t i = n; i-- > off;) {
    stride[i] = src[i - off] == 1 ? 0 : s;
    s *= src[i - off];
  }
  const int64_t total = numel(out);
  std::vector<int32_t> map(static_cast<size_t>(total));
  std::vector<int32_t> coord(n, 0);
  for (int64_t f = 0; f < total; ++f) {
    int64_t idx = 0;
    for (size_t i = 0; i < n; ++i) idx += coord[i] * stride[i];
    map[static_cast<size_t>(f)] = static_cast<int32_t>(idx);
    for (size_t i = n; i-- > 0;) {
      if (++coord[i] < out[i]) break;
      coord[i] = 0;
    }
  }
  return map;
}

bool is_index(const array& a) { return a.dtype() == Dtype::uint32 || a.dtype() == Dtype::int32; }

Workspace& scratch() {
  thread_local Workspace ws;
  return ws;
}

moe_qweight abi_weight(const array& w, const QuantizationInfo& qi, int experts, int N, int K,
                       const char* where) {
  if (!w.has_data()) bad(std::string(where) + ": the expert weight is not loaded");
  const Shape want{experts, N, K * qi.bits / 32};
  if (w.shape() != want || w.dtype() != Dtype::uint32)
    bad(std::string(where) + ": quantized weight must be uint32 " + shape_str(want) + ", got " +
        shape_str(w.shape()));
  const Shape gshape{experts, N, K / qi.group_size};
  if (qi.scales.shape() != gshape || qi.scales.dtype() != Dtype::bfloat16)
    bad(std::string(where) + ": scales must be bf16 " + shape_str(gshape));
  if (qi.biases && (qi.biases->shape() != gshape || qi.biases->dtype() != Dtype::bfloat16))
    bad(std::string(where) + ": biases must be bf16 " + shape_str(gshape));
  return moe_qweight{w.data<uint32_t>(), qi.scales.data<uint16_t>(),
                     qi.biases ? qi.biases->data<uint16_t>() : nullptr, experts, N, K, qi.group_size, qi.bits, nullptr};
}

}  // namespace

// ---- basics ---------------------------------------------------------------------
size_t itemsize(Dtype d) { return d == Dtype::bfloat16 ? 2 : 4; }

const char* dtype_name(Dtype d) {
  switch (d) {
    case Dtype::bfloat16: return "bfloat16";
    case Dtype::float32: return "float32";
    case Dtype::uint32: return "uint32";
    case Dtype::int32: return "int32";
  }
  return "?";
}

hipStream_t default_stream() { return t_stream; }
void set_default_stream(hipStream_t stream) { t_stream = stream; }

void check_status(int status, const char* where) {
  if (status == MOE_OK) return;
  std::string msg = std::string(where) + ": " + moe_status_string(status);
  if (status == MOE_E_HIP) msg += std::string(": ") + moe_last_error();
  if (status == MOE_E_INVALID_ARG || status == MOE_E_UNSUPPORTED || status == MOE_E_INDEX) bad(msg);
  throw std::runtime_error(msg);
}

// ---- array ------------------------------------------------------------------------
array::array(Shape shape, Dtype dtype) : shape_(std::move(shape)), dtype_(dtype) {
  for (int32_t d : shape_)
    if (d < 0) bad("array: negative dimension in " + shape_str(shape_));
  const size_t bytes = nbytes();
  if (bytes > 0) buf_ = device_alloc(bytes);
}

array array::from_host(const void* data, Shape shape, Dtype dtype) {
  array a(std::move(shape), dtype);
  if (a.nbytes() > 0) hip_check(hipMemcpy(a.raw(), data, a.nbytes(), hipMemcpyHostToDevice), "array::from_host");
  return a;
}

void array::to_host(void* dst) const {
  if (nbytes() == 0) return;
  hip_check(hipStreamSynchronize(default_stream()), "array::to_host");
  hip_check(hipMemcpy(dst, raw(), nbytes(), hipMemcpyDeviceToHost), "array::to_host");
}

int32_t array::shape(int axis) const {
  const int n = ndim();
  const int a = axis < 0 ? axis + n : axis;
  if (a < 0 || a >= n) bad("array::shape: axis " + std::to_string(axis) + " out of range for " + shape_str(shape_));
  return shape_[a];
}

size_t array::size() const { return static_cast<size_t>(numel(shape_)); }

array array::reshape(Shape shape) const {
  if (numel(shape) != numel(shape_)) bad("reshape: cannot reshape " + shape_str(shape_) + " to " + shape_str(shape));
  array a = *this;
  a.shape_ = std::move(shape);
  return a;
}

void* Workspace::get(size_t bytes) {
  bytes = std::max<size_t>(bytes, 256);
  if (bytes > bytes_) {
    // work queued on the old buffer finishes before it is released
    hip_check(hipStreamSynchronize(default_stream()), "Workspace::get");
    buf_.reset();
    buf_ = device_alloc(bytes);
    bytes_ = bytes;
  }
  return buf_.get();
}

// ---- registry ---------------------------------------------------------------------
QuantizedWeightRegistry& QuantizedWeightRegistry::instance() {
  static QuantizedWeightRegistry reg;
  return reg;
}

void QuantizedWeightRegistry::register_weight(const array* weight_ptr, array scales, std::optional<array> biases,
                                              int group_size, int bits) {
  registry_.insert_or_assign(weight_ptr,
                             QuantizationInfo{std::move(scales), std::move(biases), group_size, bits});
}

const QuantizationInfo* QuantizedWeightRegistry::find(const array* weight_ptr) const {
  auto it = registry_.find(weight_ptr);
  return it != registry_.end() ? &it->second : nullptr;
}

void QuantizedWeightRegistry::unregister(const array* weight_ptr) { registry_.erase(weight_ptr); }

// ---- gather_sort / scatter_unsort ----------------------------------------------------
std::tuple<array, array, array> gather_sort(const array& x, const array& indices, int num_experts) {
  if (indices.ndim() < 1 || !is_index(indices)) bad("gather_sort: indices must be an integer array [..., m]");
  if (x.ndim() < 3) bad("gather_sort: x must have at least 3 dimensions, got " + shape_str(x.shape()));
  if (num_experts <= 0) bad("gather_sort: num_experts must be positive");
  const int m = indices.shape(-1);
  const int64_t P = static_cast<int64_t>(indices.size());
  const int64_t rows = numel(x.shape(), 0, x.shape().size() - 2);
  if (m <= 0 || rows * m != P)
    bad("gather_sort: x " + shape_str(x.shape()) + " and indices " + shape_str(indices.shape()) +
        " disagree on the number of rows");
  const int64_t T = P / m;
  array perm({static_cast<int32_t>(P)}, Dtype::int32);
  array inv({static_cast<int32_t>(P)}, Dtype::uint32);
  array sorted_idx({static_cast<int32_t>(P)}, Dtype::uint32);
  const size_t bws = moe_bucket_workspace_size(T, m, num_experts);
  // offsets [E+1] then the bucket scratch, in one per-thread workspace
  const size_t off_bytes = ((static_cast<size_t>(num_experts) + 1) * 4 + 255) & ~size_t{255};
  char* ws = static_cast<char*>(scratch().get(off_bytes + bws));
  check_status(moe_bucket(indices.data<uint32_t>(), T, m, num_experts, perm.data<int32_t>(), inv.data<int32_t>(),
                          sorted_idx.data<uint32_t>(), reinterpret_cast<int32_t*>(ws), ws + off_bytes, bws,
                          abi_stream()),
               "gather_sort");
  const Shape& xs = x.shape();
  array sorted_x({static_cast<int32_t>(P), xs[xs.size() - 2], xs[xs.size() - 1]}, x.dtype());
  const int64_t row_bytes = static_cast<int64_t>(xs[xs.size() - 2]) * xs[xs.size() - 1] * itemsize(x.dtype());
  check_status(moe_take_rows(x.raw(), rows, perm.data<int32_t>(), P, m, row_bytes, sorted_x.raw(), abi_stream()),
               "gather_sort");
  return {sorted_x, sorted_idx, inv};
}

array scatter_unsort(const array& x, const array& inv_order, const Shape* shape) {
  if (!is_index(inv_order)) bad("scatter_unsort: inv_order must be an integer array");
  if (x.ndim() < 1) bad("scatter_unsort: x must have a leading axis");
  const int64_t n = static_cast<int64_t>(inv_order.size());
  Shape out_shape{static_cast<int32_t>(n)};
  out_shape.insert(out_shape.end(), x.shape().begin() + 1, x.shape().end());
  array result(out_shape, x.dtype());
  const int64_t row_bytes = numel(x.shape(), 1) * static_cast<int64_t>(itemsize(x.dtype()));
  check_status(moe_take_rows(x.raw(), x.shape(0), inv_order.data<int32_t>(), n, 1, row_bytes, result.raw(),
                             abi_stream()),
               "scatter_unsort");
  if (shape && !shape->empty()) {
    Shape ns(*shape);
    ns.insert(ns.end(), x.shape().begin() + 1, x.shape().end());
    result = result.reshape(ns);
  }
  return result;
}

// ---- moe_route ----------------------------------------------------------------------
std::pair<array, array> moe_route(const array& logits, int k) {
  if (logits.dtype() != Dtype::bfloat16 || logits.ndim() < 1) bad("moe_route: logits must be bf16 [..., E]");
  const int E = logits.shape(-1);
  const int64_t T = E > 0 ? static_cast<int64_t>(logits.size()) / E : 0;
  Shape os(logits.shape());
  os.back() = k;
  array inds(os, Dtype::uint32);
  array scores(os, Dtype::float32);
  const moe_router_params p{MOE_ROUTE_SOFTMAX_TOPK, E, k, 1, 1, 1, 1.0f};
  check_status(moe_route(logits.data<uint16_t>(), nullptr, T, &p, inds.data<uint32_t>(), scores.data<float>(),
                         abi_stream()),
               "moe_route");
  return {inds, scores};
}

// ---- SwitchLinear ---------------------------------------------------------------------
SwitchLinear::SwitchLinear(int input_dims, int output_dims, int num_experts, bool bias)
    : input_dims_(input_dims), output_dims_(output_dims), num_experts_(num_experts) {
  if (input_dims <= 0 || output_dims <= 0 || num_experts <= 0) bad("SwitchLinear: dimensions must be positive");
  if (bias) bias_ = array();
}

array SwitchLinear::operator()(const array& x, const array& indices, bool sorted_indices) {
  // quantized experts run gather_qmm, dense (bf16) ones gather_mm (switch_layers.cpp:94-109)
  const QuantizationInfo* qi = QuantizedWeightRegistry::instance().find(&weight_);
  if (x.dtype() != Dtype::bfloat16) bad(std::string("SwitchLinear: x must be bfloat16, got ") + dtype_name(x.dtype()));
  if (x.ndim() < 2 || x.shape(-1) != input_dims_)
    bad("SwitchLinear: x must be [..., M, " + std::to_string(input_dims_) + "], got " + shape_str(x.shape()));
  if (!is_index(indices)) bad("SwitchLinear: indices must be uint32 or int32");
  moe_qweight qw{};
  if (qi) {
    qw = abi_weight(weight_, *qi, num_experts_, output_dims_, input_dims_, "SwitchLinear");
  } else if (!weight_.has_data() || weight_.dtype() != Dtype::bfloat16 ||
             weight_.shape() != Shape{num_experts_, output_dims_, input_dims_}) {
    bad("SwitchLinear: a weight that is not registered as quantized must be bf16 [" + std::to_string(num_experts_) +
        ", " + std::to_string(output_dims_) + ", " + std::to_string(input_dims_) + "], got " +
        shape_str(weight_.shape()));
  }
  const uint16_t* lbias = nullptr;
  if (bias_) {  // the take(bias, indices) + add (switch_layers.cpp:111-114), applied by the kernel itself
    if (!bias_->has_data() || bias_->shape() != Shape{num_experts_, output_dims_} ||
        bias_->dtype() != Dtype::bfloat16)
      bad("SwitchLinear: bias must be bf16 [" + std::to_string(num_experts_) + ", " + std::to_string(output_dims_) +
          "]");
    lbias = bias_->data<uint16_t>();
    qw.linear_bias = lbias;
  }

  const Shape xb(x.shape().begin(), x.shape().end() - 2);
  const Shape& ib = indices.shape();
  const Shape ob = broadcast_shapes(xb, ib, "SwitchLinear");
  const int M = x.shape(-2);
  const int64_t batch = numel(ob);

  // index maps for operands that broadcast (cached per shape pair)
  const bool lhs_identity = numel(xb) == batch && xb.size() <= ob.size() &&
                            Shape(ob.end() - xb.size(), ob.end()) == xb && numel(ob, 0, ob.size() - xb.size()) == 1;
  const bool rhs_direct = ib == ob || (numel(ib) == batch && Shape(ob.end() - ib.size(), ob.end()) == ib);
  if ((!lhs_identity || !rhs_direct) && (cache_xb_ != xb || cache_ib_ != ib || !lhs_map_)) {
    const std::vector<int32_t> lm = broadcast_map(xb, ob), rm = broadcast_map(ib, ob);
    lhs_map_ = array::from_host(lm.data(), {static_cast<int32_t>(batch)}, Dtype::uint32);
    rhs_map_ = array::from_host(rm.data(), {static_cast<int32_t>(batch)}, Dtype::int32);
    cache_xb_ = xb;
    cache_ib_ = ib;
  }
  const uint32_t* lhs = lhs_identity ? nullptr : lhs_map_->data<uint32_t>();
  array rhs_b;
  const uint32_t* rhs = indices.data<uint32_t>();
  if (!rhs_direct) {
    rhs_b = array({static_cast<int32_t>(batch)}, Dtype::uint32);
    check_status(moe_take_rows(indices.raw(), static_cast<int64_t>(indices.size()), rhs_map_->data<int32_t>(), batch,
                               1, 4, rhs_b.raw(), abi_stream()),
                 "SwitchLinear");
    rhs = rhs_b.data<uint32_t>();
  }

  Shape os(ob);
  os.push_back(M);
  os.push_back(output_dims_);
  array out(os, Dtype::bfloat16);
  if (batch == 0) return out;
  if (qi) {
    const size_t wsz = moe_gather_qmm_workspace_size(batch, M, num_experts_);
    void* ws = ws_.get(wsz);
    check_status(moe_gather_qmm(x.data<uint16_t>(), &qw, lhs, rhs, batch, M, sorted_indices ? 1 : 0,
                                out.data<uint16_t>(), ws, ws_.capacity(), abi_stream()),
                 "SwitchLinear");
  } else {
    const size_t wsz = moe_gather_mm_workspace_size(batch, M, num_experts_);
    void* ws = ws_.get(wsz);
    check_status(moe_gather_mm(x.data<uint16_t>(), weight_.data<uint16_t>(), lbias, num_experts_, output_dims_,
                               input_dims_, lhs, rhs, batch, M, sorted_indices ? 1 : 0, out.data<uint16_t>(), ws,
                               ws_.capacity(), abi_stream()),
                 "SwitchLinear");
  }
  return out;
}

std::unordered_map<std::string, array*> SwitchLinear::weight_map() {
  std::unordered_map<std::string, array*> map;
  map["weight"] = &weight_;
  if (bias_) map["bias"] = &bias_.value();
  return map;
}

void SwitchLinear::adopt_fused_weight(array w, array scales, std::optional<array> biases, int group_size,
                                      int bits) {
  weight_ = std::move(w);
  QuantizedWeightRegistry::instance().register_weight(&weight_, std::move(scales), std::move(biases), group_size,
                                                      bits);
}

void SwitchLinear::release_weight() {
  QuantizedWeightRegistry::instance().unregister(&weight_);
  weight_ = array();
}

// ---- SwitchGLU -------------------------------------------------------------------------
SwitchGLU::SwitchGLU(int input_dims, int hidden_dims, int num_experts, bool bias, int activation)
    : gate_proj_(input_dims, hidden_dims, num_experts, bias),
      up_proj_(input_dims, hidden_dims, num_experts, bias),
      down_proj_(hidden_dims, input_dims, num_experts, bias),
      input_dims_(input_dims),
      hidden_dims_(hidden_dims),
      num_experts_(num_experts),
      activation_(activation) {
  if (activation != MOE_ACT_SWIGLU && activation != MOE_ACT_GPTOSS && activation != MOE_ACT_GPTOSS_UPSTREAM)
    bad("SwitchGLU: unknown activation " + std::to_string(activation));
}

bool SwitchGLU::fused_ready() const {
  auto& reg = QuantizedWeightRegistry::instance();
  const QuantizationInfo* qg = reg.find(&gate_proj_.weight());
  const QuantizationInfo* qu = reg.find(&up_proj_.weight());
  const QuantizationInfo* qd = reg.find(&down_proj_.weight());
  if (!qg || !qu || !qd) return false;
  if (qg->group_size != qu->group_size || qg->bits != qu->bits) return false;
  if (qg->biases.has_value() != qu->biases.has_value()) return false;
  // linear biases need the per-projection path
  auto& self = const_cast<SwitchGLU&>(*this);
  return !self.gate_proj_.weight_map().count("bias") && !self.up_proj_.weight_map().count("bias") &&
         !self.down_proj_.weight_map().count("bias");
}

array SwitchGLU::operator()(const array& x, const array& indices) {
  if (x.dtype() != Dtype::bfloat16) bad(std::string("SwitchGLU: x must be bfloat16, got ") + dtype_name(x.dtype()));
  if (x.ndim() < 1 || x.shape(-1) != input_dims_)
    bad("SwitchGLU: x must be [..., " + std::to_string(input_dims_) + "], got " + shape_str(x.shape()));
  if (!is_index(indices) || indices.ndim() != x.ndim() ||
      Shape(indices.shape().begin(), indices.shape().end() - 1) != Shape(x.shape().begin(), x.shape().end() - 1))
    bad("SwitchGLU: indices must be [..., k] over the leading axes of x " + shape_str(x.shape()) + ", got " +
        shape_str(indices.shape()));
  const int k = indices.shape(-1);
  const int64_t T = numel(x.shape(), 0, x.shape().size() - 1);
  Shape os(indices.shape());
  os.push_back(input_dims_);

  if (fused_ready()) {
    // gather_sort + fused gate|up + swiglu + down + scatter_unsort in one call
    auto& reg = QuantizedWeightRegistry::instance();
    const moe_qweight g = abi_weight(gate_proj_.weight(), *reg.find(&gate_proj_.weight()), num_experts_,
                                     hidden_dims_, input_dims_, "SwitchGLU.gate_proj");
    const moe_qweight u = abi_weight(up_proj_.weight(), *reg.find(&up_proj_.weight()), num_experts_, hidden_dims_,
                                     input_dims_, "SwitchGLU.up_proj");
    const moe_qweight d = abi_weight(down_proj_.weight(), *reg.find(&down_proj_.weight()), num_experts_,
                                     input_dims_, hidden_dims_, "SwitchGLU.down_proj");
    array out(os, Dtype::bfloat16);
    if (T == 0 || k == 0) return out;
    const size_t wsz = moe_switch_glu_workspace_size(&g, &d, T, k);
    void* ws = ws_.get(wsz);
    check_status(moe_switch_glu(&g, &u, &d, x.data<uint16_t>(), indices.data<uint32_t>(), T, k, activation_,
                                out.data<uint16_t>(), ws, ws_.capacity(), abi_stream()),
                 "SwitchGLU");
    return out;
  }

  // per-projection path (linear biases): the reference's sequence, switch_layers.cpp:200-245
  Shape xe(x.shape().begin(), x.shape().end() - 1);
  xe.push_back(1);
  xe.push_back(1);
  xe.push_back(input_dims_);
  array work_x = x.reshape(xe);
  static const int sort_min = [] {
    const char* e = std::getenv("MLX_MOE_SORT_MIN");
    return e ? std::atoi(e) : 64;
  }();
  const bool do_sort = static_cast<int64_t>(indices.size()) >= sort_min;
  array idx = indices;
  array inverse_order;
  if (do_sort) {
    auto [sx, si, io] = gather_sort(work_x, indices, num_experts_);
    work_x = sx;
    idx = si;
    inverse_order = io;
  }
  array x_up = up_proj_(work_x, idx, do_sort);
  array x_gate = gate_proj_(work_x, idx, do_sort);
  array h;
  if (activation_ == MOE_ACT_SWIGLU) {
    h = array(x_gate.shape(), Dtype::bfloat16);
    check_status(moe_swiglu(x_gate.data<uint16_t>(), x_up.data<uint16_t>(), static_cast<int64_t>(h.size()),
                            h.data<uint16_t>(), abi_stream()),
                 "SwitchGLU");
  } else {  // GPT-OSS: swiglu(x_gate, x_up) as gptoss.cpp:158 calls it (or the upstream roles)
    h = activation_ == MOE_ACT_GPTOSS ? gptoss_swiglu(x_gate, x_up) : gptoss_swiglu(x_up, x_gate);
  }
  array y = down_proj_(h, idx, do_sort);
  if (do_sort) {
    const Shape& ishape = indices.shape();
    y = scatter_unsort(y, inverse_order, &ishape);
  }
  return y.reshape(os);  // squeeze(-2)
}

// ---- GPT-OSS's clipped SwiGLU (gptoss.cpp:50-58) ---------------------------------------
array gptoss_swiglu(const array& x_linear, const array& x_glu) {
  if (x_linear.dtype() != Dtype::bfloat16 || x_glu.dtype() != Dtype::bfloat16)
    bad("gptoss_swiglu: x_linear and x_glu must be bfloat16");
  if (x_linear.shape() != x_glu.shape())
    bad("gptoss_swiglu: shapes differ: " + shape_str(x_linear.shape()) + " vs " + shape_str(x_glu.shape()));
  array h(x_linear.shape(), Dtype::bfloat16);
  check_status(moe_gptoss_swiglu(x_linear.data<uint16_t>(), x_glu.data<uint16_t>(), static_cast<int64_t>(h.size()),
                                 h.data<uint16_t>(), abi_stream()),
               "gptoss_swiglu");
  return h;
}

std::unordered_map<std::string, array*> SwitchGLU::weight_map() {
  std::unordered_map<std::string, array*> map;
  for (auto& [k, v] : gate_proj_.weight_map()) map["gate_proj." + k] = v;
  for (auto& [k, v] : up_proj_.weight_map()) map["up_proj." + k] = v;
  for (auto& [k, v] : down_proj_.weight_map()) map["down_proj." + k] = v;
  return map;
}

}  // namespace mi355x
}  // namespace mlx_lm
