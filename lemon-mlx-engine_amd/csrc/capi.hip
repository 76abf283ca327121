// capi.hip -- the extern "C" boundary declared in include/moe_mi355x.h.
//
// Every entry point validates its arguments on the host, never throws, and
// returns a moe_status.  Device work is enqueued on the caller's stream.

#include <cstdio>
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "internal.hpp"

// Scratch of moe_block_forward_noalloc: the block's workspace for callers that
// cannot allocate.  Every GPU the library runs on holds its own copy for the
// life of the process.  The name is a host-side stand-in in host code: the
// device address comes from hipGetSymbolAddress (static_scratch below).
constexpr size_t kStaticScratchBytes = static_cast<size_t>(64) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace moe {

namespace {

thread_local char g_last_error[256] = "";

// Bump allocator over a caller workspace (or a dry run that only measures).
class Carve {
 public:
  explicit Carve(void* base) : base_(static_cast<char*>(base)) {}
  template <class T>
  T* take(int64_t count) {
    const size_t bytes = static_cast<size_t>(count > 0 ? count : 0) * sizeof(T);
    off_ = (off_ + 255) & ~static_cast<size_t>(255);
    T* p = base_ ? reinterpret_cast<T*>(base_ + off_) : nullptr;
    off_ += bytes;
    return p;
  }
  char* raw(size_t bytes) {
    off_ = (off_ + 255) & ~static_cast<size_t>(255);
    char* p = base_ ? base_ + off_ : nullptr;
    off_ += bytes;
    return p;
  }
  size_t size() const { return (off_ + 255) & ~static_cast<size_t>(255); }

 private:
  char* base_;
  size_t off_ = 0;
};

// The bucket {0, T} of a one-expert projection over T rows (shared expert,
// quantized router) for the large-bucket GEMM (on the per-16-row kernel the
// rows go as 16-row slots whose records the kernel derives itself).
__global__ void fill_shared_meta(int32_t* offsets, int32_t* active, int32_t* num_active, int T) {
  if (threadIdx.x == 0) {
    offsets[0] = 0;
    offsets[1] = T;
    active[0] = 0;  // slot record {expert 0, first row 0, T rows}
    active[1] = 0;
    active[2] = T;
    active[3] = 0;
    num_active[0] = 1;
  }
}

// pair i = (b, m) takes expert rhs[b].  A pair whose expert is out of range
// is left out by the bucketing; its output row (row i of out [*, N]) is
// written as zeros here so that it never returns stale memory.
__global__ void expand_pairs(const uint32_t* __restrict__ rhs, int64_t batch, int M, int E,
                             uint32_t* __restrict__ pair_expert, uint16_t* __restrict__ out, int N) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= batch * M) return;
  const uint32_t e = rhs[i / M];
  pair_expert[i] = e;
  if (e >= static_cast<uint32_t>(E))
    for (int c = 0; c < N; ++c) out[i * N + c] = 0;
}

__global__ void make_in_rows(const int32_t* __restrict__ perm, const uint32_t* __restrict__ lhs,
                             int64_t n, int M, int32_t* __restrict__ in_rows) {
  const int64_t pos = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (pos >= n) return;
  const int64_t f = perm[pos];
  if (f < 0 || f >= n) {  // a position past the buckets (pairs of out-of-range experts): never read
    in_rows[pos] = 0;
    return;
  }
  const int64_t b = f / M, m = f % M;
  const int64_t src = lhs ? static_cast<int64_t>(lhs[b]) : b;
  in_rows[pos] = static_cast<int32_t>(src * M + m);
}

struct BlockPlan {
  uint16_t* logits;
  uint32_t* inds;
  float* scores;
  BucketOut bk;
  char* bucket_ws;
  size_t bucket_ws_bytes;
  uint16_t* xp;  // x in pair K order (input of the large-bucket gate|up GEMMs)
  uint16_t* h;
  uint16_t* Y;
  uint16_t* sgl;
  uint16_t* hs;
  uint16_t* Ys;
  int32_t* sh_offsets;
  int32_t* sh_active;
  int32_t* sh_num;
  int32_t* tiles;
  int32_t* sh_tiles;
  float* gsum;
  float* hsum;  // group sums of h (written by the gate|up GEMM for down)
  float* rpart;  // small batches: the router projection's partial sums [ks][T][E]
  int rks;       // their slice count (0: the small-batch router is not used)
  float* tpart;  // many tokens: the K-split projection's partial sums [tks][T][E]
  int tks;       // their slice count (1: one slice, bf16 logits straight from the projection)
};

bool activation_ok(int act) {
  return act == MOE_ACT_SWIGLU || act == MOE_ACT_GPTOSS || act == MOE_ACT_GPTOSS_UPSTREAM;
}

int block_validate(const moe_block_desc* d) {
  if (!d) return MOE_E_INVALID_ARG;
  const int H = d->hidden, I = d->intermediate, E = d->num_experts;
  if (H <= 0 || I <= 0 || E <= 0) return MOE_E_INVALID_ARG;
  if (d->router.num_experts != E) return MOE_E_INVALID_ARG;
  int st = route_validate(&d->router);
  if (st != MOE_OK) return st;
  if (d->router_q.w) {  // quantized router [1][E, H]
    st = qweight_check(&d->router_q);
    if (st != MOE_OK) return st;
    if (d->router_q.experts != 1 || d->router_q.N != E || d->router_q.K != H) return MOE_E_INVALID_ARG;
  } else if (!d->router_weight) {
    return MOE_E_INVALID_ARG;
  }
  if (moe::route_needs_bias(d->router.variant) && !d->score_bias) return MOE_E_INVALID_ARG;
  const moe_qweight* ws[3] = {&d->gate, &d->up, &d->down};
  for (const moe_qweight* w : ws) {
    st = qweight_check(w);
    if (st != MOE_OK) return st;
    if (w->experts != E) return MOE_E_INVALID_ARG;
  }
  if (d->gate.N != I || d->gate.K != H || d->up.N != I || d->up.K != H || d->down.N != H ||
      d->down.K != I)
    return MOE_E_INVALID_ARG;
  if (!activation_ok(d->activation)) return MOE_E_INVALID_ARG;
  if (I % 16 != 0) return MOE_E_UNSUPPORTED;  // gate|up run as whole 16-row tiles
  if (d->shared_intermediate < 0) return MOE_E_INVALID_ARG;
  if (d->shared_intermediate > 0) {
    const int Is = d->shared_intermediate;
    const moe_qweight* ss[3] = {&d->shared_gate, &d->shared_up, &d->shared_down};
    for (const moe_qweight* w : ss) {
      st = qweight_check(w);
      if (st != MOE_OK) return st;
      if (w->experts != 1) return MOE_E_INVALID_ARG;
    }
    if (d->shared_gate.N != Is || d->shared_gate.K != H || d->shared_up.N != Is ||
        d->shared_up.K != H || d->shared_down.N != H || d->shared_down.K != Is)
      return MOE_E_INVALID_ARG;
    if (d->shared_gate_q.w) {  // quantized sigmoid gate [1][1, H]
      st = qweight_check(&d->shared_gate_q);
      if (st != MOE_OK) return st;
      if (d->shared_gate_q.experts != 1 || d->shared_gate_q.N != 1 || d->shared_gate_q.K != H)
        return MOE_E_INVALID_ARG;
      if (H % 8 != 0) return MOE_E_UNSUPPORTED;
    }
  }
  return MOE_OK;
}

BlockPlan plan_block(const moe_block_desc* d, int64_t T, void* ws, size_t* total) {
  Carve c(ws);
  BlockPlan p{};
  const int E = d->num_experts, k = d->router.top_k, H = d->hidden, I = d->intermediate;
  const int64_t P = T * k;
  p.logits = c.take<uint16_t>(T * E);
  p.inds = c.take<uint32_t>(P);
  p.scores = c.take<float>(P);
  p.bk.perm = c.take<int32_t>(P);
  p.bk.inv_perm = c.take<int32_t>(P);
  p.bk.sorted_expert = nullptr;
  p.bk.sorted_token = c.take<int32_t>(P);
  p.bk.offsets = c.take<int32_t>(E + 1);
  p.bk.active = c.take<int32_t>(4 * static_cast<int64_t>(E));
  p.bk.num_active = c.take<int32_t>(1);
  p.tiles = c.take<int32_t>(moe::prefill_tile_ints(P, E));
  {
    int64_t g = T * moe::prefill_gsum_stride(&d->gate);
    g = std::max<int64_t>(g, P * moe::prefill_gsum_stride(&d->down));
    if (d->shared_intermediate > 0) {
      g = std::max<int64_t>(g, T * moe::prefill_gsum_stride(&d->shared_gate));
      g = std::max<int64_t>(g, T * moe::prefill_gsum_stride(&d->shared_down));
    }
    p.gsum = c.take<float>(g);
  }
  p.hsum = c.take<float>(P * moe::prefill_gsum_stride(&d->down));
  p.rks = d->router_q.w ? 0 : moe::router_partial_ks(T, E, H);
  p.rpart = c.take<float>(static_cast<int64_t>(p.rks) * T * E);
  p.tks = d->router_q.w ? 1 : moe::router_tile32_ks(T, E, H, d->gate.group_size);
  p.tpart = c.take<float>(p.tks > 1 ? static_cast<int64_t>(p.tks) * T * E : 0);
  p.bucket_ws_bytes = bucket_workspace_bytes(P, E);
  p.bucket_ws = c.raw(p.bucket_ws_bytes);
  p.xp = c.take<uint16_t>(T * H);
  p.h = c.take<uint16_t>(P * I);
  p.Y = c.take<uint16_t>(P * H);
  if (d->shared_intermediate > 0) {
    p.sgl = c.take<uint16_t>(T);
    p.hs = c.take<uint16_t>(T * d->shared_intermediate);
    p.Ys = c.take<uint16_t>(T * H);
  }
  if (d->shared_intermediate > 0 || d->router_q.w) {  // one-expert projections over the T rows
    p.sh_offsets = c.take<int32_t>(2);
    p.sh_active = c.take<int32_t>(4);
    p.sh_num = c.take<int32_t>(1);
    p.sh_tiles = c.take<int32_t>(moe::prefill_tile_ints(T, 1));
  }
  *total = c.size();
  return p;
}

struct SwitchGluPlan {
  BucketOut bk;
  char* bucket_ws;
  size_t bucket_ws_bytes;
  int32_t* tiles;
  float* gsum;
  float* hsum;
  uint16_t* xp;  // x in pair K order (input of the large-bucket gate|up GEMM)
  uint16_t* h;
};

int switch_glu_validate(const moe_qweight* gate, const moe_qweight* up, const moe_qweight* down, int k) {
  if (!gate || !up || !down || k <= 0) return MOE_E_INVALID_ARG;
  const moe_qweight* ws[3] = {gate, up, down};
  for (const moe_qweight* w : ws) {
    const int st = qweight_check(w);
    if (st != MOE_OK) return st;
  }
  const int E = gate->experts, I = gate->N, H = gate->K;
  if (up->experts != E || down->experts != E || up->N != I || up->K != H || down->N != H || down->K != I)
    return MOE_E_INVALID_ARG;
  if (k > E) return MOE_E_INVALID_ARG;
  return MOE_OK;
}

SwitchGluPlan plan_switch_glu(const moe_qweight* gate, const moe_qweight* down, int64_t T, int k, void* ws,
                              size_t* total) {
  Carve c(ws);
  SwitchGluPlan p{};
  const int E = gate->experts;
  const int64_t P = T * k;
  p.bk.perm = c.take<int32_t>(P);
  p.bk.inv_perm = nullptr;
  p.bk.sorted_expert = nullptr;
  p.bk.sorted_token = c.take<int32_t>(P);
  p.bk.offsets = c.take<int32_t>(E + 1);
  p.bk.active = c.take<int32_t>(4 * static_cast<int64_t>(E));
  p.bk.num_active = c.take<int32_t>(1);
  p.tiles = c.take<int32_t>(moe::prefill_tile_ints(P, E));
  p.gsum = c.take<float>(std::max<int64_t>(T * moe::prefill_gsum_stride(gate),
                                           P * moe::prefill_gsum_stride(down)));
  p.hsum = c.take<float>(P * moe::prefill_gsum_stride(down));
  p.bucket_ws_bytes = bucket_workspace_bytes(P, E);
  p.bucket_ws = c.raw(p.bucket_ws_bytes);
  p.xp = c.take<uint16_t>(T * gate->K);
  p.h = c.take<uint16_t>(P * gate->N);
  *total = c.size();
  return p;
}

}  // namespace

namespace {
struct ProfRecord {
  const char* name;
  hipEvent_t start, stop;
};
struct Profiler {
  bool on = false;
  std::vector<ProfRecord> recs;
  std::vector<hipEvent_t> pool;
  size_t used = 0;
  hipEvent_t event() {
    if (used == pool.size()) {
      hipEvent_t e = nullptr;
      if (hipEventCreate(&e) != hipSuccess) return nullptr;
      pool.push_back(e);
    }
    return pool[used++];
  }
};
Profiler g_prof;
}  // namespace

thread_local ProfLabel g_prof_label = ProfLabel::kNone;
ProfScope::ProfScope(ProfLabel l) : prev(g_prof_label) { g_prof_label = l; }
ProfScope::~ProfScope() { g_prof_label = prev; }

// the record name of kernel label `name` under the current scope
const char* scoped_name(const char* name) {
  if (g_prof_label == ProfLabel::kNone) return name;
  static const char* const kMap[][3] = {  // label, shared expert, quantized router
      {"qmm_gate_up_swiglu", "shared_qmm_gate_up_swiglu", "router_q_qmm"},
      {"qmm_down", "shared_qmm_down", "router_q_qmm"},
      {"gemm_gate_up_swiglu", "shared_gemm_gate_up_swiglu", "router_q_gemm"},
      {"gemm_down", "shared_gemm_down", "router_q_gemm"},
      {"group_sums", "shared_group_sums", "router_q_group_sums"},
      {"make_tiles", "shared_make_tiles", "router_q_make_tiles"},
      {"router_logits", "shared_gate", "router_logits"}};
  const int col = g_prof_label == ProfLabel::kShared ? 1 : 2;
  for (const auto& m : kMap)
    if (std::strcmp(m[0], name) == 0) return m[col];
  return name;
}

void prof_begin(hipStream_t stream, const char* name) {
  if (!g_prof.on) return;
  ProfRecord r{scoped_name(name), g_prof.event(), nullptr};
  if (r.start) (void)hipEventRecord(r.start, stream);
  g_prof.recs.push_back(r);
}

void prof_end(hipStream_t stream) {
  if (!g_prof.on || g_prof.recs.empty()) return;
  ProfRecord& r = g_prof.recs.back();
  r.stop = g_prof.event();
  if (r.stop) (void)hipEventRecord(r.stop, stream);
}

void set_last_error(const char* where, hipError_t e) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s", where, hipGetErrorString(e));
}

int launch_status(const char* where) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_last_error(where, e);
    return MOE_E_HIP;
  }
  return MOE_OK;
}

}  // namespace moe

using moe::BucketOut;

extern "C" {

int moe_version(void) { return MOE_ABI_VERSION; }

int moe_profile_enable(int enable) {
  moe::g_prof.on = enable != 0;
  if (enable) {
    moe::g_prof.recs.clear();
    moe::g_prof.used = 0;
  }
  return MOE_OK;
}

int moe_profile_count(void) { return static_cast<int>(moe::g_prof.recs.size()); }

int moe_profile_record(int index, const char** name, float* milliseconds) {
  if (index < 0 || index >= static_cast<int>(moe::g_prof.recs.size()) || !name || !milliseconds)
    return MOE_E_INVALID_ARG;
  const moe::ProfRecord& r = moe::g_prof.recs[index];
  *name = r.name;
  *milliseconds = 0.0f;
  if (!r.start || !r.stop) return MOE_E_HIP;
  hipError_t e = hipEventSynchronize(r.stop);
  if (e == hipSuccess) e = hipEventElapsedTime(milliseconds, r.start, r.stop);
  if (e != hipSuccess) {
    moe::set_last_error("moe_profile_record", e);
    return MOE_E_HIP;
  }
  return MOE_OK;
}

const char* moe_status_string(int status) {
  switch (status) {
    case MOE_OK: return "ok";
    case MOE_E_INVALID_ARG: return "invalid argument";
    case MOE_E_UNSUPPORTED: return "unsupported shape, bit width or group size";
    case MOE_E_WORKSPACE: return "workspace missing or too small";
    case MOE_E_HIP: return "HIP runtime error";
    case MOE_E_INDEX: return "expert index out of range";
    default: return "unknown status";
  }
}

const char* moe_last_error(void) { return moe::g_last_error; }

int moe_router_logits(const uint16_t* x, const uint16_t* wg, const uint16_t* bias, int64_t T, int32_t H, int32_t E,
                      uint16_t* logits, moe_stream_t stream) {
  return moe::router_logits(x, wg, bias, T, H, E, logits, reinterpret_cast<hipStream_t>(stream));
}

int moe_route(const uint16_t* logits, const float* score_bias, int64_t T,
              const moe_router_params* params, uint32_t* inds, float* scores,
              moe_stream_t stream) {
  if (params && moe::route_needs_bias(params->variant) && !score_bias) return MOE_E_INVALID_ARG;
  return moe::route(logits, score_bias, T, params, inds, scores,
                    reinterpret_cast<hipStream_t>(stream));
}

size_t moe_bucket_workspace_size(int64_t T, int32_t k, int32_t E) {
  if (T < 0 || k <= 0 || E <= 0) return 0;
  return moe::bucket_workspace_bytes(T * k, E);
}

int moe_bucket(const uint32_t* inds, int64_t T, int32_t k, int32_t E, int32_t* perm,
               int32_t* inv_perm, uint32_t* sorted_expert, int32_t* offsets, void* workspace,
               size_t workspace_bytes, moe_stream_t stream) {
  BucketOut o{perm, inv_perm, sorted_expert, nullptr, offsets, nullptr, nullptr};
  return moe::bucket(inds, T, k, E, o, workspace, workspace_bytes,
                     reinterpret_cast<hipStream_t>(stream));
}

static moe::Carve gqmm_layout(void* ws, int64_t n, int32_t E, int32_t gstride, uint32_t** pair_expert,
                              int32_t** perm, int32_t** offsets, int32_t** active,
                              int32_t** num_active, int32_t** in_rows, int32_t** tiles, float** gsum,
                              char** bws, size_t* bws_bytes) {
  moe::Carve c(ws);
  *pair_expert = c.take<uint32_t>(n);
  *perm = c.take<int32_t>(n);
  *offsets = c.take<int32_t>(E + 1);
  *active = c.take<int32_t>(4 * static_cast<int64_t>(E));
  *num_active = c.take<int32_t>(1);
  *in_rows = c.take<int32_t>(n);
  *tiles = c.take<int32_t>(moe::prefill_tile_ints(n, E));
  *gsum = c.take<float>(n * gstride);
  *bws_bytes = moe::bucket_workspace_bytes(n, E);
  *bws = c.raw(*bws_bytes);
  return c;
}

// The workspace covers the large-bucket GEMM's group sums for K up to 16384
// with group size 64 (256 groups per row, 256 words: each group sum is kept
// as two bf16 values, hi and lo).
constexpr int32_t kGqmmMaxGstride = 256;

size_t moe_gather_qmm_workspace_size(int64_t batch, int32_t M, int32_t num_experts) {
  if (batch < 0 || M <= 0 || num_experts <= 0) return 0;
  uint32_t* pe;
  int32_t *perm, *offs, *act, *na, *inr, *tiles;
  float* gsum;
  char* bws;
  size_t bb;
  return gqmm_layout(nullptr, batch * M, num_experts, kGqmmMaxGstride, &pe, &perm, &offs, &act, &na, &inr,
                     &tiles, &gsum, &bws, &bb)
      .size();
}

int moe_gather_qmm(const uint16_t* x, const moe_qweight* w, const uint32_t* lhs,
                   const uint32_t* rhs, int64_t batch, int32_t M, int32_t sorted_indices,
                   uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  (void)sorted_indices;
  int st = moe::qweight_check(w);
  if (st != MOE_OK) return st;
  if (batch < 0 || M <= 0) return MOE_E_INVALID_ARG;
  if (batch == 0) return MOE_OK;
  if (!x || !rhs || !out) return MOE_E_INVALID_ARG;
  const int64_t n = batch * M;
  if (n > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  const size_t need = moe_gather_qmm_workspace_size(batch, M, w->experts);
  if (!workspace || workspace_bytes < need) return MOE_E_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t* pe;
  int32_t *perm, *offs, *act, *na, *inr, *tiles;
  float* gsum;
  char* bws;
  size_t bb;
  gqmm_layout(workspace, n, w->experts, kGqmmMaxGstride, &pe, &perm, &offs, &act, &na, &inr, &tiles, &gsum,
              &bws, &bb);
  const unsigned nb = static_cast<unsigned>((n + 255) / 256);
  MOE_LAUNCH("expand_pairs", moe::expand_pairs, dim3(nb), dim3(256), 0, s, rhs, batch, M, w->experts, pe, out,
             w->N);
  MOE_CHECK_LAUNCH("gather_qmm.expand");
  const int slots = static_cast<int>(n < w->experts ? n : w->experts);
  const bool pf_ok = moe::prefill_gsum_stride(w) <= kGqmmMaxGstride;
  BucketOut o{perm, nullptr, nullptr, nullptr, offs, act, na};
  // the bucketing also writes the large-bucket GEMM's token-tile table
  const bool pf_tiles = pf_ok && moe::use_prefill(n, slots, w, nullptr);
  if (pf_tiles) o.tiles = tiles;
  st = moe::bucket(pe, n, 1, w->experts, o, bws, bb, s);
  if (st != MOE_OK) return st;
  MOE_LAUNCH("make_in_rows", moe::make_in_rows, dim3(nb), dim3(256), 0, s, perm, lhs, n, M, inr);
  MOE_CHECK_LAUNCH("gather_qmm.rows");
  moe::PrefillScratch pf{tiles, gsum, -1};
  pf.tiles_ready = pf_tiles;
  return moe::grouped_qmm(x, inr, perm, offs, act, na, slots, n, pf_ok ? &pf : nullptr, w, nullptr, out, s);
}

static moe::Carve gmm_layout(void* ws, int64_t n, int32_t E, uint32_t** pair_expert, int32_t** perm,
                             int32_t** offsets, int32_t** active, int32_t** num_active, int32_t** in_rows, char** bws,
                             size_t* bws_bytes) {
  moe::Carve c(ws);
  *pair_expert = c.take<uint32_t>(n);
  *perm = c.take<int32_t>(n);
  *offsets = c.take<int32_t>(E + 1);
  *active = c.take<int32_t>(4 * static_cast<int64_t>(E));
  *num_active = c.take<int32_t>(1);
  *in_rows = c.take<int32_t>(n);
  *bws_bytes = moe::bucket_workspace_bytes(n, E);
  *bws = c.raw(*bws_bytes);
  return c;
}

size_t moe_gather_mm_workspace_size(int64_t batch, int32_t M, int32_t num_experts) {
  if (batch < 0 || M <= 0 || num_experts <= 0) return 0;
  uint32_t* pe;
  int32_t *perm, *offs, *act, *na, *inr;
  char* bws;
  size_t bb;
  return gmm_layout(nullptr, batch * M, num_experts, &pe, &perm, &offs, &act, &na, &inr, &bws, &bb).size();
}

int moe_gather_mm(const uint16_t* x, const uint16_t* w, const uint16_t* linear_bias, int32_t num_experts, int32_t N,
                  int32_t K, const uint32_t* lhs, const uint32_t* rhs, int64_t batch, int32_t M,
                  int32_t sorted_indices, uint16_t* out, void* workspace, size_t workspace_bytes,
                  moe_stream_t stream) {
  (void)sorted_indices;
  if (batch < 0 || M <= 0 || num_experts <= 0 || N <= 0 || K <= 0) return MOE_E_INVALID_ARG;
  if (!w) return MOE_E_INVALID_ARG;
  if (K % 32 != 0 || (reinterpret_cast<uintptr_t>(w) & 15u)) return MOE_E_UNSUPPORTED;
  if (batch == 0) return MOE_OK;
  if (!x || !rhs || !out) return MOE_E_INVALID_ARG;
  const int64_t n = batch * M;
  if (n > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  const size_t need = moe_gather_mm_workspace_size(batch, M, num_experts);
  if (!workspace || workspace_bytes < need) return MOE_E_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint32_t* pe;
  int32_t *perm, *offs, *act, *na, *inr;
  char* bws;
  size_t bb;
  gmm_layout(workspace, n, num_experts, &pe, &perm, &offs, &act, &na, &inr, &bws, &bb);
  const unsigned nb = static_cast<unsigned>((n + 255) / 256);
  MOE_LAUNCH("expand_pairs", moe::expand_pairs, dim3(nb), dim3(256), 0, s, rhs, batch, M, num_experts, pe, out,
             N);
  MOE_CHECK_LAUNCH("gather_mm.expand");
  BucketOut o{perm, nullptr, nullptr, nullptr, offs, act, na};
  int st = moe::bucket(pe, n, 1, num_experts, o, bws, bb, s);
  if (st != MOE_OK) return st;
  MOE_LAUNCH("make_in_rows", moe::make_in_rows, dim3(nb), dim3(256), 0, s, perm, lhs, n, M, inr);
  MOE_CHECK_LAUNCH("gather_mm.rows");
  const int slots = static_cast<int>(n < num_experts ? n : num_experts);
  return moe::grouped_mm(x, inr, perm, act, slots, w, linear_bias, N, K, out, s);
}

int moe_add_rms_norm(const uint16_t* a, const uint16_t* b, const uint16_t* weight, float eps, int64_t T,
                     int32_t H, uint16_t* sum_out, uint16_t* normed_out, moe_stream_t stream) {
  return moe::add_rms_norm(a, b, weight, eps, T, H, sum_out, normed_out, reinterpret_cast<hipStream_t>(stream));
}

int moe_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h,
               moe_stream_t stream) {
  return moe::swiglu(gate, up, n, h, reinterpret_cast<hipStream_t>(stream));
}

int moe_gptoss_swiglu(const uint16_t* x_linear, const uint16_t* x_glu, int64_t n, uint16_t* h,
                      moe_stream_t stream) {
  return moe::gptoss_swiglu(x_linear, x_glu, n, h, reinterpret_cast<hipStream_t>(stream));
}

int moe_combine(const uint16_t* Y, const int32_t* inv_perm, const float* scores, int64_t T,
                int32_t k, int32_t H, uint16_t* y, moe_stream_t stream) {
  return moe::combine(Y, inv_perm, scores, T, k, H, nullptr, nullptr, y,
                      reinterpret_cast<hipStream_t>(stream));
}

int moe_take_rows(const void* src, int64_t src_rows, const int32_t* rows, int64_t n,
                  int32_t divisor, int64_t row_bytes, void* dst, moe_stream_t stream) {
  return moe::take_rows(src, src_rows, rows, n, divisor, row_bytes, dst,
                        reinterpret_cast<hipStream_t>(stream));
}

int moe_add_expert_bias(uint16_t* out, const uint16_t* bias, const uint32_t* rhs, int64_t batch,
                        int32_t M, int32_t N, int32_t num_experts, moe_stream_t stream) {
  return moe::add_expert_bias(out, bias, rhs, batch, M, N, num_experts,
                              reinterpret_cast<hipStream_t>(stream));
}

size_t moe_switch_glu_workspace_size(const moe_qweight* gate, const moe_qweight* down, int64_t T,
                                     int32_t k) {
  if (!gate || !down || T < 0 || k <= 0 || gate->experts <= 0) return 0;
  size_t total = 0;
  moe::plan_switch_glu(gate, down, T, k, nullptr, &total);
  return total;
}

int moe_switch_glu(const moe_qweight* gate, const moe_qweight* up, const moe_qweight* down,
                   const uint16_t* x, const uint32_t* inds, int64_t T, int32_t k, int32_t activation,
                   uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream) {
  int st = moe::switch_glu_validate(gate, up, down, k);
  if (st != MOE_OK) return st;
  if (!moe::activation_ok(activation)) return MOE_E_INVALID_ARG;
  if (T < 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!x || !inds || !out) return MOE_E_INVALID_ARG;
  const int64_t P = T * k;
  if (P > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  size_t need = 0;
  moe::plan_switch_glu(gate, down, T, k, nullptr, &need);
  if (!workspace || workspace_bytes < need) return MOE_E_WORKSPACE;
  moe::SwitchGluPlan p = moe::plan_switch_glu(gate, down, T, k, workspace, &need);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int E = gate->experts;
  const int slots = static_cast<int>(P < E ? P : E);
  const bool pf_up = moe::use_prefill(P, slots, gate, up), pf_down = moe::use_prefill(P, slots, down, nullptr);
  // the bucketing also writes the large-bucket GEMM's token-tile table (one for both GEMMs)
  p.bk.tiles = pf_up || pf_down ? p.tiles : nullptr;
  st = moe::bucket(inds, T, k, E, p.bk, p.bucket_ws, p.bucket_ws_bytes, s);
  if (st != MOE_OK) return st;
  const bool fuse_hsum = pf_up && pf_down;
  moe::PrefillScratch pf1{p.tiles, p.gsum, T, false, fuse_hsum ? p.hsum : nullptr, down};
  pf1.tiles_ready = p.bk.tiles != nullptr;
  pf1.xp = p.xp;
  pf1.act = activation;
  // h in pair K order for a down GEMM that reads it so
  const bool h_pairs = pf_down || down->bits == 4;
  pf1.out_p8 = h_pairs;
  st = moe::grouped_qmm(x, p.bk.sorted_token, nullptr, p.bk.offsets, p.bk.active, p.bk.num_active,
                        slots, P, &pf1, gate, up, p.h, s);
  if (st != MOE_OK) return st;
  // down writes each pair's row at its flat index t*k + j: out is [T, k, H]
  moe::PrefillScratch pf2{p.tiles, fuse_hsum ? p.hsum : p.gsum, P, fuse_hsum};
  pf2.tiles_ready = p.bk.tiles != nullptr;
  pf2.in_p8 = h_pairs;
  return moe::grouped_qmm(p.h, nullptr, p.bk.perm, p.bk.offsets, p.bk.active, p.bk.num_active, slots,
                          P, &pf2, down, nullptr, out, s);
}

size_t moe_switch_mlp_workspace_size(const moe_qweight* up, const moe_qweight* down, int64_t T, int32_t k) {
  return moe_switch_glu_workspace_size(up, down, T, k);
}

int moe_switch_mlp_relu2(const moe_qweight* up, const moe_qweight* down, const uint16_t* x, const uint32_t* inds,
                         int64_t T, int32_t k, uint16_t* out, void* workspace, size_t workspace_bytes,
                         moe_stream_t stream) {
  int st = moe::switch_glu_validate(up, up, down, k);
  if (st != MOE_OK) return st;
  if (T < 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!x || !inds || !out) return MOE_E_INVALID_ARG;
  const int64_t P = T * k;
  if (P > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  size_t need = 0;
  moe::plan_switch_glu(up, down, T, k, nullptr, &need);
  if (!workspace || workspace_bytes < need) return MOE_E_WORKSPACE;
  moe::SwitchGluPlan p = moe::plan_switch_glu(up, down, T, k, workspace, &need);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int E = up->experts;
  const int slots = static_cast<int>(P < E ? P : E);
  const bool pf1_ = moe::use_prefill(P, slots, up, nullptr), pf2_ = moe::use_prefill(P, slots, down, nullptr);
  p.bk.tiles = pf1_ || pf2_ ? p.tiles : nullptr;
  st = moe::bucket(inds, T, k, E, p.bk, p.bucket_ws, p.bucket_ws_bytes, s);
  if (st != MOE_OK) return st;
  // fc1 over the sorted pairs (h [P, I] in sorted order), relu^2 in place, fc2
  // writing each pair's row at its flat index t*k + j
  moe::PrefillScratch pf1{p.tiles, p.gsum, T};
  pf1.tiles_ready = p.bk.tiles != nullptr;
  st = moe::grouped_qmm(x, p.bk.sorted_token, nullptr, p.bk.offsets, p.bk.active, p.bk.num_active, slots, P,
                        &pf1, up, nullptr, p.h, s);
  if (st != MOE_OK) return st;
  st = moe::relu_squared(p.h, P * up->N, p.h, s);
  if (st != MOE_OK) return st;
  moe::PrefillScratch pf2{p.tiles, p.gsum, P};
  pf2.tiles_ready = p.bk.tiles != nullptr;
  return moe::grouped_qmm(p.h, nullptr, p.bk.perm, p.bk.offsets, p.bk.active, p.bk.num_active, slots, P, &pf2,
                          down, nullptr, out, s);
}

size_t moe_block_workspace_size(const moe_block_desc* desc, int64_t T) {
  if (moe::block_validate(desc) != MOE_OK || T < 0) return 0;
  size_t total = 0;
  moe::plan_block(desc, T, nullptr, &total);
  return total;
}

namespace moe {
namespace {
// The block forward; pn != NULL: x (= pn->normed) is first produced from
// pn's a, b and weight by the residual add + RMSNorm -- inside the router
// projection's launch when that runs as partial sums over few tokens, else
// by add_rms_norm before it.
int block_forward(const moe_block_desc* d, const uint16_t* x, int64_t T, uint16_t* out, const moe_block_aux* aux,
                  void* workspace, size_t workspace_bytes, moe_stream_t stream, const NormIn* pn);
}  // namespace
}  // namespace moe

int moe_block_forward(const moe_block_desc* d, const uint16_t* x, int64_t T, uint16_t* out,
                      const moe_block_aux* aux, void* workspace, size_t workspace_bytes,
                      moe_stream_t stream) {
  return moe::block_forward(d, x, T, out, aux, workspace, workspace_bytes, stream, nullptr);
}

int moe_block_forward_add_norm(const moe_block_desc* d, const uint16_t* a, const uint16_t* b,
                               const uint16_t* norm_weight, float eps, int64_t T, uint16_t* sum_out,
                               uint16_t* normed_out, uint16_t* out, const moe_block_aux* aux, void* workspace,
                               size_t workspace_bytes, moe_stream_t stream) {
  if (!a || !b || !norm_weight || !sum_out || !normed_out || !(eps >= 0.0f)) return MOE_E_INVALID_ARG;
  const moe::NormIn nin{a, b, norm_weight, eps, sum_out, normed_out};
  return moe::block_forward(d, normed_out, T, out, aux, workspace, workspace_bytes, stream, &nin);
}

namespace moe {
namespace {
int block_forward(const moe_block_desc* d, const uint16_t* x, int64_t T, uint16_t* out, const moe_block_aux* aux,
                  void* workspace, size_t workspace_bytes, moe_stream_t stream, const NormIn* pn) {
  int st = moe::block_validate(d);
  if (st != MOE_OK) return st;
  if (T < 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!x || !out) return MOE_E_INVALID_ARG;
  const int64_t P = T * d->router.top_k;
  if (P > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  size_t need = 0;
  moe::plan_block(d, T, nullptr, &need);
  if (!workspace || workspace_bytes < need) return MOE_E_WORKSPACE;
  moe::BlockPlan p = moe::plan_block(d, T, workspace, &need);
  if (aux) {
    if (aux->logits) p.logits = aux->logits;
    if (aux->inds) p.inds = aux->inds;
    if (aux->scores) p.scores = aux->scores;
    if (aux->perm) p.bk.perm = aux->perm;
    if (aux->inv_perm) p.bk.inv_perm = aux->inv_perm;
    if (aux->offsets) p.bk.offsets = aux->offsets;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int E = d->num_experts, k = d->router.top_k;

  const int slots = static_cast<int>(P < E ? P : E);
  const bool qrouter = d->router_q.w != nullptr;
  // one-expert projections: the large-bucket GEMM where it applies (it reads
  // the bucket {0, T}), else the per-16-row kernel over 16-row slots
  const bool rq_large = qrouter && moe::use_prefill(T, 1, &d->router_q, nullptr);
  const bool sh_up_large = d->shared_intermediate > 0 && moe::use_prefill(T, 1, &d->shared_gate, &d->shared_up);
  const bool sh_down_large = d->shared_intermediate > 0 && moe::use_prefill(T, 1, &d->shared_down, nullptr);
  if (rq_large || sh_up_large || sh_down_large) {
    MOE_LAUNCH("shared_meta", moe::fill_shared_meta, dim3(1), dim3(64), 0, s, p.sh_offsets, p.sh_active,
               p.sh_num, static_cast<int>(T));
    MOE_CHECK_LAUNCH("shared.meta");
  }
  // when gate|up runs the large-bucket GEMM, the bf16 router projection (which
  // reads every row of x anyway) also writes the group sums of x that GEMM needs
  const bool fuse_sums =
      !qrouter && moe::router_tile32(T, d->hidden) && moe::use_prefill(P, slots, &d->gate, &d->up);
  const moe::RouterGroupSums sums{reinterpret_cast<uint16_t*>(p.gsum), d->gate.group_size,
                                  moe::prefill_gsum_stride(&d->gate) / 16};
  const bool pf_up = moe::use_prefill(P, slots, &d->gate, &d->up);
  const bool pf_down = moe::use_prefill(P, slots, &d->down, nullptr);
  // the bucketing also writes the large-bucket GEMM's token-tile table (one for both GEMMs)
  p.bk.tiles = pf_up || pf_down ? p.tiles : nullptr;
  // small batches: routing and bucketing in one workgroup, from the partial
  // sums of a router projection spread over many workgroups
  const bool small = moe::route_bucket_small_fits(T, &d->router, p.bk);
  // a few dozen tokens: the same partial sums, then one token per wave routes
  // from them (the logits are formed there) and the bucketing follows
  const bool mid = !small && moe::route_from_partials_fits(T, &d->router);
  const bool partials = (small || mid) && p.rks > 0;
  // the step before the block: inside the partial-sum projection for few
  // tokens, else a launch of its own before anything reads x
  const bool norm_fused = pn && partials && moe::router_partials_norm_fits(T, d->hidden, p.rks);
  const bool tparts = !qrouter && !partials && p.tks > 1 && moe::route_from_partials_fits_any(&d->router);
  if (pn && !norm_fused) {
    st = moe::add_rms_norm(pn->a, pn->b, pn->w, pn->eps, T, d->hidden, pn->sum_out, pn->normed, s);
    if (st != MOE_OK) return st;
  }
  if (qrouter) {  // linear_forward's quantized branch: the grouped kernels with one expert
    const moe::ProfScope scope(moe::ProfLabel::kRouterQ);
    moe::PrefillScratch pfr{p.sh_tiles, p.gsum, T};
    pfr.gemv_only = !rq_large;
    st = moe::grouped_qmm(x, nullptr, nullptr, p.sh_offsets, p.sh_active, p.sh_num,
                          rq_large ? 1 : moe::one_expert_slots(T), T, &pfr, &d->router_q, nullptr, p.logits, s);
  } else if (partials) {
    st = norm_fused ? moe::router_partials_norm(*pn, d->router_weight, T, d->hidden, E, p.rpart, p.rks, p.xp, s)
                    : moe::router_partials(x, d->router_weight, T, d->hidden, E, p.rpart, p.rks, p.xp, s);
  } else if (tparts) {
    // many tokens, the projection's grid one workgroup per CU or fewer: K split
    // over two workgroups (partial sums; the routing adds them and the bias)
    st = moe::router_partials_tile32(x, d->router_weight, T, d->hidden, E, p.tpart, p.tks,
                                     fuse_sums ? &sums : nullptr, p.xp, s);
  } else {
    // the projection also writes x in pair K order (the expert GEMMs' input)
    st = moe::router_logits(x, d->router_weight, d->router_bias, T, d->hidden, E, p.logits, s,
                            fuse_sums ? &sums : nullptr, p.xp);
  }
  if (st != MOE_OK) return st;
  // one token: gate|up routes it itself from the partial sums (one launch fewer)
  moe::PrefillScratch pf1{p.tiles, p.gsum, T};
  pf1.xp = p.xp;
  pf1.xp_ready = !qrouter;
  moe::FusedRoute froute{p.rpart, p.rks, d->router_bias, p.logits, d->score_bias, p.inds, p.scores, d->router, p.bk};
  const bool route_in_gemv = partials && moe::gate_up_route_fits(P, slots, pf1, &d->gate, &d->up, d->router, p.rks);
  if (route_in_gemv) {
    pf1.route = &froute;
  } else if (small) {
    st = moe::route_bucket_small(partials ? nullptr : p.logits, partials ? p.rpart : nullptr, p.rks,
                                 d->router_bias, p.logits, d->score_bias, T, &d->router, p.inds, p.scores, p.bk, s);
    if (st != MOE_OK) return st;
  } else if (moe::route_bucket_fits(T, &d->router)) {  // small batch: one launch
    st = moe::route_bucket(p.logits, d->score_bias, T, &d->router, p.inds, p.scores, p.bk, s);
    if (st != MOE_OK) return st;
  } else {
    st = partials  ? moe::route_from_partials(p.rpart, p.rks, d->router_bias, p.logits, d->score_bias, T, &d->router,
                                              p.inds, p.scores, s)
         : tparts ? moe::route_from_partials(p.tpart, p.tks, d->router_bias, p.logits, d->score_bias, T, &d->router,
                                             p.inds, p.scores, s, true)
                  : moe::route(p.logits, d->score_bias, T, &d->router, p.inds, p.scores, s);
    if (st != MOE_OK) return st;
    st = moe::bucket(p.inds, T, k, E, p.bk, p.bucket_ws, p.bucket_ws_bytes, s);
    if (st != MOE_OK) return st;
  }
  // when both expert GEMMs run the large-bucket path, gate|up also writes the
  // group sums of h that down reads
  const bool fuse_hsum = pf_up && pf_down;
  pf1.gsum_ready = fuse_sums;
  pf1.next_gsum = fuse_hsum ? p.hsum : nullptr;
  pf1.next_w = &d->down;
  pf1.tiles_ready = p.bk.tiles != nullptr;
  // (xp_ready false: the large-bucket GEMM writes x in pair order with the group sums)
  pf1.act = d->activation;
  // one token: down and the combine in one launch (h in natural K order)
  const bool dc_fused = T == 1 && !pf_down && moe::down_combine_one_fits(&d->down, k);
  // h in pair K order for a down GEMM that reads it so
  const bool h_pairs = !dc_fused && (pf_down || d->down.bits == 4);
  pf1.out_p8 = h_pairs;
  st = moe::grouped_qmm(x, p.bk.sorted_token, nullptr, p.bk.offsets, p.bk.active, p.bk.num_active,
                        slots, P, &pf1, &d->gate, &d->up, p.h, s);
  if (st != MOE_OK) return st;
  if (d->shared_intermediate > 0) {
    const moe::ProfScope scope(moe::ProfLabel::kShared);
    if (d->shared_gate_q.w) {  // linear_forward's quantized branch for the gate (qwen3_next.cpp:488)
      st = moe::qrow(x, T, &d->shared_gate_q, p.sgl, s);
      if (st != MOE_OK) return st;
    } else if (d->shared_gate_weight) {
      st = moe::router_logits(x, d->shared_gate_weight, nullptr, T, d->hidden, 1, p.sgl, s);
      if (st != MOE_OK) return st;
    }
    const bool sh_down = sh_down_large;
    moe::PrefillScratch pf3{p.sh_tiles, p.gsum, T};
    pf3.xp = p.xp;
    pf3.xp_ready = !qrouter || pf_up;  // written by the bf16 router projection or by gate|up's group-sum pass
    const bool sh_pairs = sh_down || d->shared_down.bits == 4;
    pf3.out_p8 = sh_pairs;
    pf3.gemv_only = !sh_up_large;
    st = moe::grouped_qmm(x, nullptr, nullptr, p.sh_offsets, p.sh_active, p.sh_num,
                          sh_up_large ? 1 : moe::one_expert_slots(T), T, &pf3, &d->shared_gate, &d->shared_up,
                          p.hs, s);
    if (st != MOE_OK) return st;
    moe::PrefillScratch pf4{p.sh_tiles, p.gsum, T};
    pf4.in_p8 = sh_pairs;
    pf4.gemv_only = !sh_down;
    st = moe::grouped_qmm(p.hs, nullptr, nullptr, p.sh_offsets, p.sh_active, p.sh_num,
                          sh_down ? 1 : moe::one_expert_slots(T), T, &pf4, &d->shared_down, nullptr, p.Ys, s);
    if (st != MOE_OK) return st;
  }
  const uint16_t* Ys = d->shared_intermediate > 0 ? p.Ys : nullptr;
  const uint16_t* sgl =
      d->shared_intermediate > 0 && (d->shared_gate_weight || d->shared_gate_q.w) ? p.sgl : nullptr;
  if (dc_fused) return moe::down_combine_one(p.h, p.bk.perm, p.bk.active, p.scores, k, &d->down, Ys, sgl, out, s);
  // down writes each pair's row of Y at its flat index t*k + j (row perm[pos]),
  // so the combine reads a token's k rows without a lookup
  moe::PrefillScratch pf2{p.tiles, fuse_hsum ? p.hsum : p.gsum, P, fuse_hsum};
  pf2.tiles_ready = p.bk.tiles != nullptr;
  pf2.in_p8 = h_pairs;
  st = moe::grouped_qmm(p.h, nullptr, p.bk.perm, p.bk.offsets, p.bk.active, p.bk.num_active, slots,
                        P, &pf2, &d->down, nullptr, p.Y, s);
  if (st != MOE_OK) return st;
  return moe::combine(p.Y, nullptr, p.scores, T, k, d->hidden, Ys, sgl, out, s);
}
}  // namespace
}  // namespace moe

namespace moe {
namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, looked up once per device
// with that device current.
int static_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_last_error("moe_block_forward_noalloc: hipGetDevice", e);
    return MOE_E_HIP;
  }
  hipDevice_t sdev = -1;
  e = hipStreamGetDevice(stream, &sdev);
  if (e != hipSuccess) {
    set_last_error("moe_block_forward_noalloc: hipStreamGetDevice", e);
    return MOE_E_HIP;
  }
  if (sdev != dev) {
    std::snprintf(g_last_error, sizeof(g_last_error),
                  "moe_block_forward_noalloc: stream of device %d, current device %d", static_cast<int>(sdev), dev);
    return MOE_E_INVALID_ARG;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) return MOE_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // the lookup may load the library's code object onto the device: never
    // inside a stream capture (the first call on a device must be eager)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) {
      set_last_error("moe_block_forward_noalloc: hipStreamIsCapturing", e);
      return MOE_E_HIP;
    }
    if (cs != hipStreamCaptureStatusNone) {
      std::snprintf(g_last_error, sizeof(g_last_error),
                    "moe_block_forward_noalloc: the first call on device %d is under stream capture; make one "
                    "eager call first",
                    dev);
      return MOE_E_INVALID_ARG;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_last_error("moe_block_forward_noalloc: hipGetSymbolAddress(scratch)", e);
      return MOE_E_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}
}  // namespace
}  // namespace moe

extern "C" {

int moe_block_forward_noalloc(const moe_block_desc* d, const uint16_t* x, int64_t T, uint16_t* out,
                              const moe_block_aux* aux, moe_stream_t stream) {
  int st = moe::block_validate(d);
  if (st != MOE_OK) return st;
  if (T < 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!x || !out) return MOE_E_INVALID_ARG;
  const size_t need = moe_block_workspace_size(d, T);
  if (need == 0) return MOE_E_INVALID_ARG;
  if (need > kStaticScratchBytes) {
    std::snprintf(moe::g_last_error, sizeof(moe::g_last_error),
                  "moe_block_forward_noalloc: T = %lld needs %zu bytes of scratch; the static scratch holds %zu",
                  static_cast<long long>(T), need, kStaticScratchBytes);
    return MOE_E_WORKSPACE;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  st = moe::static_scratch(s, &ws);
  if (st != MOE_OK) return st;
  return moe_block_forward(d, x, T, out, aux, ws, kStaticScratchBytes, stream);
}

}  // extern "C"

struct moe_block_graph_s {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

int moe_block_graph_create(const moe_block_desc* d, const uint16_t* x, int64_t T, uint16_t* out, void* workspace,
                           size_t workspace_bytes, moe_block_graph* graph) {
  if (!graph) return MOE_E_INVALID_ARG;
  *graph = nullptr;
  int st = moe::block_validate(d);
  if (st != MOE_OK) return st;
  if (T <= 0 || !x || !out) return MOE_E_INVALID_ARG;
  size_t need = moe_block_workspace_size(d, T);
  if (!workspace || workspace_bytes < need) return MOE_E_WORKSPACE;
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) {
    moe::set_last_error("moe_block_graph_create", e);
    return MOE_E_HIP;
  }
  moe_block_graph_s g;
  e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (e == hipSuccess) {
    st = moe_block_forward(d, x, T, out, nullptr, workspace, workspace_bytes, s);
    e = hipStreamEndCapture(s, &g.graph);  // ends the capture also after a failed enqueue
  }
  if (e == hipSuccess && st == MOE_OK) e = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
  (void)hipStreamDestroy(s);
  if (e != hipSuccess || st != MOE_OK) {
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (g.graph) (void)hipGraphDestroy(g.graph);
    if (st != MOE_OK) return st;
    moe::set_last_error("moe_block_graph_create", e);
    return MOE_E_HIP;
  }
  *graph = new moe_block_graph_s(g);
  return MOE_OK;
}

int moe_block_graph_launch(moe_block_graph graph, moe_stream_t stream) {
  if (!graph || !graph->exec) return MOE_E_INVALID_ARG;
  const hipError_t e = hipGraphLaunch(graph->exec, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) {
    moe::set_last_error("moe_block_graph_launch", e);
    return MOE_E_HIP;
  }
  return MOE_OK;
}

int moe_block_graph_destroy(moe_block_graph graph) {
  if (!graph) return MOE_OK;
  if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
  if (graph->graph) (void)hipGraphDestroy(graph->graph);
  delete graph;
  return MOE_OK;
}

}  // extern "C"
