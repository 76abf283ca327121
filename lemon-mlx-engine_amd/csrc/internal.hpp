// internal.hpp -- declarations shared between the library's translation units
// (not part of the public C ABI).
#pragma once

#include <algorithm>

#include "common.hpp"

namespace moe {

// Outputs of the bucketing step; any pointer except offsets may be NULL.
// Token-tile table of the large-bucket GEMM, built per forward from the
// bucket sizes.  Expert e's bucket of c rows is cut into c / 128 tiles of 128
// rows and one tile for the remainder, its height the remainder rounded up to
// 32 rows: 4 units of 32 -> a partial 128-row tile, 3 -> 96 rows, 2 -> 64, 1
// -> 32 (one tile of the rounded height lives shorter than two smaller ones:
// at the Qwen3 shape a 128-row tile 69 us against 51 + 34 us for a 64- and a
// 32-row tile).  int4 0 = {n4, n3, n2, n1} (tiles of 128, 96, 64 and 32
// rows); int4 1 + i = tile i {expert, first sorted row, rows, 0}: the n4
// 128-row tiles (experts in order), then the n3 96-row, the n2 64-row and the
// n1 32-row tiles.
__device__ __forceinline__ void tile_counts(int c, int& c4, int& c3, int& c2, int& c1) {
  const int units = ((c & 127) + 31) >> 5;
  c4 = (c >> 7) + (units == 4 ? 1 : 0);
  c3 = units == 3 ? 1 : 0;
  c2 = units == 2 ? 1 : 0;
  c1 = units == 1 ? 1 : 0;
}
// Expert e's entries (bucket at sorted row o0, c rows); b4/b3/b2/b1 = its
// first index within each class, n4/n3/n2 = the class totals.
__device__ __forceinline__ void write_tiles(int32_t* tiles, int e, int o0, int c, int c4, int c3, int c2, int c1,
                                            int b4, int b3, int b2, int b1, int n4, int n3, int n2) {
  int4* tab = reinterpret_cast<int4*>(tiles) + 1;
  for (int j = 0; j < c4; ++j) tab[b4 + j] = make_int4(e, o0 + 128 * j, min(128, c - 128 * j), 0);
  const int rem0 = o0 + 128 * (c >> 7), r = c & 127;
  if (c3) tab[n4 + b3] = make_int4(e, rem0, r, 0);
  if (c2) tab[n4 + n3 + b2] = make_int4(e, rem0, r, 0);
  if (c1) tab[n4 + n3 + n2 + b1] = make_int4(e, rem0, r, 0);
}

struct BucketOut {
  int32_t* perm;           // [P]   sorted position -> flat pair index
  int32_t* inv_perm;       // [P]   flat pair index -> sorted position
  uint32_t* sorted_expert; // [P]
  int32_t* sorted_token;   // [P]   perm / k
  int32_t* offsets;        // [E+1]
  int32_t* active;         // [E][4] slot records {expert, first sorted row, rows, 0}: the
                           //       experts with a non-empty bucket, ascending, then rows = 0
  int32_t* num_active;     // [1]
  int32_t* tiles = nullptr;  // optional: the large-bucket GEMM's token-tile table (prefill_tile_ints)
};

// Group sums of x produced by the router projection for the expert GEMM
// (layout of prefill_gsum_stride: nch 16-group chunks of 2 bf16 planes, hi and
// lo, per row).
struct RouterGroupSums {
  uint16_t* xhl;
  int gs, nch;
};
// Token counts from which the router projection runs the 32x128-tile kernel
// (the only one that can also emit group sums).
constexpr int64_t kRouterTile32MinT = 512;
bool router_tile32(int64_t T, int32_t H);
// logits = bf16(x . wg^T + bias) (bias [E] or NULL: one rounding either way)
int router_logits(const uint16_t* x, const uint16_t* wg, const uint16_t* bias, int64_t T, int32_t H, int32_t E,
                  uint16_t* logits, hipStream_t stream, const RouterGroupSums* sums = nullptr,
                  uint16_t* xp = nullptr);
int route_validate(const moe_router_params* p);
// The variants that read the score-correction bias.
inline bool route_needs_bias(int variant) {
  return variant == MOE_ROUTE_SIGMOID_GROUP || variant == MOE_ROUTE_SIGMOID_GROUP_DROP_BEST ||
         variant == MOE_ROUTE_SIGMOID_CORRECTED || variant == MOE_ROUTE_GLM4_SIGMOID ||
         variant == MOE_ROUTE_GLM4_SOFTMAX;
}
int route(const uint16_t* logits, const float* bias, int64_t T, const moe_router_params* p,
          uint32_t* inds, float* scores, hipStream_t stream);
// Routing and bucketing of a small batch in one launch (T <= kRouteBucketMaxT,
// one token per wave of the workgroup; E <= 512): same outputs as route()
// followed by bucket().
constexpr int64_t kRouteBucketMaxT = 16;
bool route_bucket_fits(int64_t T, const moe_router_params* p);
int route_bucket(const uint16_t* logits, const float* bias, int64_t T, const moe_router_params* p,
                 uint32_t* inds, float* scores, const BucketOut& o, hipStream_t stream);
// Small batches (T <= kRouterPartialMaxT): the router projection as fp32
// partial sums over ks slices of H (router_partial_ks: 0 = not available for
// this shape), part [ks][T][E].  Up to kRouteSmallMaxT tokens
// route_bucket_small then forms the bf16 logits (into logits_out) from them
// plus the router bias rbias ([E] or NULL), or reads `logits` when part is
// NULL, routes and buckets in one workgroup (no token-tile table); above it
// route_from_partials routes one token per wave from them, and bucket()
// follows.
constexpr int64_t kRouterPartialMaxT = 64;
constexpr int64_t kRouteSmallMaxT = 16;
int router_partial_ks(int64_t T, int32_t E, int32_t H);
int router_partials(const uint16_t* x, const uint16_t* wg, int64_t T, int32_t H, int32_t E, float* part, int ks,
                    uint16_t* xp, hipStream_t stream);
// The step before the block (add_rms_norm) as the router projection's input:
// normed = bf16(bf16(a + b) * scale * w) with add_rms_norm's scale, written
// with sum_out = bf16(a + b); the projection reads the normed values it forms.
struct NormIn {
  const uint16_t* a;
  const uint16_t* b;
  const uint16_t* w;
  float eps;
  uint16_t* sum_out;
  uint16_t* normed;
};
// Up to kNormFuseMaxT tokens the partial-sum projection also runs the step
// before the block (every workgroup reads the whole rows of its tokens once
// for their scales); bit-identical to add_rms_norm then router_partials.
constexpr int64_t kNormFuseMaxT = 16;
bool router_partials_norm_fits(int64_t T, int32_t H, int ks);
int router_partials_norm(const NormIn& nin, const uint16_t* wg, int64_t T, int32_t H, int32_t E, float* part,
                         int ks, uint16_t* xp, hipStream_t stream);
bool route_from_partials_fits(int64_t T, const moe_router_params* p);
// any_t: any token count (the many-token projection's partial sums), else
// route_from_partials_fits
int route_from_partials(const float* part, int ks, const uint16_t* rbias, uint16_t* logits_out, const float* bias,
                        int64_t T, const moe_router_params* p, uint32_t* inds, float* scores, hipStream_t stream,
                        bool any_t = false);
// The many-token router projection (router_tile32) with K split over ks
// workgroups: fp32 partial sums part [ks][T][E] (no bias), plus the group sums
// and x in pair order as router_logits writes them; router_tile32_ks gives ks
// (1: use router_logits)
int router_tile32_ks(int64_t T, int32_t E, int32_t H, int gs);
// whether route_from_partials (any_t) routes this router's experts
bool route_from_partials_fits_any(const moe_router_params* p);
int router_partials_tile32(const uint16_t* x, const uint16_t* wg, int64_t T, int32_t H, int32_t E, float* part,
                           int ks, const RouterGroupSums* sums, uint16_t* xp, hipStream_t stream);
bool route_bucket_small_fits(int64_t T, const moe_router_params* p, const BucketOut& o);
int route_bucket_small(const uint16_t* logits, const float* part, int ks, const uint16_t* rbias,
                       uint16_t* logits_out, const float* bias, int64_t T, const moe_router_params* p, uint32_t* inds,
                       float* scores, const BucketOut& o, hipStream_t stream);
size_t bucket_workspace_bytes(int64_t P, int E);
int bucket(const uint32_t* inds, int64_t T, int k, int E, const BucketOut& o, void* ws,
           size_t ws_bytes, hipStream_t stream);
int qweight_check(const moe_qweight* w);
// Scratch of the large-bucket (prefill) GEMM path.
// One token (T = 1) routed inside the per-16-row gate|up kernel: every
// workgroup forms the bf16 logits from the router's partial sums, routes the
// token and sorts its k experts into the grid's slot records itself (no wait
// between workgroups); workgroup 0 also writes the logits, inds, scores and
// the bucketing outputs, exactly what route_bucket_small writes, for the
// kernels after it.  Replaces the route_bucket_small launch between the
// router projection and gate|up (see gate_up_route_fits).
struct FusedRoute {
  const float* part = nullptr;       // [ks][E] fp32 partial sums (router_partials)
  int ks = 0;
  const uint16_t* rbias = nullptr;   // router bias [E] or NULL
  uint16_t* logits_out = nullptr;    // [E] bf16 logits
  const float* score_bias = nullptr; // score-correction bias [E] or NULL
  uint32_t* inds = nullptr;          // [k]
  float* scores = nullptr;           // [k]
  moe_router_params params{};
  BucketOut o{};
};

struct PrefillScratch {
  int32_t* tiles;   // [prefill_tile_ints(P, E)] token tile table
  float* gsum;      // [max(x_rows, P) * prefill_gsum_stride] 4-byte words: group sums as bf16 hi/lo planes
  int64_t x_rows;   // rows of x if known, else -1
  bool gsum_ready = false;  // gsum already holds the sums of x's rows (x_rows >= 0)
  // gate|up GEMM only: also write the group sums of its output rows (h), for
  // the projection next_w that reads h, into next_gsum (rows = output rows)
  float* next_gsum = nullptr;
  const moe_qweight* next_w = nullptr;
  bool tiles_ready = false;  // tiles already holds the table for these offsets
  // Pair K order (within 8 consecutive K values: 0, 4, 1, 5, 2, 6, 3, 7): the
  // GEMM reads its operand of 4-bit codes in it at 7 instead of 9 VALU
  // instructions per code word.  gate|up (w1 != NULL) reads its input from
  // xp [x_rows, K], x in pair order, written with the group sums unless
  // gsum_ready (then the router projection wrote both); out_p8: gate|up writes
  // h in pair order (for a down GEMM that reads it so: large-bucket, or 4-bit
  // per-16-row); in_p8: down's input rows are in pair order.  The per-16-row
  // kernel (4-bit) reads x from xp when xp_ready.
  uint16_t* xp = nullptr;
  bool xp_ready = false;  // xp already holds x in pair order (the router projection wrote it)
  bool out_p8 = false;
  bool in_p8 = false;
  // one expert's P rows on the per-16-row kernel even where the large-bucket
  // GEMM would apply, spread over one_expert_slots(P) slots of equal height
  // (a multiple of 16 rows; the last slots may hold fewer or none) whose
  // records the kernel derives itself
  bool gemv_only = false;
  // gate|up: moe_activation of h = act(gate, up)
  int act = MOE_ACT_SWIGLU;
  // gate|up at one token: route it in the kernel (gate_up_route_fits)
  const FusedRoute* route = nullptr;
};
constexpr int kOneExpertSlots = 64;
inline int one_expert_slots(int64_t P) { return static_cast<int>(std::min<int64_t>((P + 15) / 16, kOneExpertSlots)); }

// Grouped dequant matmul over expert buckets.  P = total rows; `pf` (may be
// NULL) enables the large-bucket GEMM path.
int grouped_qmm(const uint16_t* x, const int32_t* row_in, const int32_t* row_out,
                const int32_t* offsets, const int32_t* active, const int32_t* num_active,
                int slots, int64_t P, const PrefillScratch* pf, const moe_qweight* w0,
                const moe_qweight* w1, uint16_t* out, hipStream_t stream);
bool prefill_supported(const moe_qweight* w0, const moe_qweight* w1);
int prefill_gsum_stride(const moe_qweight* w);
int64_t prefill_tile_ints(int64_t P, int E);
bool use_prefill(int64_t P, int slots, const moe_qweight* w0, const moe_qweight* w1);
// Whether grouped_qmm's gate|up launch for these arguments can route a single
// token itself (pf.route): one token (P = k = slots), 4-bit codes with x in
// pair K order, the per-16-row kernel with K split over four waves, E <= 512.
bool gate_up_route_fits(int64_t P, int slots, const PrefillScratch& pf, const moe_qweight* gate,
                        const moe_qweight* up, const moe_router_params& rp, int ks);
int grouped_gemm_prefill(const uint16_t* x, const int32_t* row_in, const int32_t* row_out, const PrefillScratch& pf,
                         const int32_t* offsets, int E, int64_t P, int slots, const moe_qweight* w0,
                         const moe_qweight* w1, uint16_t* out, hipStream_t stream);
// Grouped dense (bf16) matmul over expert buckets (gather_mm): out[row_out[pos]]
// = x[row_in[pos]] . w[e]^T (+ linear_bias[e]) for the rows of each slot record.
int grouped_mm(const uint16_t* x, const int32_t* row_in, const int32_t* row_out, const int32_t* active, int slots,
               const uint16_t* w, const uint16_t* linear_bias, int N, int K, uint16_t* out, hipStream_t stream);
// y[T] = bf16(x . dequant(w)^T) for a single quantized row w (experts 1, N 1)
int qrow(const uint16_t* x, int64_t T, const moe_qweight* w, uint16_t* y, hipStream_t stream);
int swiglu(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* h, hipStream_t stream);
// GPT-OSS's clipped SwiGLU, h = bf16(gptoss_glu(xl, xg)) (gptoss.cpp:50-58)
int gptoss_swiglu(const uint16_t* xl, const uint16_t* xg, int64_t n, uint16_t* h, hipStream_t stream);
int relu_squared(const uint16_t* in, int64_t n, uint16_t* out, hipStream_t stream);
int add_rms_norm(const uint16_t* a, const uint16_t* b, const uint16_t* w, float eps, int64_t T, int H,
                 uint16_t* sum_out, uint16_t* normed, hipStream_t stream);
int combine(const uint16_t* Y, const int32_t* inv_perm, const float* scores, int64_t T, int k,
            int H, const uint16_t* Ys, const uint16_t* sgl, uint16_t* y, hipStream_t stream);
// One token: down projection of its k expert rows (h in sorted order, natural
// K order) and the combine in one launch; fits: the shapes it takes.
bool down_combine_one_fits(const moe_qweight* w, int k);
int down_combine_one(const uint16_t* h, const int32_t* perm, const int32_t* active, const float* scores, int k,
                     const moe_qweight* w, const uint16_t* Ys, const uint16_t* sgl, uint16_t* out,
                     hipStream_t stream);
int take_rows(const void* src, int64_t src_rows, const int32_t* rows, int64_t n, int32_t divisor,
              int64_t row_bytes, void* dst, hipStream_t stream);
int add_expert_bias(uint16_t* out, const uint16_t* bias, const uint32_t* rhs, int64_t batch, int32_t M,
                    int32_t N, int32_t E, hipStream_t stream);

}  // namespace moe
