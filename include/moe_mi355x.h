/*
 * moe_mi355x.h -- C ABI of the MI355X-native quantized mixture-of-experts
 * block (router, top-k, expert bucketing, grouped 4/8-bit affine-dequant
 * matmuls with SwiGLU, weighted combine, shared expert).
 *
 * Every entry point is extern "C", takes plain device pointers and sizes, never
 * throws, and returns an int status (MOE_OK or a negative MOE_E_* code).  Work
 * is enqueued on the caller's HIP stream and is asynchronous; device buffers
 * are owned by the caller.  Entry points that need scratch memory take a
 * caller-provided workspace whose size is given by the matching
 * *_workspace_size() query, so calls on distinct workspaces and streams are
 * re-entrant.
 *
 * Data formats (reference include/mlx-lm/common/quantized_linear.h:16-21 and
 * the MLX affine layout restated in debug_numerical_trace.py:67-98):
 *   bf16      uint16_t bit pattern of a bfloat16.
 *   qweight   packed uint32 [E, N, K*bits/32]; element c of a row is bits
 *             [c*bits, c*bits + bits) of the row's little-endian bit stream,
 *             least significant first (2, 4, 8 bits: word c/(32/bits) at bit
 *             (c%(32/bits))*bits; 3 / 5 / 6 bits: eight / eight / four codes
 *             per three / five / three bytes);
 *             scales and biases bf16 [E, N, K/group_size]; w = s*q + b.
 *             bits in {2, 3, 4, 5, 6, 8} (MLX's affine widths: 4, 6, 8 are the
 *             ones examples/convert.cpp:10 emits and examples/test_qbits.cpp:45
 *             runs gather_qmm at; its --bits option takes the others); K a
 *             multiple of 128 at 3 and 5 bits; group_size 32, 64 or 128.
 *             Widths other than 4 and 8, and group size 32, run on the
 *             per-16-row kernel at every bucket size (the large-bucket GEMM
 *             is 4/8-bit with groups of 64 or 128).
 *
 * Host code above this ABI (the C++ SwitchLinear / SwitchGLU classes in
 * lemon-mlx-engine_amd/host/) keeps the reference's module interface; this
 * header is the device boundary those classes call.
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Version of this ABI: moe_version() returns it.  Bumped whenever a struct
 * layout or an entry point's signature changes, so a binding can refuse a
 * library built from another header (3: moe_block_desc.activation,
 * moe_switch_glu's activation argument, moe_gptoss_swiglu). */
#define MOE_ABI_VERSION 3

/* hipStream_t without pulling in the HIP headers (same underlying type). */
typedef struct ihipStream_t* moe_stream_t;

enum moe_status {
  MOE_OK = 0,
  MOE_E_INVALID_ARG = -1, /* null pointer, negative size, inconsistent shape  */
  MOE_E_UNSUPPORTED = -2, /* bits / group size / E / k outside supported set  */
  MOE_E_WORKSPACE = -3,   /* workspace pointer null or smaller than required  */
  MOE_E_HIP = -4,         /* a HIP runtime call or kernel launch failed       */
  MOE_E_INDEX = -6        /* an expert index >= num_experts (host-visible)    */
};

/* Router variants.  Each one restates one of the reference's routers. */
enum moe_route_variant {
  /* R1: top-k of the logits, weights = softmax over all experts gathered,
   * optional renorm.  src/llm/models/qwen3_moe.cpp:155-168 */
  MOE_ROUTE_TOPK_LOGITS = 1,
  /* R2: top-k of the softmax probabilities, optional renorm.
   * src/llm/models/qwen3_next.cpp:452-469 */
  MOE_ROUTE_TOPK_PROBS = 2,
  /* R3/R4: top-k of the logits, weights = softmax over the k selected.
   * src/llm/models/phimoe.cpp:93-101; src/common/gated_delta.cpp:385-422 */
  MOE_ROUTE_SOFTMAX_TOPK = 3,
  /* R5: DeepSeek-V3 gate as written: bf16 sigmoid, top-k, renorm * scale.
   * src/llm/models/deepseek_v3.cpp:304-350 */
  MOE_ROUTE_SIGMOID = 5,
  /* R6: sigmoid + score-correction bias + group-limited top-k (the
   * topk_group best groups kept, the upstream DeepSeek noaux_tc rule), renorm,
   * routed scaling.  src/llm/models/nemotron_h.cpp:405-468 */
  MOE_ROUTE_SIGMOID_GROUP = 6,
  /* R6 exactly as src/llm/models/nemotron_h.cpp:425-447 writes it: the group
   * scores are negated before argpartition, so the n_group - topk_group BEST
   * groups are the ones zeroed; otherwise as R6. */
  MOE_ROUTE_SIGMOID_GROUP_DROP_BEST = 7,
  /* Bailing (src/llm/models/bailing_moe.cpp:173-199): top-k of sigmoid +
   * correction bias with no group limit (its group index is never applied);
   * the weights are those corrected scores, renormalised (+1e-20) when k > 1
   * and norm_topk_prob, times routed_scaling_factor, rounded to bf16. */
  MOE_ROUTE_SIGMOID_CORRECTED = 8,
  /* GLM4-MoE's gate (src/llm/models/glm4_moe.cpp:158-191), scoring_func
   * "sigmoid" / "softmax": fp32 scores of the bf16 logits, top-k of scores +
   * correction bias with no group limit (its group index is computed but
   * never applied, :168-188), weights = the uncorrected scores, divided by
   * their sum (no epsilon) when k > 1 and norm_topk_prob, times
   * routed_scaling_factor, fp32. */
  MOE_ROUTE_GLM4_SIGMOID = 9,
  MOE_ROUTE_GLM4_SOFTMAX = 10,
  /* LFM2-MoE (src/llm/models/lfm2_moe.cpp:219-238): fp32 softmax of the bf16
   * logits plus the expert bias (score_bias, or none when NULL), top-k of
   * those biased probabilities, which are also the weights: divided by their
   * sum + 1e-20 when norm_topk_prob (for any k), then rounded to bf16; no
   * routed scaling. */
  MOE_ROUTE_LFM2 = 11
};

/* GLU activation of the routed experts' MLP, applied to the bf16 gate value
 * g and up value u (each the projection output, plus its SwitchLinear bias):
 *   MOE_ACT_SWIGLU          h = silu(g) * u (include/mlx-lm/common/activations.h:22-30)
 *   MOE_ACT_GPTOSS          GPT-OSS's clipped SwiGLU swiglu(x_linear, x_glu)
 *                           of src/llm/models/gptoss.cpp:50-58 as the MoE MLP
 *                           calls it, swiglu(x_gate, x_up) (:158): x_linear = g,
 *                           x_glu = u; h = xg * sigmoid(1.702 xg) * (xl + 1) with
 *                           xl = clip(x_linear, -7, 7), xg = min(x_glu, 7)
 *   MOE_ACT_GPTOSS_UPSTREAM the same function with the roles of the upstream
 *                           GPT-OSS MLP (x_linear = u, x_glu = g)
 * h is stored as bf16 (the reference's fp32 scalar operands promote its GPT-OSS
 * h to fp32; the difference is at most half a bf16 ulp of h per element). */
enum moe_activation {
  MOE_ACT_SWIGLU = 0,
  MOE_ACT_GPTOSS = 1,
  MOE_ACT_GPTOSS_UPSTREAM = 2
};

typedef struct moe_router_params {
  int32_t variant;        /* moe_route_variant                                */
  int32_t num_experts;    /* E  (<= 1024)                                     */
  int32_t top_k;          /* k  (1..16, <= E)                                 */
  int32_t norm_topk_prob; /* renormalise the k weights                        */
  int32_t n_group;        /* R6/R6' group count (1 = no group limit)          */
  int32_t topk_group;     /* R6/R6' topk_group                                */
  float routed_scaling_factor; /* R5-R8                                       */
} moe_router_params;

/* One stacked quantized projection [experts, N, K]. */
typedef struct moe_qweight {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases; /* may be NULL (treated as 0) */
  int32_t experts, N, K, group_size, bits;
  /* SwitchLinear's bias [experts, N] bf16, or NULL (zero-initialise to leave
   * it unused): every output becomes bf16(bf16(x . W^T) + linear_bias[e, n]),
   * the take(bias, indices) + add of src/common/switch_layers.cpp:111-114
   * (GPT-OSS, src/llm/models/gptoss.cpp:120-124). */
  const uint16_t* linear_bias;
} moe_qweight;

/* A whole MoE block.  gate and up are separate stacked projections [E, I, H]
 * (the kernel reads both, which is what the reference's lazily fused gate|up
 * weight buys, src/common/switch_layers.cpp:154-197, without the copy); down
 * is [E, H, I]. */
typedef struct moe_block_desc {
  int32_t hidden;          /* H */
  int32_t intermediate;    /* I */
  int32_t num_experts;     /* E */
  moe_router_params router;
  const uint16_t* router_weight; /* [E, H] bf16                               */
  const float* score_bias;       /* [E] fp32 (R6 correction bias) or NULL     */
  moe_qweight gate, up, down;
  int32_t shared_intermediate;   /* 0 = no shared expert                      */
  moe_qweight shared_gate, shared_up, shared_down; /* experts == 1           */
  const uint16_t* shared_gate_weight; /* [1, H] bf16 sigmoid gate, NULL = ungated */
  /* Quantized router projection (experts == 1, N == E, K == H), used instead
   * of router_weight when router_q.w != NULL: logits = bf16(x . dequant(Wq)^T),
   * the quantized branch of linear_forward (quantized_linear.h:73-96) that a
   * checkpoint with a quantized mlp.gate takes (examples/convert.cpp:56-60).
   * Zero-initialise to leave it unused. */
  moe_qweight router_q;
  /* Bias [E] bf16 of the bf16 router projection, or NULL: logits =
   * bf16(x . Wg^T + router_bias) with one rounding, addmm in linear_forward
   * (quantized_linear.h:86-94), GPT-OSS's router (gptoss.cpp:130).  A
   * quantized router takes its bias in router_q.linear_bias instead. */
  const uint16_t* router_bias;
  /* Quantized shared-expert gate [1][1, H] (experts == 1, N == 1, K == H),
   * used instead of shared_gate_weight when its w != NULL: the gate logit is
   * bf16(x . dequant(w)^T), linear_forward's quantized branch at
   * src/llm/models/qwen3_next.cpp:488 (MLX conversions quantize this gate).
   * Zero-initialise to leave it unused. */
  moe_qweight shared_gate_q;
  /* moe_activation of the routed experts (0 = SwiGLU).  The shared expert
   * always uses SwiGLU (every model with one does, qwen3_next.cpp:426-429,
   * deepseek_v3.cpp:366-369). */
  int32_t activation;
} moe_block_desc;

/* Optional device outputs of moe_block_forward (any member may be NULL). */
typedef struct moe_block_aux {
  uint16_t* logits;        /* [T, E] bf16 */
  uint32_t* inds;          /* [T, k] canonical slot order */
  float* scores;           /* [T, k] */
  int32_t* perm;           /* [T*k]  sorted position -> flat pair index */
  int32_t* inv_perm;       /* [T*k]  flat pair index -> sorted position */
  int32_t* offsets;        /* [E+1]  per-expert start in sorted order */
} moe_block_aux;

/* ---- library ---------------------------------------------------------- */
/* MOE_ABI_VERSION of the header the library was built from. */
int moe_version(void);
const char* moe_status_string(int status);
/* Last HIP error text recorded by a failing call on this thread. */
const char* moe_last_error(void);

/* ---- the step before the block: residual add + RMSNorm ----------------
 * sum_out[T, H] = bf16(a + b) (fp32 add); normed_out = bf16(sum_out *
 * rsqrt(mean((a + b)^2) + eps) * weight), the mean over the fp32 sums.  H a
 * multiple of 8, at most 8192; all pointers 16-byte aligned.
 * Replaces add_rms_norm(x, h, weight, eps), src/common/gated_delta.cpp:313-345
 * (kernel) as called at src/llm/models/qwen35_moe.cpp:787-788 to produce the
 * MoE input. */
int moe_add_rms_norm(const uint16_t* a, const uint16_t* b, const uint16_t* weight, float eps, int64_t T,
                     int32_t H, uint16_t* sum_out, uint16_t* normed_out, moe_stream_t stream);

/* ---- a1: router projection --------------------------------------------
 * logits[T, E] = bf16(x[T, H] . Wg[E, H]^T + bias[E]), fp32 accumulation and
 * one rounding; bias (bf16 [E]) may be NULL.
 * Replaces linear_forward(x, gate_weight, bias*) (dense branch: matmul, or
 * addmm with a bias), include/mlx-lm/common/quantized_linear.h:73-96, called
 * at src/llm/models/qwen3_moe.cpp:156 and (with a bias) gptoss.cpp:130. */
int moe_router_logits(const uint16_t* x, const uint16_t* wg, const uint16_t* bias, int64_t T, int32_t H,
                      int32_t E, uint16_t* logits, moe_stream_t stream);

/* ---- a2: scoring, top-k, renormalisation --------------------------------
 * inds[T, k] in canonical slot order (selection value descending, expert
 * index ascending); scores[T, k] fp32 (bf16-exact for R1-R4, whose reference
 * outputs are bf16).  score_bias [E] fp32 is read by R6 only.
 * Replaces moe_route(logits, k), include/mlx-lm/common/gated_delta.h:117-119
 * (src/common/gated_delta.cpp:973-998), and the per-model argpartition
 * routers listed in moe_route_variant. */
int moe_route(const uint16_t* logits, const float* score_bias, int64_t T,
              const moe_router_params* params, uint32_t* inds, float* scores,
              moe_stream_t stream);

/* ---- a3: expert bucketing ----------------------------------------------
 * Stable sort of the P = T*k flat pairs by expert id.  perm[pos] = flat pair
 * index at sorted position pos; inv_perm = perm^-1; sorted_expert[pos];
 * offsets[E+1] = exclusive scan of the expert histogram.  Any output may be
 * NULL except offsets.  Replaces gather_sort's argsort / argsort / take,
 * src/common/switch_layers.cpp:17-30. */
size_t moe_bucket_workspace_size(int64_t T, int32_t k, int32_t E);
int moe_bucket(const uint32_t* inds, int64_t T, int32_t k, int32_t E, int32_t* perm,
               int32_t* inv_perm, uint32_t* sorted_expert, int32_t* offsets, void* workspace,
               size_t workspace_bytes, moe_stream_t stream);

/* ---- a5/a7: grouped affine-dequant matmul (gather_qmm) ------------------
 * out[b, m, :] = x[lhs[b], m, :] . dequant(w[rhs[b]])^T for b < batch,
 * m < M, with x [*, M, K] bf16 and out [batch, M, N] bf16.  lhs NULL means
 * the identity over the batch.  lhs and rhs are the already-broadcast flat
 * index arrays of length batch.  sorted_indices asserts rhs is ascending (it
 * is accepted for contract parity; results do not depend on it).
 * Preconditions (not checked on the host: the indices live on the device):
 * lhs[b] indexes a row group of x; rhs[b] < w->experts, and an output row
 * whose rhs[b] is not is written as zeros (MLX leaves such an index
 * undefined).
 * Exactly the call at src/common/switch_layers.cpp:94-102 (transpose=true,
 * mode "affine"). */
size_t moe_gather_qmm_workspace_size(int64_t batch, int32_t M, int32_t num_experts);
int moe_gather_qmm(const uint16_t* x, const moe_qweight* w, const uint32_t* lhs,
                   const uint32_t* rhs, int64_t batch, int32_t M, int32_t sorted_indices,
                   uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* ---- gather_mm: the dense (unquantized) expert path ----------------------
 * out[b, m, :] = x[lhs[b], m, :] . w[rhs[b]]^T (+ linear_bias[rhs[b]]) for
 * b < batch, m < M: x [*, M, K] bf16, w [num_experts, N, K] bf16 (the
 * SwitchLinear weight as stored), out [batch, M, N] bf16, fp32 accumulation;
 * K a multiple of 32, x and w 16-byte aligned.  lhs NULL means the identity;
 * linear_bias [num_experts, N] bf16 or NULL, added to the bf16 product and
 * rounded again.  Index preconditions as for moe_gather_qmm (rows whose
 * rhs[b] >= num_experts are written as zeros).  Replaces SwitchLinear::operator()'s non-quantized branch,
 * mx::gather_mm(x, swapaxes(weight, -1, -2), lhs, rhs, sorted) plus its bias,
 * src/common/switch_layers.cpp:103-115. */
size_t moe_gather_mm_workspace_size(int64_t batch, int32_t M, int32_t num_experts);
int moe_gather_mm(const uint16_t* x, const uint16_t* w, const uint16_t* linear_bias, int32_t num_experts, int32_t N,
                  int32_t K, const uint32_t* lhs, const uint32_t* rhs, int64_t batch, int32_t M,
                  int32_t sorted_indices, uint16_t* out, void* workspace, size_t workspace_bytes,
                  moe_stream_t stream);

/* ---- a6: SwiGLU ----------------------------------------------------------
 * h = bf16(silu(g) * u) elementwise over n values.  Replaces swiglu(),
 * include/mlx-lm/common/activations.h:22-30. */
int moe_swiglu(const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* h,
               moe_stream_t stream);

/* ---- GPT-OSS's clipped SwiGLU ----------------------------------------------
 * h = bf16(xg * sigmoid(1.702 * xg) * (xl + 1)) elementwise over n values,
 * xl = clip(x_linear, -7, 7), xg = min(x_glu, 7), fp32 arithmetic.  Replaces
 * the file-local swiglu(x_linear, x_glu, alpha = 1.702, limit = 7) of
 * src/llm/models/gptoss.cpp:50-58; the GPT-OSS MoE MLP calls it as
 * swiglu(x_gate, x_up) (:158).  (The reference's h is fp32: see
 * moe_activation.) */
int moe_gptoss_swiglu(const uint16_t* x_linear, const uint16_t* x_glu, int64_t n, uint16_t* h,
                      moe_stream_t stream);

/* ---- a8/a9: unsort + weighted combine -------------------------------------
 * y[t, :] = bf16(sum_j scores[t, j] * Y[row(t, j), :]) where row(t, j) =
 * inv_perm[t*k + j] when inv_perm is given (Y in sorted order), else t*k + j
 * (Y in [T, k, H] order).  Replaces scatter_unsort
 * (src/common/switch_layers.cpp:32-46) plus the model-side
 * sum(y * scores, -2) (src/llm/models/qwen3_moe.cpp:173-174). */
int moe_combine(const uint16_t* Y, const int32_t* inv_perm, const float* scores, int64_t T,
                int32_t k, int32_t H, uint16_t* y, moe_stream_t stream);

/* ---- a3/a8: row gather --------------------------------------------------------
 * dst row i = src row (rows[i] / divisor) for i < n; rows are row_bytes bytes
 * (a multiple of 2) and src holds src_rows of them.  divisor = k with rows = a
 * sorted pair order (moe_bucket's perm) is gather_sort's
 * take(x_flat, order // k) (src/common/switch_layers.cpp:21-26); divisor = 1
 * with rows = the inverse order is scatter_unsort's take(x, inv_order, 0)
 * (:32-46).  A row index outside [0, src_rows) leaves a zero row. */
int moe_take_rows(const void* src, int64_t src_rows, const int32_t* rows, int64_t n,
                  int32_t divisor, int64_t row_bytes, void* dst, moe_stream_t stream);

/* ---- SwitchLinear linear bias ------------------------------------------------
 * out[b, m, :] = bf16(out[b, m, :] + bias[rhs[b], :]) for b < batch, m < M, with
 * out [batch, M, N] and bias [num_experts, N] bf16; rows whose rhs[b] >=
 * num_experts are left unchanged.  The take(bias, indices) + add of
 * SwitchLinear::operator(), src/common/switch_layers.cpp:111-114. */
int moe_add_expert_bias(uint16_t* out, const uint16_t* bias, const uint32_t* rhs, int64_t batch,
                        int32_t M, int32_t N, int32_t num_experts, moe_stream_t stream);

/* ---- SwitchGLU ---------------------------------------------------------------
 * out[t, j, :] = down_e(bf16(act(gate_e(x[t]), up_e(x[t])))) with
 * e = inds[t, j], for t < T, j < k, act the moe_activation `activation`
 * (MOE_ACT_SWIGLU: silu(g) * u): x [T, H] bf16, inds [T, k], out
 * [T, k, H] bf16 (the reference's [B, L, k, H] with T = B*L), gate/up
 * [E, I, H] and down [E, H, I] quantized.  No routing weights are applied:
 * the model combines (moe_combine with inv_perm = NULL).  Replaces
 * SwitchGLU::operator() with quantized experts, src/common/switch_layers.cpp:
 * 200-245 (gather_sort, fused gate|up gather_qmm, swiglu, down gather_qmm,
 * scatter_unsort, squeeze). */
size_t moe_switch_glu_workspace_size(const moe_qweight* gate, const moe_qweight* down, int64_t T,
                                     int32_t k);
int moe_switch_glu(const moe_qweight* gate, const moe_qweight* up, const moe_qweight* down,
                   const uint16_t* x, const uint32_t* inds, int64_t T, int32_t k, int32_t activation,
                   uint16_t* out, void* workspace, size_t workspace_bytes, moe_stream_t stream);

/* ---- SwitchMLP with squared ReLU (Nemotron-H experts) --------------------
 * out[t, j, :] = down_e(bf16(relu(up_e(x[t]))^2)), e = inds[t, j]: up [E, I,
 * H], down [E, H, I] quantized, out [T, k, H].  Replaces
 * NemotronHSwitchMLP::operator(), src/llm/models/nemotron_h.cpp:484-511
 * (fc1, relu_squared of include/mlx-lm/common/activations.h:45-55, fc2). */
size_t moe_switch_mlp_workspace_size(const moe_qweight* up, const moe_qweight* down, int64_t T, int32_t k);
int moe_switch_mlp_relu2(const moe_qweight* up, const moe_qweight* down, const uint16_t* x, const uint32_t* inds,
                         int64_t T, int32_t k, uint16_t* out, void* workspace, size_t workspace_bytes,
                         moe_stream_t stream);

/* ---- whole block -----------------------------------------------------------
 * out[T, H] = combine(SwitchGLU(x, route(x))) (+ shared expert), the
 * Qwen3MoESparseMoeBlock / Qwen3NextSparseMoeBlock / PhiMoE / DeepseekV3MoE
 * operator() of src/llm/models/{qwen3_moe.cpp:155-175, qwen3_next.cpp:
 * 452-490, phimoe.cpp:93-105, deepseek_v3.cpp:371-381}. */
size_t moe_block_workspace_size(const moe_block_desc* desc, int64_t T);
int moe_block_forward(const moe_block_desc* desc, const uint16_t* x, int64_t T, uint16_t* out,
                      const moe_block_aux* aux, void* workspace, size_t workspace_bytes,
                      moe_stream_t stream);

/* ---- the step before the block and the block in one call ------------------
 * moe_add_rms_norm(a, b, norm_weight, eps, T, H, sum_out, normed_out)
 * followed by moe_block_forward(desc, normed_out, T, out, aux, ...), with the
 * same results bit for bit (sum_out and normed_out are written too).  For up
 * to 16 tokens with a bf16 router the residual add + RMSNorm runs inside the
 * router projection's launch, one launch fewer per layer; otherwise it is a
 * launch of its own first.  H = desc->hidden, a multiple of 8, at most 8192;
 * a, b, norm_weight, sum_out, normed_out 16-byte aligned, and sum_out and
 * normed_out overlap no input.  The workspace is moe_block_workspace_size's.
 * Replaces the decode layer's add_rms_norm (src/common/gated_delta.cpp:
 * 313-345, called at src/llm/models/qwen35_moe.cpp:787-788) and the MoE
 * block call that consumes its output (:792). */
int moe_block_forward_add_norm(const moe_block_desc* desc, const uint16_t* a, const uint16_t* b,
                               const uint16_t* norm_weight, float eps, int64_t T, uint16_t* sum_out,
                               uint16_t* normed_out, uint16_t* out, const moe_block_aux* aux, void* workspace,
                               size_t workspace_bytes, moe_stream_t stream);

/* ---- whole block without a workspace argument -----------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): moe_block_forward with the workspace taken from a static
 * device array of the library, MOE_NOALLOC_SCRATCH_BYTES (64 MiB) per GPU,
 * held until the process ends.  Calls no hipMalloc / hipFree.  A T whose
 * moe_block_workspace_size exceeds that returns MOE_E_WORKSPACE (text in
 * moe_last_error) before any launch; 64 MiB holds every benchmark
 * configuration at decode sizes (T <= 64) and Qwen3-30B-A3B up to 1024 tokens.
 * The stream must belong to the current device.  The first call on each
 * device looks up the array's device address and must not be under stream
 * capture (it returns MOE_E_INVALID_ARG there); later calls may be captured
 * and replayed.  All calls on one GPU share that GPU's array: calls that
 * overlap on one GPU (several streams, threads, or replays of graphs that
 * captured this call) race on it. */
#define MOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int moe_block_forward_noalloc(const moe_block_desc* desc, const uint16_t* x, int64_t T, uint16_t* out,
                              const moe_block_aux* aux, moe_stream_t stream);

/* ---- decode-loop integration: the block as one captured HIP graph ------
 * Captures moe_block_forward(desc, x, T, out, NULL, workspace, ...) on a
 * stream of the library's own into a graph whose launches read the given
 * buffers, so a decode loop that refills x in place replays the whole layer
 * (router through combine) with one hipGraphLaunch.  The descriptor's
 * weights, x, out and workspace must stay allocated and unchanged in address
 * while the graph lives; T is fixed.  Replays on one stream run in order;
 * replays of one graph on several streams at once race on its workspace.
 * Replaces the per-layer MoE launches of the reference's decode loop
 * (src/common/generate.cpp:362-500, one step per token) for this block. */
typedef struct moe_block_graph_s* moe_block_graph;
int moe_block_graph_create(const moe_block_desc* desc, const uint16_t* x, int64_t T, uint16_t* out,
                           void* workspace, size_t workspace_bytes, moe_block_graph* graph);
int moe_block_graph_launch(moe_block_graph graph, moe_stream_t stream);
int moe_block_graph_destroy(moe_block_graph graph);

/* ---- per-kernel timing ------------------------------------------------------
 * When enabled, every kernel the library launches is bracketed by two HIP
 * events recorded on the launch stream.  moe_profile_record(i) waits for
 * record i and returns its kernel name and duration.  A single-threaded
 * measurement facility (the counterpart of the reference's wall-clock [TPS]
 * timing, src/common/generate.cpp:285-294); disabled by default.
 * moe_profile_enable(1) clears earlier records. */
int moe_profile_enable(int enable);
int moe_profile_count(void);
int moe_profile_record(int index, const char** name, float* milliseconds);

/* ---- host-side data formats (no GPU needed) ------------------------------
 * Seeded counter-based generator: element i of tensor `tensor_id` is
 * mean + std * z_i with z_i a Box-Muller normal from SplitMix64 draws, rounded
 * to bf16 (or kept fp32).  Writes elements [first, first + n) so a tensor can
 * be produced in slices.  Identical on every host.  Not a reference op: it
 * makes the seeded synthetic inputs the reference's benchmark configs name. */
int moe_synth_normal_bf16(uint64_t seed, uint64_t tensor_id, float mean, float std_dev,
                          int64_t first, int64_t n, uint16_t* out);
int moe_synth_normal_f32(uint64_t seed, uint64_t tensor_id, float mean, float std_dev,
                         int64_t first, int64_t n, float* out);
/* MLX affine quantizer (the mx::quantize call of examples/convert.cpp:225):
 * per group of group_size along K, scale/bias from the group's min/max,
 * q = clip(round((w - bias) / scale), 0, 2^bits - 1), packed LSB first
 * (bits 2, 3, 4, 5, 6 or 8; group_size * bits a multiple of 32). */
int moe_quantize_affine(const uint16_t* w, int64_t rows, int32_t K, int32_t group_size,
                        int32_t bits, uint32_t* wq, uint16_t* scales, uint16_t* biases);

#ifdef __cplusplus
}
#endif
#endif /* MOE_MI355X_H */
