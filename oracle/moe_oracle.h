/*
 * moe_oracle.h -- CPU restatement of lemon-mlx-engine's quantized MoE block.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (the HIP library declared in
 * include/moe_mi355x.h) never calls it.
 *
 * The reference's arithmetic lives in an MLX fork (gather_qmm, quantize,
 * argpartition, softmax, ...) that is fetched at configure time and is absent
 * from this machine (reference CMakeLists.txt:33-42), so the reference cannot
 * be built or run here.  This file restates the algorithm the reference's
 * call sites ask of MLX.  Every function names the reference lines it follows.
 *
 * Pin status (how each function is checked, see tests/test_oracle.py):
 *   oracle_dequant        pinned: reference KAT examples/diagnose.cpp:297-311
 *                         (0x76543210, s=1, b=0, gs=8, 4-bit -> 0..7), an 8-bit
 *                         analogue, closed form w = s*q + b against numpy.
 *   oracle_gather_qmm     pinned: examples/test_qbits.cpp:51-58 construction
 *                         (take + dequantize + matmul) in fp64 numpy, one-hot x,
 *                         integer-exact case (s=1, b=0), lhs/rhs broadcast cases.
 *   oracle_router_logits  pinned: fp64 numpy matmul, bf16 rounding bound.
 *   oracle_route          pinned: selection against numpy lexsort brute force on
 *                         the oracle's own selection values; weights against
 *                         fp64 closed forms; group limit against brute-force
 *                         enumeration of groups; R3 == R1+renorm identity.
 *   oracle_bucket         pinned: numpy argsort(kind="stable"), argsort of the
 *                         permutation, bincount + cumsum.
 *   oracle_swiglu / oracle_combine / oracle_moe_experts / oracle_block_forward
 *                         pinned: independent fp64 numpy restatement of the
 *                         whole block on small shapes; linearity in scores.
 *   Unpinned (MLX internals that only an MLX import could fix; absent here):
 *   MLX's gather_qmm summation order and accumulator type, argpartition tie
 *   order, bf16 softmax rounding, mx::compile intermediate rounding.  The
 *   canonical choices below are this build's definitions and are documented
 *   per function.
 *
 * Storage conventions: bf16 values are uint16_t bit patterns.  Quantized
 * weights use MLX's affine layout: w[E][N][K*bits/32] uint32, element c of a
 * row is bits [c*bits, c*bits + bits) of the row's little-endian bit stream,
 * LSB first (4 and 8 bits: word c/(32/bits) at bit (c%(32/bits))*bits; 6 bits:
 * four codes per three bytes; the 6-bit byte layout is parity unpinned, MLX being
 * absent: it follows MLX's published packing of 3-byte groups); scales and
 * biases are bf16 [E][N][K/group_size] (reference
 * include/mlx-lm/common/quantized_linear.h:16-21, debug_numerical_trace.py:67-98).
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Router variants (canonical names for the reference's per-model routers). */
enum {
  ORACLE_ROUTE_TOPK_LOGITS = 1,   /* R1 qwen3_moe.cpp:156-168            */
  ORACLE_ROUTE_TOPK_PROBS = 2,    /* R2 qwen3_next.cpp:453-469           */
  ORACLE_ROUTE_SOFTMAX_TOPK = 3,  /* R3/R4 phimoe.cpp:96-101, gated_delta.cpp:385-422 */
  ORACLE_ROUTE_SIGMOID = 5,       /* R5 deepseek_v3.cpp:304-350          */
  ORACLE_ROUTE_SIGMOID_GROUP = 6, /* R6 nemotron_h.cpp:405-468 (upstream noaux_tc: keep the best groups) */
  ORACLE_ROUTE_SIGMOID_GROUP_DROP_BEST = 7, /* R6 as written, nemotron_h.cpp:425-447: drop the best groups */
  ORACLE_ROUTE_SIGMOID_CORRECTED = 8, /* bailing_moe.cpp:173-199: weights from the corrected scores */
  ORACLE_ROUTE_GLM4_SIGMOID = 9,      /* glm4_moe.cpp:158-191, scoring_func "sigmoid" */
  ORACLE_ROUTE_GLM4_SOFTMAX = 10,     /* glm4_moe.cpp:158-191, scoring_func "softmax" */
  ORACLE_ROUTE_LFM2 = 11              /* lfm2_moe.cpp:219-238 */
};

typedef struct oracle_router_params {
  int32_t variant;
  int32_t num_experts;
  int32_t top_k;
  int32_t norm_topk_prob;
  int32_t n_group;
  int32_t topk_group;
  float routed_scaling_factor;
} oracle_router_params;

typedef struct oracle_qweight {
  const uint32_t* w;
  const uint16_t* scales;
  const uint16_t* biases; /* may be NULL: treated as 0 */
  int32_t experts, N, K, group_size, bits;
  /* SwitchLinear's bias [experts, N] bf16 or NULL: out = bf16(bf16(x.W^T) +
   * bias[e]) (src/common/switch_layers.cpp:111-114) */
  const uint16_t* linear_bias;
} oracle_qweight;

typedef struct oracle_block {
  int32_t hidden, intermediate, num_experts;
  oracle_router_params router;
  const uint16_t* router_weight; /* [E, H] bf16 */
  const float* score_bias;       /* [E] fp32 or NULL */
  oracle_qweight gate, up, down; /* [E, I, H], [E, I, H], [E, H, I] */
  int32_t shared_intermediate;   /* 0: no shared expert */
  oracle_qweight shared_gate, shared_up, shared_down; /* experts == 1 */
  const uint16_t* shared_gate_weight; /* [1, H] bf16, NULL: ungated */
  oracle_qweight router_q; /* w != NULL: quantized router [1][E, H], used instead of router_weight */
  const uint16_t* router_bias; /* [E] bf16 or NULL: the dense router's bias (addmm, one rounding) */
  oracle_qweight shared_gate_q; /* w != NULL: quantized shared-expert gate [1][1, H] */
  /* GLU activation of the routed experts (ORACLE_ACT_*; the shared expert is
   * always SwiGLU). */
  int32_t activation;
  /* 1: the routed experts' h stays fp32 (no bf16 rounding), the down
   * projection multiplies fp32 activations and its output Y (plus the linear
   * bias) stays fp32 into the combine.  This is what the reference's GPT-OSS
   * MLP computes: its swiglu mixes bf16 arrays with fp32 scalar arrays
   * (mx::array(7.0f), gptoss.cpp:50-58), which MLX's type promotion makes
   * fp32, and gather_qmm returns the dtype of its fp32 input (parity of the
   * promotion itself unpinned: MLX is absent).  0: h and Y are bf16. */
  int32_t hidden_f32;
} oracle_block;

/* GLU activations (the product's moe_activation values). */
enum {
  ORACLE_ACT_SWIGLU = 0,          /* silu(g) * u, activations.h:22-30 */
  ORACLE_ACT_GPTOSS = 1,          /* gptoss.cpp:50-58 swiglu(x_linear = g, x_glu = u), as called at :158 */
  ORACLE_ACT_GPTOSS_UPSTREAM = 2  /* the same function with x_linear = u, x_glu = g */
};

int oracle_num_threads(void);
void oracle_set_num_threads(int n);

/* canonical exp / sigmoid shared by the router definition */
float oracle_canon_expf(float x);

void oracle_dequant(const uint32_t* w, const uint16_t* scales,
                    const uint16_t* biases, int64_t rows, int32_t K,
                    int32_t group_size, int32_t bits, float* out);

/* logits[T,E] = bf16(x[T,H] . Wg[E,H]^T + bias[E]), fp32 accumulation, one
 * rounding (bias NULL: none). */
int oracle_router_logits(const uint16_t* x, const uint16_t* wg, const uint16_t* bias, int64_t T,
                         int32_t H, int32_t E, uint16_t* logits);

/* Per-token scoring, top-k selection, renormalisation and scaling.
 * inds[T,k] in canonical slot order (selection value desc, expert asc);
 * scores[T,k] fp32 (bf16-exact for the bf16 variants).  sel_out[T,E]
 * (optional) receives the values the selection compares. */
int oracle_route(const uint16_t* logits, const float* score_bias, int64_t T,
                 const oracle_router_params* p, uint32_t* inds, float* scores,
                 float* sel_out);

/* Stable bucketing of the T*k (token, expert) pairs by expert id. */
int oracle_bucket(const uint32_t* inds, int64_t T, int32_t k, int32_t E,
                  int32_t* perm, int32_t* inv_perm, uint32_t* sorted_expert,
                  int32_t* offsets);

/* out[b,m,:] = x[lhs[b],m,:] . dequant(w[rhs[b]])^T, bf16 out. lhs NULL =
 * identity. */
int oracle_gather_qmm(const uint16_t* x, const oracle_qweight* w,
                      const uint32_t* lhs, const uint32_t* rhs, int64_t batch,
                      int32_t M, uint16_t* out);

/* out[b,m,:] = x[lhs[b],m,:] . w[rhs[b]]^T (+ linear_bias[rhs[b]]) with dense
 * bf16 weights w [E, N, K]: gather_mm as SwitchLinear's non-quantized branch
 * calls it (switch_layers.cpp:103-115).  fp32 accumulation in increasing k,
 * bf16 output, the bias added to the rounded product and rounded again. */
int oracle_gather_mm(const uint16_t* x, const uint16_t* w, const uint16_t* linear_bias, int32_t E, int32_t N,
                     int32_t K, const uint32_t* lhs, const uint32_t* rhs, int64_t batch, int32_t M,
                     uint16_t* out);

/* h = bf16(silu(g) * u) elementwise. */
/* add_rms_norm, reference src/common/gated_delta.cpp:313-345: s = a + b in
 * fp32, sum_out = bf16(s); the squares of the unrounded s summed as the
 * reference does (32 lane-strided partial sums, then an xor tree over the
 * lanes); normed = bf16(fp32(sum_out) * scale * w) with scale =
 * 1/sqrt(ss/H + eps) correctly rounded (the reference's rsqrtf may differ by
 * an ulp). */
void oracle_add_rms_norm(const uint16_t* a, const uint16_t* b, const uint16_t* w, float eps, int64_t T,
                         int32_t H, uint16_t* sum_out, uint16_t* normed);
void oracle_swiglu(const uint16_t* g, const uint16_t* u, int64_t n,
                   uint16_t* h);

/* GPT-OSS's clipped SwiGLU (gptoss.cpp:50-58, alpha 1.702, limit 7):
 * xl = clip(x_linear, -7, 7), xg = min(x_glu, 7), v = (xg * sigmoid(1.702 *
 * xg)) * (xl + 1) in fp32.  h (bf16, may be NULL) = bf16(v); h_f32 (may be
 * NULL) = v, the reference's own fp32 output. */
void oracle_gptoss_swiglu(const uint16_t* x_linear, const uint16_t* x_glu, int64_t n, uint16_t* h,
                          float* h_f32);

/* gather_qmm with fp32 activations (x [*, M, K] fp32) and fp32 output: MLX's
 * gather_qmm on an fp32 input, as the reference's relu_squared and GPT-OSS
 * paths feed their promoted fp32 hidden values to the down projection.
 * linear_bias (if any) is added in fp32. */
int oracle_gather_qmm_f32x(const float* x, const oracle_qweight* w, const uint32_t* lhs, const uint32_t* rhs,
                           int64_t batch, int32_t M, float* out);

/* y[t] = bf16(sum_j scores[t,j] * Y[t,j,:]) */
void oracle_combine(const uint16_t* Y, const float* scores, int64_t T,
                    int32_t k, int32_t H, uint16_t* y);

/* Routed experts + combine + shared expert for given routing.  term_mag
 * [T, H] (optional) receives sum_j |scores[t,j] * Y[t,j,c]| + |gate * Ys[t,c]|,
 * the magnitude of the bf16-rounded terms the output sums (for error models). */
int oracle_moe_experts(const oracle_block* b, const uint16_t* x, int64_t T,
                       const uint32_t* inds, const float* scores,
                       uint16_t* out, float* term_mag);

/* Whole block: logits -> route -> experts -> combine (+ shared). Optional
 * outputs may be NULL. */
int oracle_block_forward(const oracle_block* b, const uint16_t* x, int64_t T,
                         uint16_t* out, uint16_t* logits_out,
                         uint32_t* inds_out, float* scores_out);

#ifdef __cplusplus
}
#endif
#endif
