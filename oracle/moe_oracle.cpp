// moe_oracle.cpp -- CPU restatement of lemon-mlx-engine's quantized MoE block.
//
// TEST INFRASTRUCTURE ONLY: this is the checker for the HIP library and the
// timed CPU baseline.  Nothing in the product links or calls it.  See
// moe_oracle.h for the pin status of every function.
//
// Compiled with -ffp-contract=off so that every fp32 expression rounds exactly
// where it is written; the canonical router arithmetic (canon_expf, the
// 64-way strided softmax denominator) is defined by the order written here.

#include "moe_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

inline float bf2f(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// float -> bf16, round to nearest even (NaN kept quiet).
inline uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

inline float bfr(float f) { return bf2f(f2bf(f)); }

// Canonical exp used by every router score (softmax, sigmoid).  Cody-Waite
// reduction x = n*ln2 + r with a two-part ln2 (ln2_hi has 15 significant
// bits), then exp(r) on |r| <= ln2/2 by the degree-7 Taylor polynomial in
// Horner form with fused multiply-adds, then scaling by 2^n.  Inputs below -87
// return 0 (no subnormal results), above 88.72 return +inf.  The HIP router
// evaluates the identical sequence, so router scores are reproducible
// bit-for-bit on both sides; accuracy is within 2 ulp of libm expf (tested).
float canon_expf_impl(float x) {
  if (x != x) return x;
  if (x > 88.72f) return INFINITY;
  if (x < -87.0f) return 0.0f;
  const float n = std::rint(x * 1.44269504f);
  float r = std::fma(n, -0.693145751953125f, x);
  r = std::fma(n, -1.42860677e-6f, r);
  float p = 1.98412698e-4f;           // 1/7!
  p = std::fma(p, r, 1.38888889e-3f); // 1/6!
  p = std::fma(p, r, 8.33333333e-3f); // 1/5!
  p = std::fma(p, r, 4.16666667e-2f); // 1/4!
  p = std::fma(p, r, 1.66666667e-1f); // 1/3!
  p = std::fma(p, r, 0.5f);
  p = std::fma(p, r, 1.0f);
  p = std::fma(p, r, 1.0f);
  return std::ldexp(p, static_cast<int>(n));
}

inline float canon_sigmoid(float v) { return 1.0f / (1.0f + canon_expf_impl(-v)); }

// Plain fp32 SiLU for the expert MLP (tolerance-checked, not canonical).
inline float silu_f32(float g) { return g * (1.0f / (1.0f + std::exp(-g))); }

// GPT-OSS's file-local swiglu, src/llm/models/gptoss.cpp:50-58, with its
// defaults alpha = 1.702, limit = 7, step by step: xlin = clip(x_linear, -7,
// 7); xg = clip(x_glu, max 7); glu_scaled = alpha * xg; sig =
// sigmoid(glu_scaled); out_glu = xg * sig; out = out_glu * (xlin + 1).
// Every step is fp32 (the fp32 scalar arrays promote the bf16 inputs).
inline float gptoss_glu_f32(float x_linear, float x_glu) {
  const float xlin = std::min(std::max(x_linear, -7.0f), 7.0f);
  const float xg = std::min(x_glu, 7.0f);
  const float glu_scaled = 1.702f * xg;
  const float sig = 1.0f / (1.0f + std::exp(-glu_scaled));
  const float out_glu = xg * sig;
  return out_glu * (xlin + 1.0f);
}

// The expert MLP's activation of the gate value g and up value u.
inline float glu_act_f32(int32_t act, float g, float u) {
  if (act == ORACLE_ACT_GPTOSS) return gptoss_glu_f32(g, u);  // swiglu(x_gate, x_up), gptoss.cpp:158
  if (act == ORACLE_ACT_GPTOSS_UPSTREAM) return gptoss_glu_f32(u, g);
  return silu_f32(g) * u;
}

// Code c of a row is bits [c*bits, c*bits + bits) of the row's little-endian
// bit stream (MLX's affine packing, least significant first: at 4 and 8 bits a
// code never crosses a 32-bit word; at 6 bits four codes fill three bytes).
inline uint32_t code_at(const uint32_t* row, int32_t c, int32_t bits) {
  const int64_t bit = static_cast<int64_t>(c) * bits;
  const int64_t wi = bit >> 5;
  const int32_t sh = static_cast<int32_t>(bit & 31);
  uint64_t v = row[wi];
  if (sh + bits > 32) v |= static_cast<uint64_t>(row[wi + 1]) << 32;
  return static_cast<uint32_t>(v >> sh) & ((1u << bits) - 1u);
}

inline float dequant_one(const uint32_t* row, const uint16_t* s, const uint16_t* b,
                         int32_t c, int32_t gs, int32_t bits) {
  const uint32_t q = code_at(row, c, bits);
  const int32_t g = c / gs;
  const float sc = bf2f(s[g]);
  const float bi = b ? bf2f(b[g]) : 0.0f;
  return sc * static_cast<float>(q) + bi;  // s*q is exact in fp32, one rounding
}

// Dequantize rows [r0, r0+nr) of a [rows, K] quantized matrix into fp32.
void dequant_rows(const oracle_qweight& w, int64_t expert, int64_t r0, int64_t nr, float* out) {
  const int64_t wpr = static_cast<int64_t>(w.K) * w.bits / 32;
  const int64_t gpr = w.K / w.group_size;
  for (int64_t r = 0; r < nr; ++r) {
    const int64_t row = expert * w.N + r0 + r;
    const uint32_t* wr = w.w + row * wpr;
    const uint16_t* sr = w.scales + row * gpr;
    const uint16_t* br = w.biases ? w.biases + row * gpr : nullptr;
    for (int32_t c = 0; c < w.K; ++c) out[r * w.K + c] = dequant_one(wr, sr, br, c, w.group_size, w.bits);
  }
}

// One output of a SwitchLinear: bf16 of the dot product, then (with a linear
// bias) bf16 of that plus the bias (switch_layers.cpp:111-114).
inline float lin_out(float dot, const oracle_qweight& w, int64_t e, int32_t n) {
  const float v = bfr(dot);
  return w.linear_bias ? bfr(v + bf2f(w.linear_bias[e * w.N + n])) : v;
}

inline float dot_f32(const float* a, const float* b, int32_t n) {
  float acc = 0.0f;
  for (int32_t i = 0; i < n; ++i) acc += a[i] * b[i];
  return acc;
}

bool qweight_ok(const oracle_qweight& w) {
  if (!w.w || !w.scales) return false;
  if (w.bits < 2 || w.bits > 8 || w.bits == 7) return false;
  if (w.group_size <= 0 || w.K % w.group_size != 0) return false;
  if ((static_cast<int64_t>(w.K) * w.bits) % 32 != 0) return false;
  return w.experts > 0 && w.N > 0 && w.K > 0;
}

// Top-k by (value desc, index asc): the canonical slot order (the tie rule of
// the reference's moe_route kernel, src/common/gated_delta.cpp:398-406).
void topk_canonical(const float* sel, int32_t E, int32_t k, uint32_t* out) {
  std::vector<int32_t> idx(E);
  std::iota(idx.begin(), idx.end(), 0);
  std::partial_sort(idx.begin(), idx.begin() + k, idx.end(), [&](int32_t a, int32_t b) {
    if (sel[a] > sel[b]) return true;
    if (sel[a] < sel[b]) return false;
    return a < b;
  });
  for (int32_t j = 0; j < k; ++j) out[j] = static_cast<uint32_t>(idx[j]);
}

// Canonical softmax over one row of bf16 logits -> bf16 probabilities (fp32
// ones with round_bf16 = false).
// Denominator: 64 strided fp32 partial sums (expert e goes to partial e%64,
// added in increasing e), then an xor-butterfly over the 64 partials with
// offsets 32,16,8,4,2,1.  This is the order a wave64 computes it in.
void softmax_canonical(const float* l, int32_t E, float* probs, bool round_bf16 = true) {
  float m = l[0];
  for (int32_t e = 1; e < E; ++e) m = std::max(m, l[e]);
  std::vector<float> ex(E);
  float parts[64];
  for (float& v : parts) v = 0.0f;
  for (int32_t e = 0; e < E; ++e) {
    ex[e] = canon_expf_impl(l[e] - m);
    parts[e & 63] += ex[e];
  }
  for (int32_t off = 32; off >= 1; off >>= 1) {
    float nxt[64];
    for (int32_t i = 0; i < 64; ++i) nxt[i] = parts[i] + parts[i ^ off];
    std::memcpy(parts, nxt, sizeof(parts));
  }
  const float sum = parts[0];
  for (int32_t e = 0; e < E; ++e) probs[e] = round_bf16 ? bfr(ex[e] / sum) : ex[e] / sum;
}

bool router_params_ok(const oracle_router_params* p) {
  if (!p) return false;
  const int32_t E = p->num_experts, k = p->top_k;
  if (E <= 0 || k <= 0 || k > E) return false;
  switch (p->variant) {
    case ORACLE_ROUTE_TOPK_LOGITS:
    case ORACLE_ROUTE_TOPK_PROBS:
    case ORACLE_ROUTE_SOFTMAX_TOPK:
    case ORACLE_ROUTE_SIGMOID:
      return true;
    case ORACLE_ROUTE_SIGMOID_CORRECTED:
    case ORACLE_ROUTE_GLM4_SIGMOID:
    case ORACLE_ROUTE_GLM4_SOFTMAX:
      return true;  // group index computed but unused (bailing_moe.cpp:173-185, glm4_moe.cpp:168-188)
    case ORACLE_ROUTE_LFM2:
      return true;
    case ORACLE_ROUTE_SIGMOID_GROUP:
    case ORACLE_ROUTE_SIGMOID_GROUP_DROP_BEST:
      if (p->n_group <= 1) return true;
      if (E % p->n_group != 0 || E / p->n_group < 2) return false;
      if (p->topk_group < 1 || p->topk_group > p->n_group) return false;
      return true;
    default:
      return false;
  }
}

// One token of the router.  Semantics per variant:
//  R1 qwen3_moe.cpp:156-168: select top-k of the bf16 logits; weights are the
//     bf16 softmax over all E gathered at the selection; renorm divides by the
//     bf16 sum of the k weights.
//  R2 qwen3_next.cpp:453-469: select top-k of the bf16 softmax probabilities;
//     weights and renorm as R1.
//  R3 phimoe.cpp:96-101 / R4 gated_delta.cpp:385-422 (moe_route): select top-k
//     of the logits, weights = softmax over the k selected logits.
//  R5 deepseek_v3.cpp:304-350 as written: bf16 sigmoid of the logits, select on
//     it (the correction bias and group scores are computed but unused there);
//     if k>1 && norm: w / (bf16 sum + 1e-20) * scaling in fp32.
//  R6 nemotron_h.cpp:405-468 (DeepSeek noaux_tc): o = fp32 sigmoid, select on
//     o + bias with group limit (group score = sum of the two largest corrected
//     scores; the topk_group best groups are kept, the others multiplied by 0);
//     weights o gathered; if k>1 && norm: w / (sum + 1e-20); always * scaling.
//  R6 as written (nemotron_h.cpp:425-447): argpartition of the NEGATED group
//     scores picks the n_group - topk_group groups to zero, i.e. the best
//     ones (by group score desc, group index asc); otherwise as R6.
//  Bailing (bailing_moe.cpp:173-199): select on o + bias with no group limit
//     (its group index is computed but never applied); the weights are the
//     corrected scores o + bias gathered, renormalised (+1e-20) if k>1 &&
//     norm, times scaling, cast to the logits' dtype (bf16).
//  GLM4-MoE (glm4_moe.cpp:158-191): o = fp32 sigmoid or fp32 softmax of the
//     logits (scoring_func), select on o + bias (the group index is computed
//     but never applied, :168-188); weights o gathered; if k>1 && norm:
//     w / sum (no epsilon); always * scaling; fp32.
//  LFM2-MoE (lfm2_moe.cpp:219-238): g = fp32 softmax of the logits plus the
//     expert bias (when present); select on g; the weights are g gathered
//     (the biased values), divided by (sum + 1e-20) when norm (any k), cast
//     to bf16; no scaling.
void route_token(const uint16_t* lrow, const float* bias, const oracle_router_params& p,
                 uint32_t* inds, float* scores, float* sel_out) {
  const int32_t E = p.num_experts, k = p.top_k;
  std::vector<float> l(E), sel(E), base(E);
  for (int32_t e = 0; e < E; ++e) l[e] = bf2f(lrow[e]);

  switch (p.variant) {
    case ORACLE_ROUTE_TOPK_LOGITS:
      softmax_canonical(l.data(), E, base.data());
      sel = l;
      break;
    case ORACLE_ROUTE_TOPK_PROBS:
      softmax_canonical(l.data(), E, base.data());
      sel = base;
      break;
    case ORACLE_ROUTE_SOFTMAX_TOPK:
      sel = l;
      break;
    case ORACLE_ROUTE_SIGMOID:
      for (int32_t e = 0; e < E; ++e) base[e] = bfr(canon_sigmoid(l[e]));
      sel = base;
      break;
    case ORACLE_ROUTE_GLM4_SOFTMAX:
    case ORACLE_ROUTE_LFM2:
      softmax_canonical(l.data(), E, base.data(), false);
      for (int32_t e = 0; e < E; ++e) sel[e] = base[e] + (bias ? bias[e] : 0.0f);
      break;
    case ORACLE_ROUTE_SIGMOID_GROUP:
    case ORACLE_ROUTE_SIGMOID_GROUP_DROP_BEST:
    case ORACLE_ROUTE_SIGMOID_CORRECTED:
    case ORACLE_ROUTE_GLM4_SIGMOID: {
      for (int32_t e = 0; e < E; ++e) {
        base[e] = canon_sigmoid(l[e]);
        sel[e] = base[e] + (bias ? bias[e] : 0.0f);
      }
      if (p.n_group > 1 && (p.variant == ORACLE_ROUTE_SIGMOID_GROUP ||
                            p.variant == ORACLE_ROUTE_SIGMOID_GROUP_DROP_BEST)) {
        const int32_t G = p.n_group, gsz = E / G;
        std::vector<float> gscore(G);
        for (int32_t g = 0; g < G; ++g) {
          float v1 = -INFINITY, v2 = -INFINITY;  // largest, second largest
          for (int32_t i = 0; i < gsz; ++i) {
            const float v = sel[g * gsz + i];
            if (v > v1) {
              v2 = v1;
              v1 = v;
            } else if (v > v2) {
              v2 = v;
            }
          }
          gscore[g] = v2 + v1;
        }
        std::vector<uint32_t> gorder(G);
        topk_canonical(gscore.data(), G, G, gorder.data());
        // zero groups of rank r0 <= r < r1 in the canonical group order
        const bool drop_best = p.variant == ORACLE_ROUTE_SIGMOID_GROUP_DROP_BEST;
        const int32_t r0 = drop_best ? 0 : p.topk_group, r1 = drop_best ? G - p.topk_group : G;
        for (int32_t r = r0; r < r1; ++r) {
          const int32_t g = static_cast<int32_t>(gorder[r]);
          for (int32_t i = 0; i < gsz; ++i) sel[g * gsz + i] = sel[g * gsz + i] * 0.0f;
        }
      }
      break;
    }
    default:
      return;
  }

  topk_canonical(sel.data(), E, k, inds);
  if (sel_out) std::memcpy(sel_out, sel.data(), sizeof(float) * E);

  switch (p.variant) {
    case ORACLE_ROUTE_TOPK_LOGITS:
    case ORACLE_ROUTE_TOPK_PROBS: {
      for (int32_t j = 0; j < k; ++j) scores[j] = base[inds[j]];
      if (p.norm_topk_prob) {
        float s = 0.0f;
        for (int32_t j = 0; j < k; ++j) s += scores[j];
        s = bfr(s);
        for (int32_t j = 0; j < k; ++j) scores[j] = bfr(scores[j] / s);
      }
      break;
    }
    case ORACLE_ROUTE_SOFTMAX_TOPK: {
      const float m = l[inds[0]];
      float s = 0.0f;
      for (int32_t j = 0; j < k; ++j) {
        scores[j] = canon_expf_impl(l[inds[j]] - m);
        s += scores[j];
      }
      for (int32_t j = 0; j < k; ++j) scores[j] = bfr(scores[j] / s);
      break;
    }
    case ORACLE_ROUTE_SIGMOID: {
      for (int32_t j = 0; j < k; ++j) scores[j] = base[inds[j]];
      if (k > 1 && p.norm_topk_prob) {
        float s = 0.0f;
        for (int32_t j = 0; j < k; ++j) s += scores[j];
        const float denom = bfr(s) + 1e-20f;
        for (int32_t j = 0; j < k; ++j) scores[j] = (scores[j] / denom) * p.routed_scaling_factor;
      }
      break;
    }
    case ORACLE_ROUTE_SIGMOID_GROUP:
    case ORACLE_ROUTE_SIGMOID_GROUP_DROP_BEST:
    case ORACLE_ROUTE_SIGMOID_CORRECTED: {
      const bool corrected = p.variant == ORACLE_ROUTE_SIGMOID_CORRECTED;
      for (int32_t j = 0; j < k; ++j) scores[j] = corrected ? sel[inds[j]] : base[inds[j]];
      if (k > 1 && p.norm_topk_prob) {
        float s = 0.0f;
        for (int32_t j = 0; j < k; ++j) s += scores[j];
        const float denom = s + 1e-20f;
        for (int32_t j = 0; j < k; ++j) scores[j] = scores[j] / denom;
      }
      for (int32_t j = 0; j < k; ++j) scores[j] = scores[j] * p.routed_scaling_factor;
      if (corrected)
        for (int32_t j = 0; j < k; ++j) scores[j] = bfr(scores[j]);
      break;
    }
    case ORACLE_ROUTE_LFM2: {
      for (int32_t j = 0; j < k; ++j) scores[j] = sel[inds[j]];
      if (p.norm_topk_prob) {
        float s = 0.0f;
        for (int32_t j = 0; j < k; ++j) s += scores[j];
        const float denom = s + 1e-20f;
        for (int32_t j = 0; j < k; ++j) scores[j] = scores[j] / denom;
      }
      for (int32_t j = 0; j < k; ++j) scores[j] = bfr(scores[j]);
      break;
    }
    case ORACLE_ROUTE_GLM4_SIGMOID:
    case ORACLE_ROUTE_GLM4_SOFTMAX: {
      for (int32_t j = 0; j < k; ++j) scores[j] = base[inds[j]];
      if (k > 1 && p.norm_topk_prob) {
        float s = 0.0f;
        for (int32_t j = 0; j < k; ++j) s += scores[j];
        for (int32_t j = 0; j < k; ++j) scores[j] = scores[j] / s;
      }
      for (int32_t j = 0; j < k; ++j) scores[j] = scores[j] * p.routed_scaling_factor;
      break;
    }
    default:
      break;
  }
}

}  // namespace

extern "C" {

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

float oracle_canon_expf(float x) { return canon_expf_impl(x); }

// Dequantize (reference: examples/diagnose.cpp:297-311 KAT, and the numpy
// restatement debug_numerical_trace.py:67-98): w = s*q + b per group.
void oracle_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    int64_t rows, int32_t K, int32_t group_size, int32_t bits, float* out) {
  oracle_qweight q{w, scales, biases, 1, static_cast<int32_t>(rows), K, group_size, bits, nullptr};
  dequant_rows(q, 0, 0, rows, out);
}

// Router projection, reference quantized_linear.h:73-96 (dense branch
// mx::matmul(x, transpose(w)), or mx::addmm(bias, x, transpose(w)) with a
// bias: one fp32 result, one rounding) called at qwen3_moe.cpp:156,
// gptoss.cpp:130 and friends.
int oracle_router_logits(const uint16_t* x, const uint16_t* wg, const uint16_t* bias, int64_t T, int32_t H,
                         int32_t E, uint16_t* logits) {
  if (!x || !wg || !logits || T < 0 || H <= 0 || E <= 0) return -1;
  std::vector<float> wf(static_cast<size_t>(E) * H);
  for (size_t i = 0; i < wf.size(); ++i) wf[i] = bf2f(wg[i]);
#pragma omp parallel
  {
    std::vector<float> xf(H);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
      for (int32_t h = 0; h < H; ++h) xf[h] = bf2f(x[t * H + h]);
      for (int32_t e = 0; e < E; ++e) {
        const float v = dot_f32(xf.data(), &wf[static_cast<size_t>(e) * H], H);
        logits[t * E + e] = f2bf(bias ? v + bf2f(bias[e]) : v);
      }
    }
  }
  return 0;
}

int oracle_route(const uint16_t* logits, const float* score_bias, int64_t T,
                 const oracle_router_params* p, uint32_t* inds, float* scores, float* sel_out) {
  if (!logits || !inds || !scores || T < 0 || !router_params_ok(p)) return -1;
  const int32_t E = p->num_experts, k = p->top_k;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t)
    route_token(logits + t * E, score_bias, *p, inds + t * k, scores + t * k,
                sel_out ? sel_out + t * E : nullptr);
  return 0;
}

// gather_sort, reference src/common/switch_layers.cpp:17-30: order =
// argsort(flat indices) (canonically stable), inverse = argsort(order); plus
// the per-expert offsets (exclusive scan of the expert histogram) that the
// grouped kernels consume.
int oracle_bucket(const uint32_t* inds, int64_t T, int32_t k, int32_t E, int32_t* perm,
                  int32_t* inv_perm, uint32_t* sorted_expert, int32_t* offsets) {
  if (!inds || T < 0 || k <= 0 || E <= 0) return -1;
  const int64_t P = T * k;
  std::vector<int64_t> cnt(E + 1, 0);
  for (int64_t i = 0; i < P; ++i) {
    if (inds[i] >= static_cast<uint32_t>(E)) return -6;
    cnt[inds[i] + 1]++;
  }
  for (int32_t e = 0; e < E; ++e) cnt[e + 1] += cnt[e];
  if (offsets)
    for (int32_t e = 0; e <= E; ++e) offsets[e] = static_cast<int32_t>(cnt[e]);
  std::vector<int64_t> cursor(cnt.begin(), cnt.end() - 1);
  for (int64_t i = 0; i < P; ++i) {
    const int64_t pos = cursor[inds[i]]++;
    if (perm) perm[pos] = static_cast<int32_t>(i);
    if (inv_perm) inv_perm[i] = static_cast<int32_t>(pos);
    if (sorted_expert) sorted_expert[pos] = inds[i];
  }
  return 0;
}

// gather_qmm as called at switch_layers.cpp:94-102 (transpose=true, affine):
// out[b, m, n] = sum_c x[lhs[b], m, c] * (s*q + b)[rhs[b], n, c], fp32
// accumulation in increasing c, bf16 output.  Test construction mirrored from
// examples/test_qbits.cpp:51-58.  With w->linear_bias, SwitchLinear's bias
// add follows (switch_layers.cpp:111-114): bf16(out + bias[rhs[b], n]).
int oracle_gather_qmm(const uint16_t* x, const oracle_qweight* w, const uint32_t* lhs,
                      const uint32_t* rhs, int64_t batch, int32_t M, uint16_t* out) {
  if (!x || !w || !rhs || !out || batch < 0 || M <= 0 || !qweight_ok(*w)) return -1;
  const int32_t N = w->N, K = w->K;
  for (int64_t b = 0; b < batch; ++b)
    if (rhs[b] >= static_cast<uint32_t>(w->experts)) return -6;
  // bucket the batch by expert so each expert's rows are dequantized once
  std::vector<std::vector<int64_t>> by_e(w->experts);
  for (int64_t b = 0; b < batch; ++b) by_e[rhs[b]].push_back(b);
  for (int32_t e = 0; e < w->experts; ++e) {
    if (by_e[e].empty()) continue;
    std::vector<float> wd(static_cast<size_t>(N) * K);
#pragma omp parallel for schedule(static)
    for (int32_t n = 0; n < N; ++n) dequant_rows(*w, e, n, 1, &wd[static_cast<size_t>(n) * K]);
    const int64_t nb = static_cast<int64_t>(by_e[e].size());
#pragma omp parallel
    {
      std::vector<float> xf(K);
#pragma omp for schedule(static)
      for (int64_t ib = 0; ib < nb * M; ++ib) {
        const int64_t b = by_e[e][ib / M];
        const int32_t m = static_cast<int32_t>(ib % M);
        const int64_t xi = lhs ? static_cast<int64_t>(lhs[b]) : b;
        const uint16_t* xr = x + (xi * M + m) * K;
        for (int32_t c = 0; c < K; ++c) xf[c] = bf2f(xr[c]);
        uint16_t* o = out + (b * M + m) * N;
        for (int32_t n = 0; n < N; ++n) {
          o[n] = f2bf(dot_f32(xf.data(), &wd[static_cast<size_t>(n) * K], K));
          if (w->linear_bias) o[n] = f2bf(bf2f(o[n]) + bf2f(w->linear_bias[static_cast<int64_t>(e) * N + n]));
        }
      }
    }
  }
  return 0;
}

// gather_mm as SwitchLinear's dense branch calls it, switch_layers.cpp:103-115:
// mx::gather_mm(x, swapaxes(weight, -1, -2), lhs, rhs) -- out[b, m, n] =
// sum_k x[lhs[b], m, k] * w[rhs[b], n, k] in fp32, increasing k, bf16 out --
// then take(bias, indices) + add.
int oracle_gather_mm(const uint16_t* x, const uint16_t* w, const uint16_t* linear_bias, int32_t E, int32_t N,
                     int32_t K, const uint32_t* lhs, const uint32_t* rhs, int64_t batch, int32_t M,
                     uint16_t* out) {
  if (!x || !w || !rhs || !out || batch < 0 || M <= 0 || E <= 0 || N <= 0 || K <= 0) return -1;
  for (int64_t b = 0; b < batch; ++b)
    if (rhs[b] >= static_cast<uint32_t>(E)) return -6;
#pragma omp parallel
  {
    std::vector<float> xf(K), wf(K);
#pragma omp for schedule(static)
    for (int64_t ib = 0; ib < batch * M; ++ib) {
      const int64_t b = ib / M;
      const int32_t m = static_cast<int32_t>(ib % M);
      const int64_t xi = lhs ? static_cast<int64_t>(lhs[b]) : b;
      const uint16_t* xr = x + (xi * M + m) * K;
      for (int32_t c = 0; c < K; ++c) xf[c] = bf2f(xr[c]);
      const int64_t e = rhs[b];
      for (int32_t n = 0; n < N; ++n) {
        const uint16_t* wr = w + (e * N + n) * K;
        for (int32_t c = 0; c < K; ++c) wf[c] = bf2f(wr[c]);
        uint16_t v = f2bf(dot_f32(xf.data(), wf.data(), K));
        if (linear_bias) v = f2bf(bf2f(v) + bf2f(linear_bias[e * N + n]));
        out[ib * N + n] = v;
      }
    }
  }
  return 0;
}

// add_rms_norm as written at src/common/gated_delta.cpp:313-345 (lane-strided
// partial sums of 32 lanes, xor-shuffle tree, then the normalised row from the
// rounded sums).
void oracle_add_rms_norm(const uint16_t* a, const uint16_t* b, const uint16_t* w, float eps, int64_t T,
                         int32_t H, uint16_t* sum_out, uint16_t* normed) {
  for (int64_t r = 0; r < T; ++r) {
    const uint16_t* ar = a + r * H;
    const uint16_t* br = b + r * H;
    uint16_t* sr = sum_out + r * H;
    uint16_t* nr = normed + r * H;
    float part[32];
    for (int l = 0; l < 32; ++l) {
      float ss = 0.0f;
      for (int32_t h = l; h < H; h += 32) {
        const float s = bf2f(ar[h]) + bf2f(br[h]);
        sr[h] = f2bf(s);
        ss += s * s;
      }
      part[l] = ss;
    }
    for (int off = 16; off > 0; off >>= 1) {
      float nxt[32];
      for (int l = 0; l < 32; ++l) nxt[l] = part[l] + part[l ^ off];
      for (int l = 0; l < 32; ++l) part[l] = nxt[l];
    }
    const float scale = 1.0f / std::sqrt(part[0] / static_cast<float>(H) + eps);
    for (int32_t h = 0; h < H; ++h) nr[h] = f2bf(bf2f(sr[h]) * scale * bf2f(w[h]));
  }
}

// swiglu, reference include/mlx-lm/common/activations.h:22-30: silu(g) * u.
void oracle_swiglu(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* h) {
  for (int64_t i = 0; i < n; ++i) h[i] = f2bf(silu_f32(bf2f(g[i])) * bf2f(u[i]));
}

// GPT-OSS's swiglu(x_linear, x_glu), reference src/llm/models/gptoss.cpp:50-58.
void oracle_gptoss_swiglu(const uint16_t* x_linear, const uint16_t* x_glu, int64_t n, uint16_t* h,
                          float* h_f32) {
  for (int64_t i = 0; i < n; ++i) {
    const float v = gptoss_glu_f32(bf2f(x_linear[i]), bf2f(x_glu[i]));
    if (h) h[i] = f2bf(v);
    if (h_f32) h_f32[i] = v;
  }
}

// gather_qmm on fp32 activations (the call at switch_layers.cpp:94-102 with
// an fp32 x): fp32 accumulation in increasing c, fp32 output; the linear bias
// (switch_layers.cpp:111-114) is added in fp32.
int oracle_gather_qmm_f32x(const float* x, const oracle_qweight* w, const uint32_t* lhs, const uint32_t* rhs,
                           int64_t batch, int32_t M, float* out) {
  if (!x || !w || !rhs || !out || batch < 0 || M <= 0 || !qweight_ok(*w)) return -1;
  const int32_t N = w->N, K = w->K;
  for (int64_t b = 0; b < batch; ++b)
    if (rhs[b] >= static_cast<uint32_t>(w->experts)) return -6;
  std::vector<std::vector<int64_t>> by_e(w->experts);
  for (int64_t b = 0; b < batch; ++b) by_e[rhs[b]].push_back(b);
  for (int32_t e = 0; e < w->experts; ++e) {
    if (by_e[e].empty()) continue;
    std::vector<float> wd(static_cast<size_t>(N) * K);
#pragma omp parallel for schedule(static)
    for (int32_t n = 0; n < N; ++n) dequant_rows(*w, e, n, 1, &wd[static_cast<size_t>(n) * K]);
    const int64_t nb = static_cast<int64_t>(by_e[e].size());
#pragma omp parallel for schedule(static)
    for (int64_t ib = 0; ib < nb * M; ++ib) {
      const int64_t b = by_e[e][ib / M];
      const int32_t m = static_cast<int32_t>(ib % M);
      const int64_t xi = lhs ? static_cast<int64_t>(lhs[b]) : b;
      const float* xr = x + (xi * M + m) * K;
      float* o = out + (b * M + m) * N;
      for (int32_t n = 0; n < N; ++n) {
        o[n] = dot_f32(xr, &wd[static_cast<size_t>(n) * K], K);
        if (w->linear_bias) o[n] += bf2f(w->linear_bias[static_cast<int64_t>(e) * N + n]);
      }
    }
  }
  return 0;
}

// Weighted combine, reference qwen3_moe.cpp:173-174: sum over k of y * scores.
void oracle_combine(const uint16_t* Y, const float* scores, int64_t T, int32_t k, int32_t H,
                    uint16_t* y) {
  for (int64_t t = 0; t < T; ++t)
    for (int32_t c = 0; c < H; ++c) {
      float acc = 0.0f;
      for (int32_t j = 0; j < k; ++j) acc += scores[t * k + j] * bf2f(Y[(t * k + j) * H + c]);
      y[t * H + c] = f2bf(acc);
    }
}

// Routed experts (SwitchGLU, switch_layers.cpp:199-245: gate|up gather_qmm,
// swiglu, down gather_qmm, unsort) followed by the model's combine
// (qwen3_moe.cpp:173-174) and the optional shared expert
// (qwen3_next.cpp:426-429 + 481-489 gated; deepseek_v3.cpp:366-379 ungated).
// Rounding: g, u, h and each expert output Y are bf16 (each reference op's
// output dtype); combine and shared contribution accumulate in fp32 and are
// rounded once.  With hidden_f32, h and Y stay fp32 (GPT-OSS's promoted
// swiglu output feeding an fp32 down projection, gptoss.cpp:50-58, 158-167).
// The routed experts' activation is b->activation (GPT-OSS:
// swiglu(x_gate, x_up) at gptoss.cpp:158).
int oracle_moe_experts(const oracle_block* b, const uint16_t* x, int64_t T, const uint32_t* inds,
                       const float* scores, uint16_t* out, float* term_mag) {
  if (!b || !x || !inds || !scores || !out || T < 0) return -1;
  const int32_t H = b->hidden, I = b->intermediate, E = b->num_experts, k = b->router.top_k;
  if (b->activation != ORACLE_ACT_SWIGLU && b->activation != ORACLE_ACT_GPTOSS &&
      b->activation != ORACLE_ACT_GPTOSS_UPSTREAM)
    return -1;
  const bool hf32 = b->hidden_f32 != 0;
  if (!qweight_ok(b->gate) || !qweight_ok(b->up) || !qweight_ok(b->down)) return -1;
  if (b->gate.N != I || b->gate.K != H || b->up.N != I || b->up.K != H || b->down.N != H ||
      b->down.K != I)
    return -1;
  const int64_t P = T * k;
  std::vector<int32_t> perm(P), offs(E + 1);
  int rc = oracle_bucket(inds, T, k, E, perm.data(), nullptr, nullptr, offs.data());
  if (rc) return rc;
  // expert outputs: bf16 values (or, hidden_f32, fp32 values) held as fp32
  std::vector<float> Y(static_cast<size_t>(P) * H);

  std::vector<float> wg(static_cast<size_t>(I) * H), wu(static_cast<size_t>(I) * H),
      wd(static_cast<size_t>(H) * I);
  for (int32_t e = 0; e < E; ++e) {
    const int32_t n_e = offs[e + 1] - offs[e];
    if (n_e == 0) continue;
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < I; ++r) {
      dequant_rows(b->gate, e, r, 1, &wg[static_cast<size_t>(r) * H]);
      dequant_rows(b->up, e, r, 1, &wu[static_cast<size_t>(r) * H]);
    }
#pragma omp parallel for schedule(static)
    for (int32_t r = 0; r < H; ++r) dequant_rows(b->down, e, r, 1, &wd[static_cast<size_t>(r) * I]);
#pragma omp parallel
    {
      std::vector<float> xf(H), hf(I);
#pragma omp for schedule(static)
      for (int32_t i = 0; i < n_e; ++i) {
        const int64_t pair = perm[offs[e] + i];
        const int64_t t = pair / k;
        for (int32_t c = 0; c < H; ++c) xf[c] = bf2f(x[t * H + c]);
        for (int32_t n = 0; n < I; ++n) {
          const float g = lin_out(dot_f32(xf.data(), &wg[static_cast<size_t>(n) * H], H), b->gate, e, n);
          const float u = lin_out(dot_f32(xf.data(), &wu[static_cast<size_t>(n) * H], H), b->up, e, n);
          const float h = glu_act_f32(b->activation, g, u);
          hf[n] = hf32 ? h : bfr(h);
        }
        for (int32_t n = 0; n < H; ++n) {
          const float dot = dot_f32(hf.data(), &wd[static_cast<size_t>(n) * I], I);
          if (hf32)  // fp32 gather_qmm output plus the bias in fp32
            Y[pair * H + n] = b->down.linear_bias
                                  ? dot + bf2f(b->down.linear_bias[static_cast<int64_t>(e) * H + n])
                                  : dot;
          else
            Y[pair * H + n] = lin_out(dot, b->down, e, n);
        }
      }
    }
  }

  std::vector<float> acc(static_cast<size_t>(T) * H, 0.0f);
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t)
    for (int32_t c = 0; c < H; ++c) {
      float a = 0.0f, m = 0.0f;
      for (int32_t j = 0; j < k; ++j) {
        const float term = scores[t * k + j] * Y[(t * k + j) * H + c];
        a += term;
        m += std::fabs(term);
      }
      acc[t * H + c] = a;
      if (term_mag) term_mag[t * H + c] = m;
    }

  if (b->shared_intermediate > 0) {
    const int32_t Is = b->shared_intermediate;
    if (!qweight_ok(b->shared_gate) || !qweight_ok(b->shared_up) || !qweight_ok(b->shared_down))
      return -1;
    std::vector<float> sg(static_cast<size_t>(Is) * H), su(static_cast<size_t>(Is) * H),
        sd(static_cast<size_t>(H) * Is), wsg(H);
    dequant_rows(b->shared_gate, 0, 0, Is, sg.data());
    dequant_rows(b->shared_up, 0, 0, Is, su.data());
    dequant_rows(b->shared_down, 0, 0, H, sd.data());
    // the sigmoid gate: bf16 [1, H], or quantized (qwen3_next.cpp:488 through linear_forward)
    const bool qgate = b->shared_gate_q.w != nullptr;
    if (qgate) {
      if (!qweight_ok(b->shared_gate_q) || b->shared_gate_q.experts != 1 || b->shared_gate_q.N != 1 ||
          b->shared_gate_q.K != H)
        return -1;
      dequant_rows(b->shared_gate_q, 0, 0, 1, wsg.data());
    } else if (b->shared_gate_weight) {
      for (int32_t c = 0; c < H; ++c) wsg[c] = bf2f(b->shared_gate_weight[c]);
    }
#pragma omp parallel
    {
      std::vector<float> xf(H), hf(Is);
#pragma omp for schedule(static)
      for (int64_t t = 0; t < T; ++t) {
        for (int32_t c = 0; c < H; ++c) xf[c] = bf2f(x[t * H + c]);
        float gate = 1.0f;
        if (qgate || b->shared_gate_weight) {
          const float gl = qgate ? lin_out(dot_f32(xf.data(), wsg.data(), H), b->shared_gate_q, 0, 0)
                                 : bfr(dot_f32(xf.data(), wsg.data(), H));
          gate = 1.0f / (1.0f + std::exp(-gl));
        }
        for (int32_t n = 0; n < Is; ++n) {
          const float g = lin_out(dot_f32(xf.data(), &sg[static_cast<size_t>(n) * H], H), b->shared_gate, 0, n);
          const float u = lin_out(dot_f32(xf.data(), &su[static_cast<size_t>(n) * H], H), b->shared_up, 0, n);
          hf[n] = bfr(silu_f32(g) * u);
        }
        for (int32_t c = 0; c < H; ++c) {
          const float ys = lin_out(dot_f32(hf.data(), &sd[static_cast<size_t>(c) * Is], Is), b->shared_down, 0, c);
          acc[t * H + c] += gate * ys;
          if (term_mag) term_mag[t * H + c] += std::fabs(gate * ys);
        }
      }
    }
  }
  for (int64_t i = 0; i < T * H; ++i) out[i] = f2bf(acc[i]);
  return 0;
}

int oracle_block_forward(const oracle_block* b, const uint16_t* x, int64_t T, uint16_t* out,
                         uint16_t* logits_out, uint32_t* inds_out, float* scores_out) {
  if (!b || !x || !out || T < 0) return -1;
  const int32_t E = b->num_experts, k = b->router.top_k;
  std::vector<uint16_t> logits(static_cast<size_t>(T) * E);
  std::vector<uint32_t> inds(static_cast<size_t>(T) * k);
  std::vector<float> scores(static_cast<size_t>(T) * k);
  int rc;
  if (b->router_q.w) {
    // quantized branch of linear_forward (quantized_linear.h:73-96): the
    // quantized matmul of every row with the one stacked matrix [E, H]
    if (b->router_q.experts != 1 || b->router_q.N != E || b->router_q.K != b->hidden) return -1;
    std::vector<uint32_t> zero(static_cast<size_t>(T), 0u);
    rc = oracle_gather_qmm(x, &b->router_q, nullptr, zero.data(), T, 1, logits.data());
  } else {
    rc = oracle_router_logits(x, b->router_weight, b->router_bias, T, b->hidden, E, logits.data());
  }
  if (rc) return rc;
  rc = oracle_route(logits.data(), b->score_bias, T, &b->router, inds.data(), scores.data(), nullptr);
  if (rc) return rc;
  rc = oracle_moe_experts(b, x, T, inds.data(), scores.data(), out, nullptr);
  if (rc) return rc;
  if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * sizeof(uint16_t));
  if (inds_out) std::memcpy(inds_out, inds.data(), inds.size() * sizeof(uint32_t));
  if (scores_out) std::memcpy(scores_out, scores.data(), scores.size() * sizeof(float));
  return 0;
}

}  // extern "C"
