// route_impl.hpp -- device code of the per-token routing (one wave per
// token) and of the bucketing of one token's k pairs, shared by the routing
// kernels (router.hip) and the gate|up kernel that routes a single token
// itself (qmm.hip).  The arithmetic of each variant follows the reference
// gates cited in router.hip and include/moe_mi355x.h; fp contraction is off
// inside these functions, so every caller evaluates the same canonical
// operation order as the CPU checker.
#pragma once

#include "internal.hpp"

namespace moe {
namespace {

struct RouteArgs {
  const uint16_t* logits;
  const float* bias;
  uint32_t* inds;
  float* scores;
  int64_t T;
  int E, k, variant, norm, n_group, topk_group;
  float rsf;
};

// Routing of token t by one whole wave (lane = lane of the wave) from its
// logits in registers: lv[i] = the bf16 logit of expert lane + 64 i (-inf
// past E).  Returns the expert of slot `lane` in lanes lane < k.
// a.inds / a.scores NULL: the weights are not formed and nothing is written
// to global memory.
template <int VPL>
__device__ __forceinline__ int route_token_lv(const RouteArgs& a, const int64_t t, const int lane,
                                              const float (&lv)[VPL], uint32_t* inds_lds = nullptr) {
#pragma clang fp contract(off)
  const int E = a.E, k = a.k;
  float sel[VPL], base[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) base[i] = 0.0f;

  if (a.variant == MOE_ROUTE_TOPK_LOGITS || a.variant == MOE_ROUTE_TOPK_PROBS ||
      a.variant == MOE_ROUTE_GLM4_SOFTMAX || a.variant == MOE_ROUTE_LFM2) {
    float m = lv[0];
#pragma unroll
    for (int i = 1; i < VPL; ++i) m = fmaxf(m, lv[i]);
    m = wave_max_fast(m);
    float part = 0.0f;
    float ex[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = lane + 64 * i;
      ex[i] = e < E ? canon_expf(lv[i] - m) : 0.0f;
      part = part + ex[i];
    }
    const float sum = wave_sum(part);
    if (a.variant == MOE_ROUTE_GLM4_SOFTMAX || a.variant == MOE_ROUTE_LFM2) {  // fp32 probabilities + bias
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int e = lane + 64 * i;
        base[i] = ex[i] / sum;
        sel[i] = base[i] + ((a.bias && e < E) ? a.bias[e] : 0.0f);
      }
    } else {
#pragma unroll
      for (int i = 0; i < VPL; ++i) base[i] = bfr(ex[i] / sum);
#pragma unroll
      for (int i = 0; i < VPL; ++i) sel[i] = a.variant == MOE_ROUTE_TOPK_LOGITS ? lv[i] : base[i];
    }
  } else if (a.variant == MOE_ROUTE_SOFTMAX_TOPK) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) sel[i] = lv[i];
  } else if (a.variant == MOE_ROUTE_SIGMOID) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      base[i] = bfr(canon_sigmoid(lv[i]));
      sel[i] = base[i];
    }
  } else {  // MOE_ROUTE_SIGMOID_GROUP, _GROUP_DROP_BEST, _CORRECTED, GLM4_SIGMOID
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = lane + 64 * i;
      base[i] = canon_sigmoid(lv[i]);
      sel[i] = base[i] + ((a.bias && e < E) ? a.bias[e] : 0.0f);
    }
    // (Bailing and GLM4-MoE compute a group index but never apply it)
    if (a.n_group > 1 && (a.variant == MOE_ROUTE_SIGMOID_GROUP || a.variant == MOE_ROUTE_SIGMOID_GROUP_DROP_BEST)) {
      const int G = a.n_group, gsz = E / G;
      int gof[VPL];  // group of each candidate (E for none), divided once
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int e = lane + 64 * i;
        gof[i] = e < E ? e / gsz : E;
      }
      float my_gs = -__builtin_inff();
      if (gsz == 16 || gsz == 32 || gsz == 64) {
        // the lanes of a register split into whole groups: every group's two
        // best at once by segmented argmax, then group g's score to lane g
        float gsv[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const int e = lane + 64 * i;
          float v1 = sel[i], v2 = sel[i];
          int i1 = e < E ? e : -1;
          if (gsz == 16) seg_argmax<16>(v1, i1);
          else if (gsz == 32) seg_argmax<32>(v1, i1);
          else seg_argmax<64>(v1, i1);
          int i2 = e < E && e != i1 ? e : -1;
          if (gsz == 16) seg_argmax<16>(v2, i2);
          else if (gsz == 32) seg_argmax<32>(v2, i2);
          else seg_argmax<64>(v2, i2);
          gsv[i] = (i2 >= 0 ? v2 : 0.0f) + (i1 >= 0 ? v1 : 0.0f);  // (a missing candidate counts 0)
        }
        const int per = 64 / gsz;  // groups per register
        const int src = (lane % per) * gsz;
        float t = gsv[0];
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const float o = __shfl(gsv[i], src, kWave);
          if (lane / per == i) t = o;
        }
        if (lane < G) my_gs = t;
      } else {
        for (int grp = 0; grp < G; ++grp) {
          // largest and second largest corrected score of the group
          float v1 = 0.0f;
          int i1 = -1;
#pragma unroll
          for (int i = 0; i < VPL; ++i) {
            const int e = lane + 64 * i;
            if (gof[i] == grp && better(sel[i], e, v1, i1)) {
              v1 = sel[i];
              i1 = e;
            }
          }
          wave_argmax(v1, i1);
          float v2 = 0.0f;
          int i2 = -1;
#pragma unroll
          for (int i = 0; i < VPL; ++i) {
            const int e = lane + 64 * i;
            if (gof[i] == grp && e != i1 && better(sel[i], e, v2, i2)) {
              v2 = sel[i];
              i2 = e;
            }
          }
          wave_argmax(v2, i2);
          if (lane == grp) my_gs = v2 + v1;
        }
      }
      // rank of group `lane` among all groups, canonical order
      int rank = 0;
      for (int g2 = 0; g2 < G; ++g2) {
        const float o = readlane_f(my_gs, g2);
        if (lane < G && better(o, g2, my_gs, lane)) ++rank;
      }
      // upstream noaux_tc keeps the topk_group best groups; as written
      // (negated group scores) the n_group - topk_group best are zeroed
      const bool keep = a.variant == MOE_ROUTE_SIGMOID_GROUP ? rank < a.topk_group : rank >= G - a.topk_group;
      const uint64_t kept = __ballot(lane < G && keep);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !((kept >> gof[i]) & 1ull)) sel[i] = sel[i] * 0.0f;
      }
    }
  }

  // k rounds of wave argmax; slot r's result is kept by lane r
  int my_idx = 0;
  float my_v = 0.0f, my_b = 0.0f;
  // the owner lane's base value of winner idx (wave-uniform idx)
  auto base_of = [&](int idx) {
    const int owner = idx & 63, isel = idx >> 6;
    float bv = base[0];
#pragma unroll
    for (int i = 1; i < VPL; ++i)
      if (i == isel) bv = base[i];
    return readlane_f(bv, owner);
  };
  bool nan_sel = false;
#pragma unroll
  for (int i = 0; i < VPL; ++i) nan_sel = nan_sel || (lane + 64 * i < E && sel[i] != sel[i]);
  if (a.variant < MOE_ROUTE_SIGMOID_GROUP && __ballot(nan_sel) == 0) {
    // the candidates are bf16 values (logits, or bf16-rounded probabilities):
    // one 32-bit key per candidate, (order-preserving 16-bit image of the
    // value) << 16 | (0xffff - expert), so the canonical order (larger value,
    // then lower index) is the unsigned order and a round is a plain wave max
    uint32_t key[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = lane + 64 * i;
      const uint32_t hb = __float_as_uint(sel[i] + 0.0f) >> 16;  // -0 -> +0 (equal values tie on the index)
      const uint32_t ord = (hb & 0x8000u) ? (~hb & 0xffffu) : (hb | 0x8000u);
      key[i] = e < E ? (ord << 16) | (0xffffu - static_cast<uint32_t>(e)) : 0u;  // real keys >= 0x007f0000
    }
    for (int r = 0; r < k; ++r) {
      uint32_t m = key[0];
#pragma unroll
      for (int i = 1; i < VPL; ++i) m = max(m, key[i]);
      m = wave_max_u32(m);
      const int idx = static_cast<int>(0xffffu - (m & 0xffffu));
      const uint32_t ord = m >> 16;
      const float v = bf2f(static_cast<uint16_t>((ord & 0x8000u) ? (ord & 0x7fffu) : (~ord & 0xffffu)));
#pragma unroll
      for (int i = 0; i < VPL; ++i) key[i] = key[i] == m ? 0u : key[i];  // taken (keys are distinct)
      const float bv = base_of(idx);
      if (lane == r) {
        my_idx = idx;
        my_v = v;
        my_b = bv;
      }
    }
  } else {
    uint32_t taken = 0;
    for (int r = 0; r < k; ++r) {
      float v = 0.0f;
      int idx = -1;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !((taken >> i) & 1u) && better(sel[i], e, v, idx)) {
          v = sel[i];
          idx = e;
        }
      }
      wave_argmax(v, idx);
      const int owner = idx & 63, isel = idx >> 6;
      if (lane == owner) taken |= 1u << isel;
      const float bv = base_of(idx);
      if (lane == r) {
        my_idx = idx;
        my_v = v;
        my_b = bv;
      }
    }
  }

  if (!a.scores) {  // the experts only
    if (lane < k && inds_lds) inds_lds[t * k + lane] = static_cast<uint32_t>(my_idx);
    return my_idx;
  }
  // weights, sums in slot order
  float w = 0.0f;
  if (a.variant == MOE_ROUTE_TOPK_LOGITS || a.variant == MOE_ROUTE_TOPK_PROBS) {
    w = my_b;
    if (a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + readlane_f(w, r);
      s = bfr(s);
      w = bfr(w / s);
    }
  } else if (a.variant == MOE_ROUTE_SOFTMAX_TOPK) {
    const float m = readlane_f(my_v, 0);
    const float ex = canon_expf(my_v - m);
    float s = 0.0f;
    for (int r = 0; r < k; ++r) s = s + readlane_f(ex, r);
    w = bfr(ex / s);
  } else if (a.variant == MOE_ROUTE_SIGMOID) {
    w = my_b;
    if (k > 1 && a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + readlane_f(w, r);
      const float denom = bfr(s) + 1e-20f;
      w = (w / denom) * a.rsf;
    }
  } else if (a.variant == MOE_ROUTE_LFM2) {
    // lfm2_moe.cpp:229-234: the biased probabilities selected are the
    // weights, renormalised with + 1e-20 for any k, cast to bf16
    w = my_v;
    if (a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + readlane_f(w, r);
      w = w / (s + 1e-20f);
    }
    w = bfr(w);
  } else if (a.variant == MOE_ROUTE_GLM4_SIGMOID || a.variant == MOE_ROUTE_GLM4_SOFTMAX) {
    // glm4_moe.cpp:180-190: the uncorrected fp32 scores, renormalised without
    // an epsilon when k > 1 and norm_topk_prob, then times the scaling factor
    w = my_b;
    if (k > 1 && a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + readlane_f(w, r);
      w = w / s;
    }
    w = w * a.rsf;
  } else {  // the sigmoid-group variants; Bailing's weights are the corrected scores, cast to bf16
    const bool corrected = a.variant == MOE_ROUTE_SIGMOID_CORRECTED;
    w = corrected ? my_v : my_b;
    if (k > 1 && a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + readlane_f(w, r);
      const float denom = s + 1e-20f;
      w = w / denom;
    }
    w = w * a.rsf;
    if (corrected) w = bfr(w);
  }
  if (lane < k) {
    a.inds[t * k + lane] = static_cast<uint32_t>(my_idx);
    a.scores[t * k + lane] = w;
    if (inds_lds) inds_lds[t * k + lane] = static_cast<uint32_t>(my_idx);
  }
  return my_idx;
}

// The same with the logits read from lrow_lds (or row t of a.logits).
template <int VPL>
__device__ __forceinline__ int route_token(const RouteArgs& a, const int64_t t, const int lane,
                                           uint32_t* inds_lds = nullptr, const uint16_t* lrow_lds = nullptr) {
  const uint16_t* lrow = lrow_lds ? lrow_lds : a.logits + t * a.E;
  float lv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    lv[i] = e < a.E ? bf2f(lrow[e]) : -__builtin_inff();
  }
  return route_token_lv<VPL>(a, t, lane, lv, inds_lds);
}

// One token's logits in the registers of one wave (lane l: experts l + 64 i,
// -inf past E) from the router's fp32 partial sums: slice q of the token's E
// values at part + q * stride (part [KS][T][E] offset to the token: stride
// T * E), KS <= 32 / VPL; each summed in slice order from slice 0 (as
// logits_from_partials), the router bias rbias (or none) added before the one
// rounding to bf16; logits_out (or NULL) receives the token's bf16 values.
// Every load is issued before the first sum; slices past KS re-read slice
// KS - 1 and are not added.
template <int VPL>
__device__ __forceinline__ void token_logits_from_partials(const float* __restrict__ part, int KS, int64_t stride,
                                                           int E, const uint16_t* __restrict__ rbias, int lane,
                                                           float (&lv)[VPL], uint16_t* __restrict__ logits_out) {
#pragma clang fp contract(off)
  constexpr int kMaxKS = 32 / VPL;
  float v[VPL][kMaxKS];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = min(lane + 64 * i, E - 1);
#pragma unroll
    for (int q = 0; q < kMaxKS; ++q) v[i][q] = part[min(q, KS - 1) * stride + e];
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    float acc = v[i][0];
#pragma unroll
    for (int q = 1; q < kMaxKS; ++q) acc = q < KS ? acc + v[i][q] : acc;
    const uint16_t b = f2bf(rbias ? acc + bf2f(rbias[min(e, E - 1)]) : acc);
    lv[i] = e < E ? bf2f(b) : -__builtin_inff();
    if (logits_out && e < E) logits_out[e] = b;
  }
}

// Bucketing of one token's k pairs by the wave that routed it (lane r < k
// holds slot r's expert).  Its experts are distinct, so sorted position of
// slot r = number of its experts below slot r's, every bucket holds one pair,
// and offsets[e] = number of its experts below e.  Same outputs as the
// general bucketing (no token-tile table).
__device__ __forceinline__ void bucket_one_token(int idx, int k, int E, const BucketOut& o) {
  const int lane = lane_id();
  int sel[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sel[r] = r < k ? __builtin_amdgcn_readlane(idx, r) : E;
  int pos = 0;
#pragma unroll
  for (int r = 0; r < 16; ++r) pos += sel[r] < idx ? 1 : 0;
  if (lane < k) {
    if (o.perm) o.perm[pos] = lane;
    if (o.inv_perm) o.inv_perm[lane] = pos;
    if (o.sorted_expert) o.sorted_expert[pos] = static_cast<uint32_t>(idx);
    if (o.sorted_token) o.sorted_token[pos] = 0;
    if (o.active) reinterpret_cast<int4*>(o.active)[pos] = make_int4(idx, pos, 1, 0);
  }
  if (o.active)
    for (int x = k + lane; x < E; x += 64) reinterpret_cast<int4*>(o.active)[x] = make_int4(0, 0, 0, 0);
  for (int e = lane; e <= E; e += 64) {
    int c = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) c += sel[r] < e ? 1 : 0;
    o.offsets[e] = c;
  }
  if (lane == 0 && o.num_active) o.num_active[0] = k;
}

// The bf16 logits of n = T*E values from the router's fp32 partial sums
// part [KS][n] (KS a power of two, KS * ceil(n / NT) <= kPartialLoads) by the
// NT threads of a workgroup: logit x = tid + NT*j is summed by its thread in
// slice order (every load of the thread issued before the first sum), the
// router bias rbias[x % E] (or none) added before the one rounding; written
// to lg (LDS) and, where logits_out is not NULL, to logits_out.
constexpr int kPartialLoads = 32;
template <int NT>
__device__ __forceinline__ void logits_from_partials(const float* __restrict__ part, int KS, int n, int E,
                                                     const uint16_t* __restrict__ rbias, uint16_t* lg,
                                                     uint16_t* __restrict__ logits_out) {
#pragma clang fp contract(off)
  // logit x = tid + NT*j takes loads u = j*KS .. j*KS + KS - 1 (slices in
  // order); loads past the end read element 0 and are never summed
  const int lks = __builtin_ctz(static_cast<unsigned>(KS));
  float v[kPartialLoads];
#pragma unroll
  for (int u = 0; u < kPartialLoads; ++u) {
    const int x = threadIdx.x + NT * (u >> lks), q = u & (KS - 1);
    v[u] = part[x < n ? q * n + x : 0];
  }
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kPartialLoads; ++u) {
    const int x = threadIdx.x + NT * (u >> lks), q = u & (KS - 1);
    acc = q == 0 ? v[u] : acc + v[u];
    if (q == KS - 1 && x < n) {
      const uint16_t b = f2bf(rbias ? acc + bf2f(rbias[x % E]) : acc);
      lg[x] = b;
      if (logits_out) logits_out[x] = b;
    }
  }
}

}  // namespace
}  // namespace moe
