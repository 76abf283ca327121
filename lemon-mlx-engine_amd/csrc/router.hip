// router.hip -- router projection and per-token scoring / top-k (gfx950).
//
// moe_router_logits: logits = bf16(x . Wg^T) on bf16 MFMA (16x16x32), fp32
//   accumulation, K split over the four waves of a workgroup.
// moe_route: one wave64 per token.  Lane l holds experts l, l+64, l+128, ...
//   in registers; the softmax denominator is 64 strided partials reduced by an
//   xor butterfly (the canonical order the CPU checker restates), top-k is k
//   rounds of a wave argmax with the canonical (value desc, index asc) order.
#pragma clang fp contract(off)

#include "internal.hpp"

namespace moe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// C[M, N] = A[M, K] . B[N, K]^T, bf16 in / bf16 out.  One workgroup = one
// 16x16 output tile; its 4 waves take interleaved 32-wide K steps and are
// summed through LDS in wave order.
__global__ __launch_bounds__(256) void gemm_nt_bf16_tile16(const uint16_t* __restrict__ A,
                                                         const uint16_t* __restrict__ B,
                                                         uint16_t* __restrict__ C, int M,
                                                         int N, int K) {
  __shared__ float red[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const int i = lane & 15, g = lane >> 4;
  const int arow = m0 + i, brow = n0 + i;
  const bool aok = arow < M, bok = brow < N;
  const uint16_t* ap = A + static_cast<int64_t>(aok ? arow : 0) * K + 8 * g;
  const uint16_t* bp = B + static_cast<int64_t>(bok ? brow : 0) * K + 8 * g;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int k0 = wave * 32; k0 < K; k0 += 128) {
    u32x4 av = aok ? *reinterpret_cast<const u32x4*>(ap + k0) : zero;
    u32x4 bv = bok ? *reinterpret_cast<const u32x4*>(bp + k0) : zero;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                  __builtin_bit_cast(bf16x8, bv), acc, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][lane * 4 + r] = acc[r];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = ((red[0][lane * 4 + r] + red[1][lane * 4 + r]) + red[2][lane * 4 + r]) +
                      red[3][lane * 4 + r];
      // D layout of 16x16 MFMA: column = lane%16, row = 4*(lane/16) + r
      const int row = m0 + 4 * g + r, col = n0 + i;
      if (row < M && col < N) C[static_cast<int64_t>(row) * N + col] = f2bf(v);
    }
  }
}

struct RouteArgs {
  const uint16_t* logits;
  const float* bias;
  uint32_t* inds;
  float* scores;
  int64_t T;
  int E, k, variant, norm, n_group, topk_group;
  float rsf;
};

template <int VPL>
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= a.T) return;
  const int E = a.E, k = a.k;
  const uint16_t* lrow = a.logits + t * E;

  float lv[VPL], sel[VPL], base[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + 64 * i;
    lv[i] = e < E ? bf2f(lrow[e]) : -__builtin_inff();
    base[i] = 0.0f;
  }

  if (a.variant == MOE_ROUTE_TOPK_LOGITS || a.variant == MOE_ROUTE_TOPK_PROBS) {
    float m = lv[0];
#pragma unroll
    for (int i = 1; i < VPL; ++i) m = fmaxf(m, lv[i]);
    m = wave_max(m);
    float part = 0.0f;
    float ex[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = lane + 64 * i;
      ex[i] = e < E ? canon_expf(lv[i] - m) : 0.0f;
      part = part + ex[i];
    }
    const float sum = wave_sum(part);
#pragma unroll
    for (int i = 0; i < VPL; ++i) base[i] = bfr(ex[i] / sum);
#pragma unroll
    for (int i = 0; i < VPL; ++i) sel[i] = a.variant == MOE_ROUTE_TOPK_LOGITS ? lv[i] : base[i];
  } else if (a.variant == MOE_ROUTE_SOFTMAX_TOPK) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) sel[i] = lv[i];
  } else if (a.variant == MOE_ROUTE_SIGMOID) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      base[i] = bfr(canon_sigmoid(lv[i]));
      sel[i] = base[i];
    }
  } else {  // MOE_ROUTE_SIGMOID_GROUP
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = lane + 64 * i;
      base[i] = canon_sigmoid(lv[i]);
      sel[i] = base[i] + ((a.bias && e < E) ? a.bias[e] : 0.0f);
    }
    if (a.n_group > 1) {
      const int G = a.n_group, gsz = E / G;
      float my_gs = -__builtin_inff();
      for (int grp = 0; grp < G; ++grp) {
        // largest and second largest corrected score of the group
        float v1 = 0.0f;
        int i1 = -1;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          const int e = lane + 64 * i;
          if (e < E && e / gsz == grp && better(sel[i], e, v1, i1)) {
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
          if (e < E && e / gsz == grp && e != i1 && better(sel[i], e, v2, i2)) {
            v2 = sel[i];
            i2 = e;
          }
        }
        wave_argmax(v2, i2);
        if (lane == grp) my_gs = v2 + v1;
      }
      // rank of group `lane` among all groups, canonical order
      int rank = 0;
      for (int g2 = 0; g2 < G; ++g2) {
        const float o = __shfl(my_gs, g2, 64);
        if (lane < G && better(o, g2, my_gs, lane)) ++rank;
      }
      const uint64_t kept = __ballot(lane < G && rank < a.topk_group);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !((kept >> (e / gsz)) & 1ull)) sel[i] = sel[i] * 0.0f;
      }
    }
  }

  // k rounds of wave argmax; slot r's result is kept by lane r
  uint32_t taken = 0;
  int my_idx = 0;
  float my_v = 0.0f, my_b = 0.0f;
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
    float bv = base[0];
#pragma unroll
    for (int i = 1; i < VPL; ++i)
      if (i == isel) bv = base[i];
    if (lane == owner) taken |= 1u << isel;
    bv = __shfl(bv, owner, 64);
    if (lane == r) {
      my_idx = idx;
      my_v = v;
      my_b = bv;
    }
  }

  // weights, sums in slot order
  float w = 0.0f;
  if (a.variant == MOE_ROUTE_TOPK_LOGITS || a.variant == MOE_ROUTE_TOPK_PROBS) {
    w = my_b;
    if (a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + __shfl(w, r, 64);
      s = bfr(s);
      w = bfr(w / s);
    }
  } else if (a.variant == MOE_ROUTE_SOFTMAX_TOPK) {
    const float m = __shfl(my_v, 0, 64);
    const float ex = canon_expf(my_v - m);
    float s = 0.0f;
    for (int r = 0; r < k; ++r) s = s + __shfl(ex, r, 64);
    w = bfr(ex / s);
  } else if (a.variant == MOE_ROUTE_SIGMOID) {
    w = my_b;
    if (k > 1 && a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + __shfl(w, r, 64);
      const float denom = bfr(s) + 1e-20f;
      w = (w / denom) * a.rsf;
    }
  } else {
    w = my_b;
    if (k > 1 && a.norm) {
      float s = 0.0f;
      for (int r = 0; r < k; ++r) s = s + __shfl(w, r, 64);
      const float denom = s + 1e-20f;
      w = w / denom;
    }
    w = w * a.rsf;
  }
  if (lane < k) {
    a.inds[t * k + lane] = static_cast<uint32_t>(my_idx);
    a.scores[t * k + lane] = w;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int router_logits(const uint16_t* x, const uint16_t* wg, int64_t T, int32_t H, int32_t E,
                  uint16_t* logits, hipStream_t stream) {
  if (!x || !wg || !logits || T < 0 || H <= 0 || E <= 0) return MOE_E_INVALID_ARG;
  if (H % 32 != 0 || !aligned16(x) || !aligned16(wg)) return MOE_E_UNSUPPORTED;
  if (T == 0) return MOE_OK;
  if ((T + 15) / 16 > 0x7fffffff) return MOE_E_UNSUPPORTED;
  dim3 grid((E + 15) / 16, static_cast<unsigned>((T + 15) / 16));
  MOE_LAUNCH("router_logits", gemm_nt_bf16_tile16, grid, dim3(256), 0, stream, x, wg, logits,
                     static_cast<int>(T), E, H);
  MOE_CHECK_LAUNCH("router_logits");
  return MOE_OK;
}

int route_validate(const moe_router_params* p) {
  if (!p) return MOE_E_INVALID_ARG;
  const int E = p->num_experts, k = p->top_k;
  if (E <= 0 || k <= 0 || k > E) return MOE_E_INVALID_ARG;
  if (E > 1024 || k > 16) return MOE_E_UNSUPPORTED;
  switch (p->variant) {
    case MOE_ROUTE_TOPK_LOGITS:
    case MOE_ROUTE_TOPK_PROBS:
    case MOE_ROUTE_SOFTMAX_TOPK:
    case MOE_ROUTE_SIGMOID:
      return MOE_OK;
    case MOE_ROUTE_SIGMOID_GROUP:
      if (p->n_group <= 1) return MOE_OK;
      if (p->n_group > 64 || E % p->n_group != 0 || E / p->n_group < 2) return MOE_E_UNSUPPORTED;
      if (p->topk_group < 1 || p->topk_group > p->n_group) return MOE_E_INVALID_ARG;
      return MOE_OK;
    default:
      return MOE_E_INVALID_ARG;
  }
}

int route(const uint16_t* logits, const float* bias, int64_t T, const moe_router_params* p,
          uint32_t* inds, float* scores, hipStream_t stream) {
  int st = route_validate(p);
  if (st != MOE_OK) return st;
  if (!logits || !inds || !scores || T < 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if ((T + 3) / 4 > 0x7fffffff) return MOE_E_UNSUPPORTED;
  RouteArgs a{logits, bias, inds, scores, T, p->num_experts, p->top_k, p->variant,
              p->norm_topk_prob, p->n_group, p->topk_group, p->routed_scaling_factor};
  dim3 grid(static_cast<unsigned>((T + 3) / 4));
  const int vpl = (p->num_experts + 63) / 64;
  if (vpl <= 1)
    MOE_LAUNCH("route", route_kernel<1>, grid, dim3(256), 0, stream, a);
  else if (vpl <= 2)
    MOE_LAUNCH("route", route_kernel<2>, grid, dim3(256), 0, stream, a);
  else if (vpl <= 4)
    MOE_LAUNCH("route", route_kernel<4>, grid, dim3(256), 0, stream, a);
  else if (vpl <= 8)
    MOE_LAUNCH("route", route_kernel<8>, grid, dim3(256), 0, stream, a);
  else
    MOE_LAUNCH("route", route_kernel<16>, grid, dim3(256), 0, stream, a);
  MOE_CHECK_LAUNCH("route");
  return MOE_OK;
}

}  // namespace moe
