// qmm.hip -- grouped affine-dequant matmul (the gather_qmm of the reference,
// src/common/switch_layers.cpp:94-102) for the MoE experts, gfx950.
//
// Work unit: one workgroup = (one expert, 16*RB output rows); its tokens are
// the expert's bucket [offsets[e], offsets[e+1]) in chunks of 16.  The waves
// of the workgroup split K in 64-wide blocks (one quantization group each)
// and are summed through LDS in wave order.
//
// Per 64-wide K block and 16x16 (token x row) tile, one wave runs two
// v_mfma_f32_16x16x32_bf16.  The weight operand is exact: a 4-bit code q
// becomes the bf16 value 128 + q by OR-ing it under the exponent pattern
// 0x4300 (bf16 has 7 mantissa bits, so 128..143 are exact), an 8-bit code is
// converted through fp32 (0..255 is exact in bf16).  Scale and bias are
// applied per group in fp32 outside the MFMA:
//     sum_k x_k (s q_k + b) = s * sum_k x_k q'_k + (b - 128 s) * sum_k x_k
// with q' = q + 128 (4-bit) or q' = q (8-bit).  No weight is rounded to bf16.
//
// Lane layout (wave64, 16x16x32 MFMA): lane = 16*g + i.  The A operand
// (tokens) takes row i, K slots 8g..8g+7; B (weights) takes column (row of W)
// i, K slots 8g..8g+7; D holds rows 4g..4g+3 of column i.  A 64-wide K block
// is split so that lane group g owns K [16g, 16g+16) of the block: slots of
// MFMA step s are K 16g + 8s + [0, 8).  For 4-bit weights the 8 codes of one
// uint32 are placed as (q0,q4,q1,q5,q2,q6,q3,q7) -- the order a shift-and-mask
// produces -- and the activations are permuted the same way.

#include "internal.hpp"

namespace moe {

struct GQArgs {
  const uint16_t* x;        // input rows [*, K] bf16
  const int32_t* row_in;    // sorted pos -> input row (NULL: pos)
  const int32_t* row_out;   // sorted pos -> output row (NULL: pos)
  const int32_t* offsets;   // [E+1]
  const int32_t* active;    // [E] non-empty experts (NULL: blockIdx.y is the expert)
  const int32_t* num_active;
  const uint32_t* w[2];
  const uint16_t* s[2];
  const uint16_t* b[2];
  int N, K, gs;
  uint16_t* out;            // [*, N] bf16
};

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 8 activations (x0..x7 as 4 packed pairs) -> (x0,x4,x1,x5,x2,x6,x3,x7)
__device__ __forceinline__ u32x4 perm_nibble_order(u32x4 v) {
  u32x4 r;
  r.x = (v.x & 0xffffu) | (v.z << 16);
  r.y = (v.x >> 16) | (v.z & 0xffff0000u);
  r.z = (v.y & 0xffffu) | (v.w << 16);
  r.w = (v.y >> 16) | (v.w & 0xffff0000u);
  return r;
}

// 8 nibbles of one word -> bf16 (128 + q) in the order (q0,q4,q1,q5,q2,q6,q3,q7)
__device__ __forceinline__ u32x4 nibbles_to_bf16(uint32_t w) {
  u32x4 r;
  r.x = (w & 0x000F000Fu) | 0x43004300u;
  r.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  r.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  r.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return r;
}

// 4 bytes of one word -> 2 packed bf16 pairs, natural order (exact: q < 256)
__device__ __forceinline__ u32x2 bytes_to_bf16(uint32_t w) {
  const uint32_t f0 = __float_as_uint(static_cast<float>(w & 0xffu));
  const uint32_t f1 = __float_as_uint(static_cast<float>((w >> 8) & 0xffu));
  const uint32_t f2 = __float_as_uint(static_cast<float>((w >> 16) & 0xffu));
  const uint32_t f3 = __float_as_uint(static_cast<float>(w >> 24));
  u32x2 r;
  r.x = (f0 >> 16) | (f1 & 0xffff0000u);
  r.y = (f2 >> 16) | (f3 & 0xffff0000u);
  return r;
}

__device__ __forceinline__ float sum8_bf16(u32x4 v) {
  float s = 0.0f;
  s += __uint_as_float(v.x << 16);
  s += __uint_as_float(v.x & 0xffff0000u);
  s += __uint_as_float(v.y << 16);
  s += __uint_as_float(v.y & 0xffff0000u);
  s += __uint_as_float(v.z << 16);
  s += __uint_as_float(v.z & 0xffff0000u);
  s += __uint_as_float(v.w << 16);
  s += __uint_as_float(v.w & 0xffff0000u);
  return s;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

template <int BITS, bool GLU, int RB>
__global__ __launch_bounds__(512) void grouped_qmm_kernel(GQArgs a) {
  constexpr int NMAT = GLU ? 2 : 1;
  __shared__ f32x4 red[8][RB * NMAT][64];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int e = blockIdx.y;
  if (a.active) {
    if (e >= a.num_active[0]) return;
    e = a.active[e];
  }
  const int beg = a.offsets[e];
  const int cnt = a.offsets[e + 1] - beg;
  if (cnt <= 0) return;

  const int g = lane >> 4, i16 = lane & 15;
  const int n0 = blockIdx.x * 16 * RB;
  const int KB = a.K >> 6;
  const int jpw = (KB + nw - 1) / nw;
  const int jb = wave * jpw;
  const int je = min(KB, jb + jpw);
  const int gpr = a.K / a.gs;
  const int gdiv = a.gs >> 6;               // 64-wide blocks per quantization group
  const int64_t wpr = static_cast<int64_t>(a.K) * BITS / 32;  // words per row

  for (int tc = 0; tc < cnt; tc += 16) {
    const int mcount = min(16, cnt - tc);
    const bool mval = i16 < mcount;
    const int pos_m = beg + tc + i16;
    const int64_t xrow = mval ? (a.row_in ? a.row_in[pos_m] : pos_m) : 0;
    const uint16_t* xp = a.x + xrow * a.K + 16 * g;

    f32x4 acc[RB][NMAT];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) acc[rb][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int j = jb; j < je; ++j) {
      const u32x4 zero = {0u, 0u, 0u, 0u};
      const u32x4 xa0 = mval ? *reinterpret_cast<const u32x4*>(xp + 64 * j) : zero;
      const u32x4 xa1 = mval ? *reinterpret_cast<const u32x4*>(xp + 64 * j + 8) : zero;
      float xs = sum8_bf16(xa0) + sum8_bf16(xa1);
      xs += __shfl_xor(xs, 16, 64);
      xs += __shfl_xor(xs, 32, 64);
      float xr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) xr[r] = __shfl(xs, 4 * g + r, 64);
      const bf16x8 A0 = __builtin_bit_cast(bf16x8, BITS == 4 ? perm_nibble_order(xa0) : xa0);
      const bf16x8 A1 = __builtin_bit_cast(bf16x8, BITS == 4 ? perm_nibble_order(xa1) : xa1);
      const int sidx = j / gdiv;

#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int64_t row = static_cast<int64_t>(e) * a.N + n0 + 16 * rb + i16;
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) {
          bf16x8 B0, B1;
          if constexpr (BITS == 4) {
            const u32x2 wq = *reinterpret_cast<const u32x2*>(a.w[mt] + row * wpr + 8 * j + 2 * g);
            B0 = __builtin_bit_cast(bf16x8, nibbles_to_bf16(wq.x));
            B1 = __builtin_bit_cast(bf16x8, nibbles_to_bf16(wq.y));
          } else {
            const u32x4 wq = *reinterpret_cast<const u32x4*>(a.w[mt] + row * wpr + 16 * j + 4 * g);
            const u32x2 p0 = bytes_to_bf16(wq.x), p1 = bytes_to_bf16(wq.y);
            const u32x2 p2 = bytes_to_bf16(wq.z), p3 = bytes_to_bf16(wq.w);
            B0 = __builtin_bit_cast(bf16x8, u32x4{p0.x, p0.y, p1.x, p1.y});
            B1 = __builtin_bit_cast(bf16x8, u32x4{p2.x, p2.y, p3.x, p3.y});
          }
          const float sc = bf2f(a.s[mt][row * gpr + sidx]);
          const float bi = a.b[mt] ? bf2f(a.b[mt][row * gpr + sidx]) : 0.0f;
          const float bp = BITS == 4 ? bi - 128.0f * sc : bi;
          f32x4 c = {0.f, 0.f, 0.f, 0.f};
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, B0, c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, B1, c, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[rb][mt][r] = fmaf(sc, c[r], fmaf(bp, xr[r], acc[rb][mt][r]));
        }
      }
    }

#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) red[wave][rb * NMAT + mt][lane] = acc[rb][mt];
    __syncthreads();
    for (int rb = wave; rb < RB; rb += nw) {
      f32x4 v[NMAT];
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt) {
        v[mt] = red[0][rb * NMAT + mt][lane];
        for (int w = 1; w < nw; ++w) v[mt] += red[w][rb * NMAT + mt][lane];
      }
      const int col = n0 + 16 * rb + i16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r;
        if (m >= mcount) continue;
        const int pos = beg + tc + m;
        const int64_t orow = a.row_out ? a.row_out[pos] : pos;
        float o;
        if constexpr (GLU) {
          const float gg = bfr(v[0][r]), uu = bfr(v[1][r]);
          o = silu(gg) * uu;
        } else {
          o = v[0][r];
        }
        a.out[orow * a.N + col] = f2bf(o);
      }
    }
    __syncthreads();
  }
}

__global__ void swiglu_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                              int64_t n, uint16_t* __restrict__ h) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) h[i] = f2bf(silu(bf2f(g[i])) * bf2f(u[i]));
}

// y[t, 8c..8c+8) = bf16(sum_j scores[t,j] * Y[row(t,j)] + gate_t * Ys[t])
__global__ void combine_kernel(const uint16_t* __restrict__ Y, const int32_t* __restrict__ inv_perm,
                               const float* __restrict__ scores, int64_t T, int k, int H,
                               const uint16_t* __restrict__ Ys, const uint16_t* __restrict__ sgl,
                               uint16_t* __restrict__ y) {
  const int cpr = H >> 3;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= T * cpr) return;
  const int64_t t = idx / cpr;
  const int c = static_cast<int>(idx % cpr) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < k; ++j) {
    const int64_t f = t * k + j;
    const int64_t row = inv_perm ? inv_perm[f] : f;
    const float s = scores[f];
    const u32x4 v = *reinterpret_cast<const u32x4*>(Y + row * H + c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += s * __uint_as_float(v[q] << 16);
      acc[2 * q + 1] += s * __uint_as_float(v[q] & 0xffff0000u);
    }
  }
  if (Ys) {
    const float gate = sgl ? 1.0f / (1.0f + __expf(-bf2f(sgl[t]))) : 1.0f;
    const u32x4 v = *reinterpret_cast<const u32x4*>(Ys + t * H + c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += gate * __uint_as_float(v[q] << 16);
      acc[2 * q + 1] += gate * __uint_as_float(v[q] & 0xffff0000u);
    }
  }
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  *reinterpret_cast<u32x4*>(y + t * H + c) = o;
}

template <int BITS, bool GLU>
int launch_rb(const GQArgs& a, int rb, dim3 grid, int nw, hipStream_t stream) {
  switch (rb) {
    case 4:
      MOE_LAUNCH(GLU ? "qmm_gate_up_swiglu" : "qmm_down", (grouped_qmm_kernel<BITS, GLU, 4>), grid, dim3(nw * 64), 0, stream, a);
      break;
    case 2:
      MOE_LAUNCH(GLU ? "qmm_gate_up_swiglu" : "qmm_down", (grouped_qmm_kernel<BITS, GLU, 2>), grid, dim3(nw * 64), 0, stream, a);
      break;
    default:
      MOE_LAUNCH(GLU ? "qmm_gate_up_swiglu" : "qmm_down", (grouped_qmm_kernel<BITS, GLU, 1>), grid, dim3(nw * 64), 0, stream, a);
      break;
  }
  return launch_status("grouped_qmm");
}

}  // namespace

// Validates one stacked quantized projection for the grouped kernel.
int qweight_check(const moe_qweight* w) {
  if (!w || !w->w || !w->scales) return MOE_E_INVALID_ARG;
  if (w->experts <= 0 || w->N <= 0 || w->K <= 0) return MOE_E_INVALID_ARG;
  if (w->bits != 4 && w->bits != 8) return MOE_E_UNSUPPORTED;
  if (w->group_size != 64 && w->group_size != 128) return MOE_E_UNSUPPORTED;
  if (w->K % w->group_size != 0 || w->N % 16 != 0) return MOE_E_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(w->w) & 15u) != 0) return MOE_E_UNSUPPORTED;
  return MOE_OK;
}

// Launch the grouped kernel.  `slots` = grid.y (experts or active slots).
// w1 non-NULL selects the gate|up + SwiGLU variant.
bool use_prefill(int64_t P, int slots, const moe_qweight* w0, const moe_qweight* w1) {
  return P >= 64 * static_cast<int64_t>(slots) && prefill_supported(w0, w1);
}

int grouped_qmm(const uint16_t* x, const int32_t* row_in, const int32_t* row_out,
                const int32_t* offsets, const int32_t* active, const int32_t* num_active,
                int slots, int64_t P, const PrefillScratch* pf, const moe_qweight* w0,
                const moe_qweight* w1, uint16_t* out, hipStream_t stream) {
  int st = qweight_check(w0);
  if (st != MOE_OK) return st;
  if (w1) {
    st = qweight_check(w1);
    if (st != MOE_OK) return st;
    if (w1->N != w0->N || w1->K != w0->K || w1->bits != w0->bits || w1->group_size != w0->group_size ||
        w1->experts != w0->experts)
      return MOE_E_INVALID_ARG;
  }
  if (!x || !offsets || !out || slots < 0) return MOE_E_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return MOE_E_UNSUPPORTED;
  if (slots == 0) return MOE_OK;
  // Large buckets (prefill): the LDS-staged GEMM.  Small buckets (decode):
  // the per-16-row kernel below.
  if (pf && use_prefill(P, slots, w0, w1))
    return grouped_gemm_prefill(x, pf->x_rows, row_in, row_out, pf->gsum, offsets, pf->tiles, w0->experts, P,
                                slots, w0, w1, out, stream);
  GQArgs a{};
  a.x = x;
  a.row_in = row_in;
  a.row_out = row_out;
  a.offsets = offsets;
  a.active = active;
  a.num_active = num_active;
  a.w[0] = w0->w;
  a.s[0] = w0->scales;
  a.b[0] = w0->biases;
  if (w1) {
    a.w[1] = w1->w;
    a.s[1] = w1->scales;
    a.b[1] = w1->biases;
  }
  a.N = w0->N;
  a.K = w0->K;
  a.gs = w0->group_size;
  a.out = out;

  const int KB = a.K / 64;
  const int per = (KB + 7) / 8;
  const int nw = (KB + per - 1) / per;
  const int tiles16 = a.N / 16;
  int rb = 1;
  if (tiles16 % 4 == 0 && static_cast<int64_t>(tiles16 / 4) * slots >= 1024) rb = 4;
  else if (tiles16 % 2 == 0 && static_cast<int64_t>(tiles16 / 2) * slots >= 1024) rb = 2;
  dim3 grid(tiles16 / rb, slots);
  if (w0->bits == 4)
    return w1 ? launch_rb<4, true>(a, rb, grid, nw, stream) : launch_rb<4, false>(a, rb, grid, nw, stream);
  return w1 ? launch_rb<8, true>(a, rb, grid, nw, stream) : launch_rb<8, false>(a, rb, grid, nw, stream);
}

int swiglu(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* h, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!g || !u || !h))) return MOE_E_INVALID_ARG;
  if (n == 0) return MOE_OK;
  MOE_LAUNCH("swiglu", swiglu_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     stream, g, u, n, h);
  return launch_status("swiglu");
}

int combine(const uint16_t* Y, const int32_t* inv_perm, const float* scores, int64_t T, int k,
            int H, const uint16_t* Ys, const uint16_t* sgl, uint16_t* y, hipStream_t stream) {
  if (T < 0 || k <= 0 || H <= 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!Y || !scores || !y) return MOE_E_INVALID_ARG;
  if (H % 8 != 0 || (reinterpret_cast<uintptr_t>(Y) & 15u) || (reinterpret_cast<uintptr_t>(y) & 15u) ||
      (Ys && (reinterpret_cast<uintptr_t>(Ys) & 15u)))
    return MOE_E_UNSUPPORTED;
  const int64_t n = T * (H / 8);
  MOE_LAUNCH("combine", combine_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     stream, Y, inv_perm, scores, T, k, H, Ys, sgl, y);
  return launch_status("combine");
}

}  // namespace moe
