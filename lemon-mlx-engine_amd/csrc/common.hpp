// common.hpp -- shared device helpers for the MI355X MoE kernels (gfx950,
// wave64).  Every .hip file of the library includes this.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "moe_mi355x.h"

namespace moe {

constexpr int kWave = 64;

// ---- bf16 <-> fp32 --------------------------------------------------------
__device__ __host__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even; NaN stays a quiet NaN.  Branch-free (a select), so
// it never splits a wave.
__device__ __host__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet = (u >> 16) | 0x40u;
  return static_cast<uint16_t>((u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

__device__ __forceinline__ float bfr(float f) { return bf2f(f2bf(f)); }

// Two floats -> packed bf16x2 (lo = a, hi = b), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return static_cast<uint32_t>(f2bf(a)) | (static_cast<uint32_t>(f2bf(b)) << 16);
}

// ---- canonical exp ---------------------------------------------------------
// Cody-Waite reduction x = n*ln2 + r (two-part ln2, ln2_hi with 15
// significant bits), exp(r) by the degree-7 Taylor polynomial in Horner form
// with fused multiply-adds, scaled by 2^n.  Inputs below -87 give 0, above
// 88.72 give +inf; no subnormal results.  The CPU checker evaluates the same
// sequence, so router scores agree bit for bit.
__device__ __forceinline__ float canon_expf(float x) {
  if (x != x) return x;
  if (x > 88.72f) return __builtin_inff();
  if (x < -87.0f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269504f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.42860677e-6f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ float canon_sigmoid(float v) { return 1.0f / (1.0f + canon_expf(-v)); }

// ---- GLU activations of the expert MLP (moe_activation) --------------------
// GPT-OSS's clipped SwiGLU, src/llm/models/gptoss.cpp:50-58 with its default
// alpha = 1.702, limit = 7: xl = clip(x_linear, -7, 7), xg = min(x_glu, 7),
// (xg * sigmoid(alpha * xg)) * (xl + 1), in fp32 in the order written there.
__device__ __forceinline__ float gptoss_glu(float x_linear, float x_glu) {
  const float xl = fminf(fmaxf(x_linear, -7.0f), 7.0f);
  const float xg = fminf(x_glu, 7.0f);
  const float sig = 1.0f / (1.0f + __expf(-(1.702f * xg)));
  return (xg * sig) * (xl + 1.0f);
}

// h of the bf16 gate value g and up value u; silu_g = silu(g) as the calling
// kernel computes it (used by MOE_ACT_SWIGLU only).  act is uniform over the
// launch (a kernel argument), so the branch is scalar.
__device__ __forceinline__ float glu_act(int act, float g, float u, float silu_g) {
  if (act == MOE_ACT_GPTOSS) return gptoss_glu(g, u);           // swiglu(x_gate, x_up), gptoss.cpp:158
  if (act == MOE_ACT_GPTOSS_UPSTREAM) return gptoss_glu(u, g);  // the upstream roles
  return silu_g * u;
}

// ---- pair K order --------------------------------------------------------------
// Within every 8 consecutive K values of an activation row the stored order is
// (0, 4, 1, 5, 2, 6, 3, 7): the order in which the expert GEMMs build their
// 4-bit code operand cheapest.  pair_pos(j) = stored position of K value j.
__host__ __device__ __forceinline__ int pair_pos(int j) { return ((j & 3) << 1) | (j >> 2); }

// natural 16-byte unit (x0..x7 as 4 packed bf16 pairs) -> pair order
template <class V4>
__device__ __forceinline__ V4 to_pair_order(V4 v) {
  V4 r;
  r[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);  // x0, x4
  r[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);  // x1, x5
  r[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);  // x2, x6
  r[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);  // x3, x7
  return r;
}

// ---- wave64 primitives -------------------------------------------------------
__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, kWave);
  return v;
}

// (value, index) argmax with the canonical order: larger value first, lower
// index on ties (and where neither value is larger, e.g. a NaN).  Index -1
// marks "no candidate" and always loses.  Written with non-short-circuit
// operators so that it compiles to compares and mask logic, not to nested
// exec-mask branches (one wave routes a token: every branch is on its path).
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  const bool a_ok = ia >= 0, b_none = ib < 0;
  const bool wins = (va > vb) | (!(va < vb) & (ia < ib));
  return b_none ? a_ok : (a_ok & wins);
}

// ---- cross-lane moves without the LDS pipeline ------------------------------
// DPP row controls (gfx9): quad permutations [1,0,3,2] and [2,3,0,1] (xor 1,
// xor 2), row_half_mirror (lane i <-> 7-i within 8), row_mirror (i <-> 15-i
// within 16).
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <int CTRL>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
  const float ov = dpp_f<CTRL>(v);
  const int oi = dpp_i<CTRL>(i);
  const bool take = better(ov, oi, v, i);
  v = take ? ov : v;
  i = take ? oi : i;
}

// (value, index) argmax within each aligned segment of SEG lanes (16, 32 or
// 64); every lane of a segment gets its segment's winner.  The rows of 16 run
// on DPP, then xor 16 (ds_swizzle) and xor 32 (ds_bpermute).
template <int SEG>
__device__ __forceinline__ void seg_argmax(float& v, int& i) {
  static_assert(SEG == 16 || SEG == 32 || SEG == 64, "segment");
  argmax_step<kDppQuadXor1>(v, i);
  argmax_step<kDppQuadXor2>(v, i);
  argmax_step<kDppHalfMirror>(v, i);
  argmax_step<kDppMirror>(v, i);
  auto merge = [&](float ov, int oi) {
    const bool take = better(ov, oi, v, i);
    v = take ? ov : v;
    i = take ? oi : i;
  };
  if constexpr (SEG >= 32)  // swizzle bit mode: and 0x1f, xor 0x10 within 32 lanes
    merge(__int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f)),
          __builtin_amdgcn_ds_swizzle(i, 0x401f));
  if constexpr (SEG == 64) merge(__shfl_xor(v, 32, kWave), __shfl_xor(i, 32, kWave));
}

// Wave-wide (value, index) argmax in the canonical order; the result is
// returned in every lane (wave-uniform).  The winner does not depend on the
// order of comparisons, so the reduction runs within each row of 16 lanes on
// DPP and finishes over the four row winners read into scalars.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  argmax_step<kDppQuadXor1>(v, i);
  argmax_step<kDppQuadXor2>(v, i);
  argmax_step<kDppHalfMirror>(v, i);
  argmax_step<kDppMirror>(v, i);
  float bv = readlane_f(v, 0);
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) {
    const float ov = readlane_f(v, 16 * r);
    const int oi = __builtin_amdgcn_readlane(i, 16 * r);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  v = bv;
  i = bi;
}

// Wave-wide max (order-free), returned in every lane.
__device__ __forceinline__ float wave_max_fast(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Wave-wide unsigned max, returned in every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(dpp_i<kDppQuadXor1>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i<kDppQuadXor2>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i<kDppHalfMirror>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i<kDppMirror>(static_cast<int>(v))));
  const uint32_t r0 = __builtin_amdgcn_readlane(static_cast<int>(v), 0);
  const uint32_t r1 = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(static_cast<int>(v), 32);
  const uint32_t r3 = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  return max(max(r0, r1), max(r2, r3));
}

// ---- direct-to-LDS loads and LDS-only barriers ------------------------------
// 16 bytes per lane from global memory straight into LDS (no VGPR staging):
// lane i's bytes land at lds_base + 16*i; lds_base is wave-uniform.
__device__ __forceinline__ void load_lds16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(src),
                                   (__attribute__((address_space(3))) void*)(lds_base), 16, 0, 0);
}

// 4 bytes per lane likewise: lane i's bytes land at lds_base + 4*i.
__device__ __forceinline__ void load_lds4(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(src),
                                   (__attribute__((address_space(3))) void*)(lds_base), 4, 0, 0);
}

// Raw buffer resource over `base` (wave-uniform): byte offsets up to 2^32 - 1,
// no stride, 32-bit data format (the gfx9 word-3 value for raw buffers).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), -1, 0x00020000);
}

// 16 bytes per lane from rsrc + voff + soff straight into LDS: lane i's bytes
// land at lds_base + 16*i.  voff is the lane's 32-bit offset, soff a
// wave-uniform one (no vector address arithmetic per step).
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff,
                                                  void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(lds_base), 16, voff,
                                           soff, 0, 0);
}

// Wait until at most N of this wave's global loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);  // vmcnt(N) expcnt(7) lgkmcnt(15)
}

// Workgroup barrier that orders LDS traffic only: this wave's LDS reads and
// writes complete (lgkmcnt(0)), then s_barrier.  Unlike __syncthreads() it
// does not wait for outstanding global loads (vmcnt), so prefetches issued
// for later K steps stay in flight across it.  The empty asm statements keep
// the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt(63) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

}  // namespace moe

// ---- host-side error plumbing --------------------------------------------------
namespace moe {
void set_last_error(const char* where, hipError_t e);
int launch_status(const char* where);
// Per-kernel event timing (no-ops unless moe_profile_enable(1) was called).
void prof_begin(hipStream_t stream, const char* name);
void prof_end(hipStream_t stream);
// Launches inside a ProfScope are recorded under the scope's label for the
// kernel (the shared expert's and the quantized router's projections run the
// routed experts' kernels; their records must not mix with the routed ones).
enum class ProfLabel { kNone, kShared, kRouterQ };
struct ProfScope {
  explicit ProfScope(ProfLabel l);
  ~ProfScope();
  ProfLabel prev;
};
}  // namespace moe

// Launch a kernel bracketed by the profiler's events.
#define MOE_LAUNCH(name, kernel, grid, block, lds, stream, ...)               \
  do {                                                                        \
    ::moe::prof_begin(stream, name);                                          \
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);        \
    ::moe::prof_end(stream);                                                  \
  } while (0)

#define MOE_CHECK_LAUNCH(where)                 \
  do {                                          \
    int _st = ::moe::launch_status(where);      \
    if (_st != MOE_OK) return _st;              \
  } while (0)
