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
// index on ties.  Index -1 marks "no candidate" and always loses.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  if (ib < 0) return ia >= 0;
  if (ia < 0) return false;
  if (va > vb) return true;
  if (va < vb) return false;
  return ia < ib;
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, kWave);
    const int oi = __shfl_xor(i, off, kWave);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

}  // namespace moe

// ---- host-side error plumbing --------------------------------------------------
namespace moe {
void set_last_error(const char* where, hipError_t e);
int launch_status(const char* where);
// Per-kernel event timing (no-ops unless moe_profile_enable(1) was called).
void prof_begin(hipStream_t stream, const char* name);
void prof_end(hipStream_t stream);
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
