// norm.hip -- the step before the MoE block: residual add + RMSNorm in one
// pass (reference add_rms_norm, src/common/gated_delta.cpp:313-345, called at
// src/llm/models/qwen35_moe.cpp:787-788 to produce the MoE input), gfx950.
//
//   s       = fp32(a) + fp32(b)                   (per element)
//   sum_out = bf16(s)
//   scale   = 1 / sqrt(sum(s^2) / H + eps)        (the unrounded s)
//   normed  = bf16(fp32(sum_out) * scale * fp32(weight))
//
// One wave per row: each lane holds 8-element (16-byte) chunks of the row in
// registers, so the row is read once and both outputs are written with 16-byte
// stores; the squares are summed per lane then across the wave.  HBM-bound:
// 4 H bytes read and 4 H bytes written per row (the weight stays in L2).

#include "internal.hpp"

namespace moe {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kNormMaxChunks = 16;  // 16-byte chunks per lane: H <= 64 * 16 * 8 = 8192

template <int NC>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(const uint16_t* __restrict__ a,
                                                           const uint16_t* __restrict__ b,
                                                           const uint16_t* __restrict__ w, float eps, int64_t T,
                                                           int H, uint16_t* __restrict__ sum_out,
                                                           uint16_t* __restrict__ normed) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= T) return;
  const int nch = H >> 3;  // 16-byte chunks of the row
  const u32x4* ar = reinterpret_cast<const u32x4*>(a + row * H);
  const u32x4* br = reinterpret_cast<const u32x4*>(b + row * H);
  u32x4 sv[NC];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nch) {
      const u32x4 va = ar[ch], vb = br[ch];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float s0 = __uint_as_float(va[q] << 16) + __uint_as_float(vb[q] << 16);
        const float s1 = __uint_as_float(va[q] & 0xffff0000u) + __uint_as_float(vb[q] & 0xffff0000u);
        ss = fmaf(s0, s0, ss);
        ss = fmaf(s1, s1, ss);
        sv[c][q] = pack_bf16x2(s0, s1);
      }
      reinterpret_cast<u32x4*>(sum_out + row * H)[ch] = sv[c];
    }
  }
  ss = wave_sum(ss);
  const float scale = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  const u32x4* wr = reinterpret_cast<const u32x4*>(w);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nch) {
      const u32x4 vw = wr[ch];
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack_bf16x2(__uint_as_float(sv[c][q] << 16) * scale * __uint_as_float(vw[q] << 16),
                           __uint_as_float(sv[c][q] & 0xffff0000u) * scale * __uint_as_float(vw[q] & 0xffff0000u));
      reinterpret_cast<u32x4*>(normed + row * H)[ch] = o;
    }
  }
}

}  // namespace

int add_rms_norm(const uint16_t* a, const uint16_t* b, const uint16_t* w, float eps, int64_t T, int H,
                 uint16_t* sum_out, uint16_t* normed, hipStream_t stream) {
  if (T < 0 || H <= 0 || !(eps >= 0.0f)) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!a || !b || !w || !sum_out || !normed) return MOE_E_INVALID_ARG;
  if (H % 8 != 0 || H > 64 * 8 * kNormMaxChunks) return MOE_E_UNSUPPORTED;
  for (const void* p : {static_cast<const void*>(a), static_cast<const void*>(b), static_cast<const void*>(w),
                        static_cast<const void*>(sum_out), static_cast<const void*>(normed)})
    if (reinterpret_cast<uintptr_t>(p) & 15u) return MOE_E_UNSUPPORTED;
  const int nc = (H / 8 + 63) / 64;
  const dim3 grid(static_cast<unsigned>((T + 3) / 4)), block(256);
  if (nc <= 2) {
    MOE_LAUNCH("add_rms_norm", add_rms_norm_kernel<2>, grid, block, 0, stream, a, b, w, eps, T, H, sum_out, normed);
  } else if (nc <= 4) {
    MOE_LAUNCH("add_rms_norm", add_rms_norm_kernel<4>, grid, block, 0, stream, a, b, w, eps, T, H, sum_out, normed);
  } else if (nc <= 8) {
    MOE_LAUNCH("add_rms_norm", add_rms_norm_kernel<8>, grid, block, 0, stream, a, b, w, eps, T, H, sum_out, normed);
  } else {
    MOE_LAUNCH("add_rms_norm", add_rms_norm_kernel<16>, grid, block, 0, stream, a, b, w, eps, T, H, sum_out, normed);
  }
  return launch_status("add_rms_norm");
}

}  // namespace moe
