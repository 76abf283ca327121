// gather_mm.hip -- grouped dense (bf16) matmul, the gather_mm that
// SwitchLinear runs for experts that are not quantized (reference
// src/common/switch_layers.cpp:103-109), gfx950.
//
// Rows are the expert buckets of the sorted pairs, as in the quantized
// kernels (qmm.hip).  A workgroup of four waves takes one expert slot and 64
// output columns, wave w the columns 16w .. 16w + 15, over the whole bucket in
// chunks of 32 rows: two 16x16 tiles of v_mfma_f32_16x16x32_bf16 per wave and
// 32-wide K step, the loads of up to kMmSteps K steps of a wave issued before
// their MFMAs.  fp32 accumulation, one bf16 rounding (and SwitchLinear's
// bias, switch_layers.cpp:111-114, on the rounded value).
#include "internal.hpp"

namespace moe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct GMArgs {
  const uint16_t* x;       // input rows [*, K] bf16
  const int32_t* row_in;   // sorted position -> input row
  const int32_t* row_out;  // sorted position -> output row
  const int32_t* active;   // [slots][4] slot records {expert, first sorted row, rows, 0}
  const uint16_t* w;       // [E, N, K] bf16
  const uint16_t* lb;      // [E, N] bf16 or NULL
  int N, K, ntiles;
  uint16_t* out;           // [*, N] bf16
};

constexpr int kMmSteps = 8;

__global__ __launch_bounds__(256) void grouped_mm_kernel(GMArgs a) {
  const int slot = blockIdx.x / a.ntiles, nt = blockIdx.x - slot * a.ntiles;
  const int4 rec = reinterpret_cast<const int4*>(a.active)[slot];
  const int e = rec.x, beg = rec.y, cnt = rec.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = nt * 64 + 16 * wave;
  if (cnt <= 0 || n0 >= a.N) return;  // wave-uniform; the kernel has no barrier
  const int i = lane & 15, g = lane >> 4;
  // B operand: weight row n0 + i (a partial last tile re-reads row N - 1), K slots 8g .. 8g + 7
  const uint16_t* bp = a.w + (static_cast<int64_t>(e) * a.N + min(n0 + i, a.N - 1)) * a.K + 8 * g;
  const int steps = a.K / 32;
  const int col = n0 + i;
  for (int tc = 0; tc < cnt; tc += 32) {
    // A operands: rows tc + i and tc + 16 + i of the bucket (clamped to its last row, never stored)
    const uint16_t* ap0 = a.x + static_cast<int64_t>(a.row_in[beg + min(tc + i, cnt - 1)]) * a.K + 8 * g;
    const uint16_t* ap1 = a.x + static_cast<int64_t>(a.row_in[beg + min(tc + 16 + i, cnt - 1)]) * a.K + 8 * g;
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < steps; s0 += kMmSteps) {
      u32x4 av0[kMmSteps], av1[kMmSteps], bv[kMmSteps];
#pragma unroll
      for (int j = 0; j < kMmSteps; ++j) {
        const int s = min(s0 + j, steps - 1);
        av0[j] = *reinterpret_cast<const u32x4*>(ap0 + 32 * s);
        av1[j] = *reinterpret_cast<const u32x4*>(ap1 + 32 * s);
        bv[j] = *reinterpret_cast<const u32x4*>(bp + 32 * s);
      }
#pragma unroll
      for (int j = 0; j < kMmSteps; ++j) {
        if (s0 + j >= steps) break;
        const bf16x8 b = __builtin_bit_cast(bf16x8, bv[j]);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av0[j]), b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av1[j]), b, acc1, 0, 0, 0);
      }
    }
    if (col >= a.N) continue;
    const float bias = a.lb ? bf2f(a.lb[static_cast<int64_t>(e) * a.N + col]) : 0.0f;
    // D layout of the 16x16 MFMA: row (bucket row) 4g + r, column (output) i.
    // Every output row index is loaded before the first store, so no store
    // waits for the one before it (loads and stores share one counter)
    int64_t orow[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = beg + min(tc + 16 * t + 4 * g + r, cnt - 1);
        orow[t][r] = a.row_out ? a.row_out[pos] : pos;
      }
    wait_vmcnt<0>();  // (the compiler would otherwise wait for everything before each conditional store)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = tc + 16 * t + 4 * g + r;
        if (m >= cnt) continue;
        const float v = t ? acc1[r] : acc0[r];
        a.out[orow[t][r] * a.N + col] = f2bf(a.lb ? bfr(v) + bias : v);
      }
  }
}

}  // namespace

int grouped_mm(const uint16_t* x, const int32_t* row_in, const int32_t* row_out, const int32_t* active, int slots,
               const uint16_t* w, const uint16_t* linear_bias, int N, int K, uint16_t* out, hipStream_t stream) {
  if (!x || !row_in || !active || !w || !out || slots < 0 || N <= 0 || K <= 0) return MOE_E_INVALID_ARG;
  if (K % 32 != 0 || (reinterpret_cast<uintptr_t>(x) & 15u) || (reinterpret_cast<uintptr_t>(w) & 15u))
    return MOE_E_UNSUPPORTED;
  if (slots == 0) return MOE_OK;
  const int ntiles = (N + 63) / 64;
  const int64_t wgs = static_cast<int64_t>(slots) * ntiles;
  if (wgs > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  GMArgs a{x, row_in, row_out, active, w, linear_bias, N, K, ntiles, out};
  MOE_LAUNCH("gather_mm", grouped_mm_kernel, dim3(static_cast<unsigned>(wgs)), dim3(256), 0, stream, a);
  return launch_status("gather_mm");
}

}  // namespace moe
