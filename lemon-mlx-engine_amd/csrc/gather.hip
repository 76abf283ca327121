// gather.hip -- row gather and per-expert bias add (gfx950).
//
// take_rows: dst row i = src row rows[i] / divisor, the data movement of the
//   reference's gather_sort (take(x_flat, order // k)) and scatter_unsort
//   (take(y, inv_order, 0)), src/common/switch_layers.cpp:17-46.  One wave per
//   destination row, 16-byte accesses when the row size and both base
//   pointers allow it, else 2-byte accesses.
// add_expert_bias: out[b, m, :] = bf16(out[b, m, :] + bias[rhs[b], :]), the
//   linear bias of SwitchLinear (switch_layers.cpp:111-114).
#include "internal.hpp"

namespace moe {
namespace {

template <typename U>
__global__ __launch_bounds__(256) void take_rows_kernel(const U* __restrict__ src, int64_t src_rows,
                                                        const int32_t* __restrict__ rows, int64_t n,
                                                        int32_t divisor, int64_t units,
                                                        U* __restrict__ dst) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (i >= n) return;
  const int lane = threadIdx.x & 63;
  const int64_t r = rows[i];
  const int64_t s = r >= 0 ? r / divisor : -1;
  U* d = dst + i * units;
  if (s < 0 || s >= src_rows) {
    // an index outside the source leaves a zero row (never an out-of-bounds read)
    for (int64_t c = lane; c < units; c += 64) d[c] = U{};
    return;
  }
  const U* p = src + s * units;
  for (int64_t c = lane; c < units; c += 64) d[c] = p[c];
}

__global__ __launch_bounds__(256) void add_expert_bias_kernel(uint16_t* __restrict__ out,
                                                              const uint16_t* __restrict__ bias,
                                                              const uint32_t* __restrict__ rhs,
                                                              int64_t rows, int M, int N, int E) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint32_t e = rhs[row / M];
  if (e >= static_cast<uint32_t>(E)) return;
  const uint16_t* b = bias + static_cast<int64_t>(e) * N;
  uint16_t* o = out + row * N;
  for (int c = threadIdx.x & 63; c < N; c += 64) o[c] = f2bf(bf2f(o[c]) + bf2f(b[c]));
}

}  // namespace

int take_rows(const void* src, int64_t src_rows, const int32_t* rows, int64_t n, int32_t divisor,
              int64_t row_bytes, void* dst, hipStream_t stream) {
  if (n < 0 || src_rows < 0 || divisor <= 0 || row_bytes < 0 || row_bytes % 2 != 0)
    return MOE_E_INVALID_ARG;
  if (n == 0 || row_bytes == 0) return MOE_OK;
  if (!src || !rows || !dst) return MOE_E_INVALID_ARG;
  if ((n + 3) / 4 > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>((n + 3) / 4));
  const bool wide = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(src) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(dst) & 15u) == 0;
  if (wide) {
    MOE_LAUNCH("take_rows", take_rows_kernel<uint4>, grid, dim3(256), 0, stream,
               static_cast<const uint4*>(src), src_rows, rows, n, divisor, row_bytes / 16,
               static_cast<uint4*>(dst));
  } else {
    MOE_LAUNCH("take_rows", take_rows_kernel<uint16_t>, grid, dim3(256), 0, stream,
               static_cast<const uint16_t*>(src), src_rows, rows, n, divisor, row_bytes / 2,
               static_cast<uint16_t*>(dst));
  }
  MOE_CHECK_LAUNCH("take_rows");
  return MOE_OK;
}

int add_expert_bias(uint16_t* out, const uint16_t* bias, const uint32_t* rhs, int64_t batch, int32_t M,
                    int32_t N, int32_t E, hipStream_t stream) {
  if (batch < 0 || M <= 0 || N <= 0 || E <= 0) return MOE_E_INVALID_ARG;
  if (batch == 0) return MOE_OK;
  if (!out || !bias || !rhs) return MOE_E_INVALID_ARG;
  const int64_t rows = batch * M;
  if ((rows + 3) / 4 > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  MOE_LAUNCH("add_expert_bias", add_expert_bias_kernel, dim3(static_cast<unsigned>((rows + 3) / 4)),
             dim3(256), 0, stream, out, bias, rhs, rows, M, N, E);
  MOE_CHECK_LAUNCH("add_expert_bias");
  return MOE_OK;
}

}  // namespace moe
