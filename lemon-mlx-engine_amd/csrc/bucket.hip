// bucket.hip -- stable bucketing of (token, expert) pairs by expert id.
//
// Output positions follow the counting-sort definition: pair i (flat index
// t*k + j) of expert e goes to offsets[e] + #{i' < i : inds[i'] == e}.  That is
// exactly a stable argsort of the flat indices (reference gather_sort,
// src/common/switch_layers.cpp:17-30), computed with integer counts only, so
// it is bit-exact and deterministic.
//
// Small P (decode): one workgroup does histogram, scan and scatter.
// Large P (prefill): per-chunk histograms, one scan workgroup, per-chunk
// scatter.  Within a chunk, ranks of equal experts are resolved with wave64
// ballots (a match over the bits of the expert id) plus per-wave counts in LDS,
// processed in pair order so the result is stable.

#include "bucket_impl.hpp"

namespace moe {

namespace {

constexpr int kChunk = 512;         // pairs per chunk (multi-block path)
// chunk-count tables up to this many entries are scanned from LDS
constexpr int kScanStagedMax = 16384;

template <int NW>
__global__ __launch_bounds__(NW * 64) void bucket_fused_kernel(const uint32_t* __restrict__ inds,
                                                              int64_t P, int E, int k, int nbits,
                                                              BucketOut o) {
  extern __shared__ int lds[];
  bucket_fused_body<NW>(inds, P, E, k, nbits, o, lds);
}

__global__ __launch_bounds__(256) void bucket_count_kernel(const uint32_t* __restrict__ inds,
                                                          int64_t P, int E,
                                                          int* __restrict__ cnt) {
  extern __shared__ int hist[];
  for (int x = threadIdx.x; x < E; x += 256) hist[x] = 0;
  __syncthreads();
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t b1 = b0 + kChunk < P ? b0 + kChunk : P;
  for (int64_t i = b0 + threadIdx.x; i < b1; i += 256) {
    const uint32_t v = inds[i];
    if (v < static_cast<uint32_t>(E)) atomicAdd(&hist[v], 1);
  }
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += 256) cnt[static_cast<int64_t>(blockIdx.x) * E + x] = hist[x];
}

// cnt[b][e] -> start position of chunk b's pairs of expert e.  STAGED: the
// whole [nblk][E] table is first read into LDS (coalesced).  The column scans
// (over chunks, per expert) are split over all 1024 threads: thread (part, e)
// sums chunks [part*L, part*L + L) of expert e, the PARTS partial sums of an
// expert are scanned through LDS, and each thread writes its range's starts.
template <bool STAGED>
__global__ __launch_bounds__(1024) void bucket_scan_kernel(int* __restrict__ cnt, int nblk, int E,
                                                          BucketOut o) {
  extern __shared__ int lds[];
  int* tot = lds;           // [E]
  int* offs = tot + E;      // [E+1]
  int* tmp = offs + E + 1;  // [16 + 2]
  int* psum = tmp + 18;     // [1024]: partial sums, [part][E]
  int* tab = psum + 1024;   // [nblk * E] (STAGED)
  const int n = nblk * E;
  if constexpr (STAGED) {  // every load of a thread in flight before its LDS stores
    constexpr int kU = kScanStagedMax / 1024;
    int v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = threadIdx.x + 1024 * u < n ? cnt[threadIdx.x + 1024 * u] : 0;
#pragma unroll
    for (int u = 0; u < kU; ++u)
      if (threadIdx.x + 1024 * u < n) tab[threadIdx.x + 1024 * u] = v[u];
  }
  const int* src = STAGED ? tab : cnt;
  const int parts = 1024 / E;  // E <= 1024
  const int L = (nblk + parts - 1) / parts;
  const int e = threadIdx.x % E, part = threadIdx.x / E;
  const bool mine = part < parts;
  const int b0 = part * L, b1 = min(nblk, b0 + L);
  if constexpr (STAGED) __syncthreads();
  int s = 0;
  if (mine)
#pragma unroll 8
    for (int b = b0; b < b1; ++b) s += src[b * E + e];
  if (mine) psum[part * E + e] = s;
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += 1024) {
    int t = 0;
    for (int q = 0; q < parts; ++q) t += psum[q * E + x];
    tot[x] = t;
  }
  __syncthreads();
  finish_offsets<1024>(tot, E, offs, tmp, o);
  if (mine) {
    int run = offs[e];
    for (int q = 0; q < part; ++q) run += psum[q * E + e];
#pragma unroll 8
    for (int b = b0; b < b1; ++b) {
      const int c = src[b * E + e];
      cnt[static_cast<int64_t>(b) * E + e] = run;
      run += c;
    }
  }
}

__global__ __launch_bounds__(256) void bucket_scatter_kernel(const uint32_t* __restrict__ inds,
                                                            int64_t P, int E, int k, int nbits,
                                                            const int* __restrict__ base,
                                                            BucketOut o) {
  extern __shared__ int lds[];
  int* running = lds;         // [E]
  int* wcnt = running + E;    // [4][E]
  for (int x = threadIdx.x; x < E; x += 256) running[x] = base[static_cast<int64_t>(blockIdx.x) * E + x];
  for (int x = threadIdx.x; x < 4 * E; x += 256) wcnt[x] = 0;
  __syncthreads();
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * kChunk;
  const int64_t b1 = b0 + kChunk < P ? b0 + kChunk : P;
  for (int64_t first = b0; first < b1; first += 256)
    scatter_subchunk<4>(inds, b1, first, E, k, nbits, running, wcnt, o);
}


}  // namespace

size_t bucket_workspace_bytes(int64_t P, int E) {
  if (P <= kFusedMaxP && E <= kFusedMaxE) return 0;
  const int64_t nblk = (P + kChunk - 1) / kChunk;
  return static_cast<size_t>(nblk) * E * sizeof(int);
}

int bucket(const uint32_t* inds, int64_t T, int k, int E, const BucketOut& o, void* ws,
           size_t ws_bytes, hipStream_t stream) {
  if (T < 0 || k <= 0 || E <= 0 || E > 1024) return E > 1024 ? MOE_E_UNSUPPORTED : MOE_E_INVALID_ARG;
  if (!o.offsets) return MOE_E_INVALID_ARG;
  const int64_t P = T * k;
  if (P > 0 && !inds) return MOE_E_INVALID_ARG;
  if (P > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  const int nbits = bits_for(E);
  if (P <= kFusedMaxP && E <= kFusedMaxE) {
    constexpr int NW = 16;
    const size_t lds = sizeof(int) * bucket_fused_lds_ints<NW>(E);
    MOE_LAUNCH("bucket_fused", bucket_fused_kernel<NW>, dim3(1), dim3(NW * 64), lds, stream, inds, P, E,
                       k, nbits, o);
    MOE_CHECK_LAUNCH("bucket_fused");
    return MOE_OK;
  }
  const size_t need = bucket_workspace_bytes(P, E);
  if (!ws || ws_bytes < need) return MOE_E_WORKSPACE;
  int* cnt = static_cast<int*>(ws);
  const int nblk = static_cast<int>((P + kChunk - 1) / kChunk);
  MOE_LAUNCH("bucket_count", bucket_count_kernel, dim3(nblk), dim3(256), sizeof(int) * E, stream, inds, P,
                     E, cnt);
  MOE_CHECK_LAUNCH("bucket_count");
  if (static_cast<int64_t>(nblk) * E <= kScanStagedMax)
    MOE_LAUNCH("bucket_scan", bucket_scan_kernel<true>, dim3(1), dim3(1024),
               sizeof(int) * (2 * E + 1 + 18 + 1024 + nblk * E), stream, cnt, nblk, E, o);
  else
    MOE_LAUNCH("bucket_scan", bucket_scan_kernel<false>, dim3(1), dim3(1024), sizeof(int) * (2 * E + 1 + 18 + 1024),
               stream, cnt, nblk, E, o);
  MOE_CHECK_LAUNCH("bucket_scan");
  MOE_LAUNCH("bucket_scatter", bucket_scatter_kernel, dim3(nblk), dim3(256), sizeof(int) * 5 * E, stream,
                     inds, P, E, k, nbits, cnt, o);
  MOE_CHECK_LAUNCH("bucket_scatter");
  return MOE_OK;
}

}  // namespace moe
