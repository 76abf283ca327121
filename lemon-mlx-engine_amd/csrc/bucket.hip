// bucket.hip -- stable bucketing of (token, expert) pairs by expert id.
//
// Output positions follow the counting-sort definition: pair i (flat index
// t*k + j) of expert e goes to offsets[e] + #{i' < i : inds[i'] == e}.  That is
// exactly a stable argsort of the flat indices (reference gather_sort,
// src/common/switch_layers.cpp:17-30), computed with integer counts only, so
// it is bit-exact and deterministic.
//
// Small P (decode): one workgroup does histogram, scan and scatter.
// Large P (prefill): per-chunk histograms, then per-chunk scatter workgroups
// that each scan the chunk-count table themselves (E <= 512 and a table of at
// most 32768 entries; beyond that one scan workgroup between the two
// launches).  Within a chunk, ranks of equal experts are resolved with wave64
// ballots (a match over the bits of the expert id) plus per-wave counts in LDS,
// processed in pair order so the result is stable.

#include "bucket_impl.hpp"

namespace moe {

namespace {

constexpr int kChunk = 512;         // pairs per chunk (multi-block path)
// chunk-count tables up to this many entries are scanned from LDS
constexpr int kScanStagedMax = 16384;
// scan + scatter in one launch (bucket_scan_scatter_kernel): chunks of 1024
// pairs, E <= 512, a chunk-count table of at most this many entries (each
// workgroup reads all of it)
constexpr int kFusedChunk = 1024;
constexpr int kScanScatterMaxE = 512;
constexpr int64_t kScanScatterMaxTable = 32768;

template <int NW>
__global__ __launch_bounds__(NW * 64) void bucket_fused_kernel(const uint32_t* __restrict__ inds,
                                                              int64_t P, int E, int k, int nbits,
                                                              BucketOut o) {
  extern __shared__ int lds[];
  bucket_fused_body<NW>(inds, P, E, k, nbits, o, lds);
}

__global__ __launch_bounds__(256) void bucket_count_kernel(const uint32_t* __restrict__ inds,
                                                          int64_t P, int E,
                                                          int* __restrict__ cnt, int chunk) {
  extern __shared__ int hist[];
  for (int x = threadIdx.x; x < E; x += 256) hist[x] = 0;
  __syncthreads();
  const int64_t b0 = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t b1 = b0 + chunk < P ? b0 + chunk : P;
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

// Scan and scatter in one launch: workgroup b forms the per-expert totals,
// the offsets and the starting positions of chunk b itself from the
// chunk-count table cnt [nblk][E] (thread (part, e) sums chunks
// [part*L, part*L + L) of expert e, those before chunk b apart; integer sums,
// so the order does not matter), then scatters chunk b.  Workgroup 0 also
// writes offsets, the slot records and the token-tile table.  The positions
// are those of bucket_scan_kernel + bucket_scatter_kernel.  1024 threads,
// E <= kScanScatterMaxE; lds: 2048 + 2E + 1 + 18 + 16E ints.
__global__ __launch_bounds__(1024) void bucket_scan_scatter_kernel(const uint32_t* __restrict__ inds, int64_t P,
                                                                  int E, int k, int nbits,
                                                                  const int* __restrict__ cnt, int nblk,
                                                                  BucketOut o) {
  extern __shared__ int lds[];
  int* ptot = lds;              // [parts][E]: partial totals
  int* ppre = ptot + 1024;      // [parts][E]: partial counts before chunk b (row 0: the sums)
  int* tot = ppre + 1024;       // [E]
  int* running = tot + E;       // [E+1]
  int* tmp = running + E + 1;   // [16 + 2]
  int* wcnt = tmp + 18;         // [16][E]
  const int b = blockIdx.x;
  const int parts = 1024 / E;
  const int L = (nblk + parts - 1) / parts;
  const int e = threadIdx.x % E, part = threadIdx.x / E;
  if (part < parts) {
    const int b0 = part * L, b1 = min(nblk, b0 + L);
    int st = 0, sp = 0;
#pragma unroll 8
    for (int bb = b0; bb < b1; ++bb) {
      const int c = cnt[static_cast<int64_t>(bb) * E + e];
      st += c;
      sp += bb < b ? c : 0;
    }
    ptot[part * E + e] = st;
    ppre[part * E + e] = sp;
  }
  for (int x = threadIdx.x; x < 16 * E; x += 1024) wcnt[x] = 0;
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += 1024) {  // (thread x alone touches column x)
    int t = 0, q = 0;
    for (int pp = 0; pp < parts; ++pp) {
      t += ptot[pp * E + x];
      q += ppre[pp * E + x];
    }
    tot[x] = t;
    ppre[x] = q;
  }
  __syncthreads();
  // offsets (every workgroup, into running); the outputs from workgroup 0
  BucketOut head = o;
  if (b != 0) {
    head.offsets = nullptr;
    head.active = nullptr;
    head.num_active = nullptr;
    head.tiles = nullptr;
  }
  finish_offsets<1024>(tot, E, running, tmp, head);
  for (int x = threadIdx.x; x < E; x += 1024) running[x] += ppre[x];
  __syncthreads();
  const int64_t c0 = static_cast<int64_t>(b) * kFusedChunk;
  const int64_t c1 = c0 + kFusedChunk < P ? c0 + kFusedChunk : P;
  scatter_subchunk<16>(inds, c1, c0, E, k, nbits, running, wcnt, o);
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
  const int64_t nblk_f = (P + kFusedChunk - 1) / kFusedChunk;
  if (E <= kScanScatterMaxE && nblk_f * E <= kScanScatterMaxTable) {
    // (the table of 1024-pair chunks is at most half the workspace's 512-pair one)
    const int nb = static_cast<int>(nblk_f);
    MOE_LAUNCH("bucket_count", bucket_count_kernel, dim3(nb), dim3(256), sizeof(int) * E, stream, inds, P, E, cnt,
               kFusedChunk);
    MOE_CHECK_LAUNCH("bucket_count");
    MOE_LAUNCH("bucket_scatter", bucket_scan_scatter_kernel, dim3(nb), dim3(1024),
               sizeof(int) * (2048 + 2 * E + 1 + 18 + 16 * E), stream, inds, P, E, k, nbits, cnt, nb, o);
    MOE_CHECK_LAUNCH("bucket_scatter");
    return MOE_OK;
  }
  const int nblk = static_cast<int>((P + kChunk - 1) / kChunk);
  MOE_LAUNCH("bucket_count", bucket_count_kernel, dim3(nblk), dim3(256), sizeof(int) * E, stream, inds, P,
                     E, cnt, kChunk);
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
