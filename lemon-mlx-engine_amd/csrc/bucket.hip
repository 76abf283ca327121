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

#include "internal.hpp"

namespace moe {

namespace {

constexpr int kChunk = 2048;        // pairs per chunk (multi-block path)
constexpr int kFusedMaxP = 16384;   // single-workgroup path up to this many pairs

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return (l == 0) ? 0ull : (~0ull >> (64 - l));
}

// Mask of lanes holding the same key (keys < 2^nbits).
__device__ __forceinline__ uint64_t match_key(uint32_t key, int nbits) {
  uint64_t peers = ~0ull;
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (key >> b) & 1u;
    const uint64_t m = __ballot(bit);
    peers &= bit ? m : ~m;
  }
  return peers;
}

// Block-wide exclusive scan of one int per thread (NT threads), returns the
// exclusive prefix; *total receives the sum.  Uses `tmp` [NT/64] LDS.
template <int NT>
__device__ int block_exclusive_scan(int v, int* tmp, int* total) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < NT / 64; ++w) {
      const int c = tmp[w];
      tmp[w] = run;
      run += c;
    }
    tmp[NT / 64] = run;
  }
  __syncthreads();
  const int excl = tmp[wave] + incl - v;
  *total = tmp[NT / 64];
  __syncthreads();
  return excl;
}

// Scatter one sub-chunk of NW*64 consecutive pairs starting at `first`,
// given running[e] = next free position of expert e.  wcnt is [NW][E] LDS,
// all zero on entry and on exit.
template <int NW>
__device__ void scatter_subchunk(const uint32_t* inds, int64_t P, int64_t first, int E, int k,
                                 int nbits, int* running, int* wcnt, const BucketOut& o) {
  const int wave = threadIdx.x >> 6;
  const int64_t i = first + threadIdx.x;
  uint32_t e = static_cast<uint32_t>(E);  // sentinel for "no pair"
  if (i < P) {
    const uint32_t v = inds[i];
    if (v < static_cast<uint32_t>(E)) e = v;
  }
  const uint64_t peers = match_key(e, nbits);
  const int rank = __popcll(peers & lanemask_lt());
  const bool leader = (peers & lanemask_lt()) == 0;
  const bool valid = e < static_cast<uint32_t>(E);
  if (valid && leader) wcnt[wave * E + e] = __popcll(peers);
  __syncthreads();
  if (valid) {
    int pos = running[e] + rank;
    for (int w = 0; w < wave; ++w) pos += wcnt[w * E + e];
    if (o.perm) o.perm[pos] = static_cast<int32_t>(i);
    if (o.inv_perm) o.inv_perm[i] = pos;
    if (o.sorted_expert) o.sorted_expert[pos] = e;
    if (o.sorted_token) o.sorted_token[pos] = static_cast<int32_t>(i / k);
  }
  __syncthreads();
  for (int x = threadIdx.x; x < E; x += NW * 64) {
    int s = 0;
    for (int w = 0; w < NW; ++w) {
      s += wcnt[w * E + x];
      wcnt[w * E + x] = 0;
    }
    running[x] += s;
  }
  __syncthreads();
}

// Writes offsets (and the active-expert list) from per-expert totals held in
// `tot` (LDS [E]); offs_lds [E+1] receives the offsets.  Requires E <= NT.
template <int NT>
__device__ void finish_offsets(const int* tot, int E, int* offs_lds, int* tmp, const BucketOut& o) {
  const int e = threadIdx.x;
  const int c = e < E ? tot[e] : 0;
  int total;
  const int ex = block_exclusive_scan<NT>(c, tmp, &total);
  if (e < E) offs_lds[e] = ex;
  if (e == 0) offs_lds[E] = total;
  __syncthreads();
  if (o.offsets)
    for (int x = threadIdx.x; x <= E; x += NT) o.offsets[x] = offs_lds[x];
  if (o.active) {
    // one 16-byte record per slot, so a GEMM workgroup finds its expert and
    // rows with a single load; slots past the count get rows = 0
    const int nz = (e < E && c > 0) ? 1 : 0;
    int na;
    const int ax = block_exclusive_scan<NT>(nz, tmp, &na);
    int4* rec = reinterpret_cast<int4*>(o.active);
    if (nz) rec[ax] = make_int4(e, ex, c, 0);
    if (e < E && e >= na) rec[e] = make_int4(0, 0, 0, 0);
    if (threadIdx.x == 0 && o.num_active) o.num_active[0] = na;
  }
}

template <int NW>
__global__ __launch_bounds__(NW * 64) void bucket_fused_kernel(const uint32_t* __restrict__ inds,
                                                              int64_t P, int E, int k, int nbits,
                                                              BucketOut o) {
  extern __shared__ int lds[];
  int* tot = lds;                   // [E]
  int* running = tot + E;           // [E+1]
  int* wcnt = running + E + 1;      // [NW][E]
  int* tmp = wcnt + NW * E;         // [NW + 2]
  for (int x = threadIdx.x; x < E; x += NW * 64) tot[x] = 0;
  for (int x = threadIdx.x; x < NW * E; x += NW * 64) wcnt[x] = 0;
  __syncthreads();
  for (int64_t i = threadIdx.x; i < P; i += NW * 64) {
    const uint32_t v = inds[i];
    if (v < static_cast<uint32_t>(E)) atomicAdd(&tot[v], 1);
  }
  __syncthreads();
  finish_offsets<NW * 64>(tot, E, running, tmp, o);
  for (int64_t first = 0; first < P; first += NW * 64)
    scatter_subchunk<NW>(inds, P, first, E, k, nbits, running, wcnt, o);
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
// whole [nblk][E] table is first read into LDS by every thread (coalesced),
// so the per-expert passes run over LDS instead of strided global loads.
template <bool STAGED>
__global__ __launch_bounds__(1024) void bucket_scan_kernel(int* __restrict__ cnt, int nblk, int E,
                                                          BucketOut o) {
  extern __shared__ int lds[];
  int* tot = lds;           // [E]
  int* offs = tot + E;      // [E+1]
  int* tmp = offs + E + 1;  // [16 + 2]
  int* tab = tmp + 18;      // [nblk * E] (STAGED)
  const int n = nblk * E;
  if constexpr (STAGED) {
    for (int i = threadIdx.x; i < n; i += 1024) tab[i] = cnt[i];
    __syncthreads();
  }
  const int* src = STAGED ? tab : cnt;
  for (int e = threadIdx.x; e < E; e += 1024) {
    int s = 0;
    for (int b = 0; b < nblk; ++b) s += src[b * E + e];
    tot[e] = s;
  }
  __syncthreads();
  finish_offsets<1024>(tot, E, offs, tmp, o);
  for (int e = threadIdx.x; e < E; e += 1024) {
    int run = offs[e];
    for (int b = 0; b < nblk; ++b) {
      const int c = src[b * E + e];
      cnt[static_cast<int64_t>(b) * E + e] = run;
      run += c;
    }
  }
}

// chunk-count tables up to this many entries are scanned from LDS
constexpr int kScanStagedMax = 12288;

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

int bits_for(int E) {
  int n = 0;
  while ((1 << n) <= E) ++n;  // keys 0..E (E = sentinel)
  return n;
}

}  // namespace

size_t bucket_workspace_bytes(int64_t P, int E) {
  if (P <= kFusedMaxP && E <= 512) return 0;
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
  if (P <= kFusedMaxP && E <= 512) {
    constexpr int NW = 16;
    const size_t lds = sizeof(int) * (E + (E + 1) + NW * E + NW + 2);
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
               sizeof(int) * (2 * E + 1 + 18 + nblk * E), stream, cnt, nblk, E, o);
  else
    MOE_LAUNCH("bucket_scan", bucket_scan_kernel<false>, dim3(1), dim3(1024), sizeof(int) * (2 * E + 1 + 18),
               stream, cnt, nblk, E, o);
  MOE_CHECK_LAUNCH("bucket_scan");
  MOE_LAUNCH("bucket_scatter", bucket_scatter_kernel, dim3(nblk), dim3(256), sizeof(int) * 5 * E, stream,
                     inds, P, E, k, nbits, cnt, o);
  MOE_CHECK_LAUNCH("bucket_scatter");
  return MOE_OK;
}

}  // namespace moe
