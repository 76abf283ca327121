// bucket_impl.hpp -- device code of the stable (token, expert) bucketing,
// shared by the bucketing kernels (bucket.hip) and the fused route + bucket
// kernel of small batches (router.hip).
//
// Output positions follow the counting-sort definition: pair i (flat index
// t*k + j) of expert e goes to offsets[e] + #{i' < i : inds[i'] == e}.  That is
// exactly a stable argsort of the flat indices (reference gather_sort,
// src/common/switch_layers.cpp:17-30), computed with integer counts only, so
// it is bit-exact and deterministic.
#pragma once

#include "internal.hpp"

namespace moe {
namespace {

constexpr int kFusedMaxP = 4096;    // single-workgroup path up to this many pairs
constexpr int kFusedMaxE = 512;

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
  // wave inclusive scan on DPP: shifts of 1, 2, 4, 8 within each row of 16
  // (lanes without a source add 0), then row 15's total into the next row
  // and lane 31's into rows 2 and 3
  int incl = v;
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xf, 0xf, true);  // row_shr:1
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xf, 0xf, true);  // row_shr:2
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xf, 0xf, true);  // row_shr:4
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xf, 0xf, true);  // row_shr:8
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  incl += __builtin_amdgcn_update_dpp(0, incl, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
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
  if (o.tiles) {  // the large-bucket GEMM's token-tile table
    int c4 = 0, c3 = 0, c2 = 0, c1 = 0;
    if (e < E) tile_counts(c, c4, c3, c2, c1);
    int n4, n3, n2, n1;
    const int b4 = block_exclusive_scan<NT>(c4, tmp, &n4);
    const int b3 = block_exclusive_scan<NT>(c3, tmp, &n3);
    const int b2 = block_exclusive_scan<NT>(c2, tmp, &n2);
    const int b1 = block_exclusive_scan<NT>(c1, tmp, &n1);
    if (threadIdx.x == 0) reinterpret_cast<int4*>(o.tiles)[0] = make_int4(n4, n3, n2, n1);
    if (e < E) write_tiles(o.tiles, e, ex, c, c4, c3, c2, c1, b4, b3, b2, b1, n4, n3, n2);
  }
}

// LDS ints of the single-workgroup bucketing with NW waves
template <int NW>
constexpr size_t bucket_fused_lds_ints(int E) {
  return static_cast<size_t>(E + (E + 1) + NW * E + NW + 2);
}

// Histogram, scan and scatter of P pairs by one workgroup of NW waves (E <=
// kFusedMaxE); lds: bucket_fused_lds_ints<NW>(E) ints.  Every thread of the
// workgroup calls it.
template <int NW>
__device__ void bucket_fused_body(const uint32_t* __restrict__ inds, int64_t P, int E, int k, int nbits,
                                  const BucketOut& o, int* lds) {
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

// Orders this wave's LDS accesses: its earlier LDS reads and writes complete
// (from every lane) before later ones, and the compiler keeps them in order.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
}

// Wave-wide exclusive prefix sum of one int per lane; *total gets the sum.
__device__ __forceinline__ int wave_exclusive_scan(int v, int* total) {
  const int lane = lane_id();
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  *total = __shfl(incl, 63, 64);
  return incl - v;
}

// The stable bucketing of a small batch (P <= kSmallMaxP pairs, E <= 512)
// by one wave with no workgroup barrier: histogram by LDS atomics, the
// exclusive scan over the experts (lane l owns experts V*l .. V*l + V - 1),
// then the scatter 64 pairs at a time, each pair's position its expert's
// running offset plus its rank among the chunk's pairs of the same expert.
// Same outputs as bucket_fused_body except the token-tile table.  inds: LDS
// [P]; cnt, offs: LDS [E + 1] each.  Only the calling wave may touch them.
constexpr int kSmallMaxP = 256;
[[maybe_unused]] __device__ void bucket_small_wave(const uint32_t* inds, int P, int E, int k, int nbits, const BucketOut& o,
                                  int* cnt, int* offs) {
  const int lane = lane_id();
  for (int x = lane; x <= E; x += 64) cnt[x] = 0;
  wave_lds_sync();
  for (int i = lane; i < P; i += 64) {
    const uint32_t v = inds[i];
    if (v < static_cast<uint32_t>(E)) atomicAdd(&cnt[v], 1);
  }
  wave_lds_sync();
  const int V = (E + 63) >> 6;
  int c[8];
  int sum = 0, nzc = 0;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const int e = V * lane + v;
    c[v] = v < V && e < E ? cnt[e] : 0;
    sum += c[v];
    nzc += c[v] > 0 ? 1 : 0;
  }
  int total, nact;
  int run = wave_exclusive_scan(sum, &total);
  int slot = wave_exclusive_scan(nzc, &nact);
  int4* rec = reinterpret_cast<int4*>(o.active);
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const int e = V * lane + v;
    if (v < V && e < E) {
      offs[e] = run;
      if (o.offsets) o.offsets[e] = run;
      if (rec && c[v] > 0) rec[slot++] = make_int4(e, run, c[v], 0);
      run += c[v];
    }
  }
  if (lane == 0) {
    offs[E] = total;
    if (o.offsets) o.offsets[E] = total;
    if (o.num_active) o.num_active[0] = nact;
  }
  if (rec)
    for (int x = nact + lane; x < E; x += 64) rec[x] = make_int4(0, 0, 0, 0);
  wave_lds_sync();
  for (int first = 0; first < P; first += 64) {
    const int i = first + lane;
    uint32_t e = static_cast<uint32_t>(E);  // sentinel for "no pair"
    if (i < P) {
      const uint32_t v = inds[i];
      if (v < static_cast<uint32_t>(E)) e = v;
    }
    const uint64_t peers = match_key(e, nbits);
    const uint64_t below = peers & lanemask_lt();
    const bool valid = e < static_cast<uint32_t>(E);
    const int base = valid ? offs[e] : 0;
    if (valid) {
      const int pos = base + __popcll(below);
      if (o.perm) o.perm[pos] = i;
      if (o.inv_perm) o.inv_perm[i] = pos;
      if (o.sorted_expert) o.sorted_expert[pos] = e;
      if (o.sorted_token) o.sorted_token[pos] = i / k;
    }
    wave_lds_sync();
    if (valid && below == 0) offs[e] = base + __popcll(peers);
    wave_lds_sync();
  }
}

int bits_for(int E) {
  int n = 0;
  while ((1 << n) <= E) ++n;  // keys 0..E (E = sentinel)
  return n;
}

}  // namespace
}  // namespace moe
