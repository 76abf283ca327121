// router.hip -- router projection and per-token scoring / top-k (gfx950).
//
// moe_router_logits: logits = bf16(x . Wg^T) on bf16 MFMA (16x16x32), fp32
//   accumulation, K split over the four waves of a workgroup.
// moe_route: one wave64 per token.  Lane l holds experts l, l+64, l+128, ...
//   in registers; the softmax denominator is 64 strided partials reduced by an
//   xor butterfly (the canonical order the CPU checker restates), top-k is k
//   rounds of a wave argmax with the canonical (value desc, index asc) order.
#pragma clang fp contract(off)

#include "bucket_impl.hpp"
#include "route_impl.hpp"

namespace moe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// C[M, N] = A[M, K] . B[N, K]^T (+ bias[N], one rounding), bf16 in / bf16
// out, for few rows (decode).
// One workgroup = one 16x16 output tile; its NW waves take interleaved
// 32-wide K steps, issuing the loads of up to 8 steps before their MFMAs
// (rows past M or N read a clamped, valid row and are never stored), and are
// summed through LDS in wave order.  Ap (optional): the workgroups of the
// first column tile also write A's rows in pair K order.
template <int NW>
__global__ __launch_bounds__(NW * 64) void gemm_nt_bf16_tile16(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ B,
                                                              const uint16_t* __restrict__ bias,
                                                              uint16_t* __restrict__ C, int M, int N, int K,
                                                              uint16_t* __restrict__ Ap) {
  __shared__ float red[NW][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * 16;
  const int i = lane & 15, g = lane >> 4;
  const uint16_t* ap = A + static_cast<int64_t>(min(m0 + i, M - 1)) * K + 8 * g;
  const uint16_t* bp = B + static_cast<int64_t>(min(n0 + i, N - 1)) * K + 8 * g;
  const int steps = K / 32;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = wave; s0 < steps; s0 += 8 * NW) {
    u32x4 av[8], bv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int s = min(s0 + j * NW, steps - 1);
      av[j] = *reinterpret_cast<const u32x4*>(ap + 32 * s);
      bv[j] = *reinterpret_cast<const u32x4*>(bp + 32 * s);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j * NW < steps)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[j]),
                                                      __builtin_bit_cast(bf16x8, bv[j]), acc, 0, 0, 0);
    if (Ap && n0 == 0 && m0 + i < M) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j * NW < steps)
          *reinterpret_cast<u32x4*>(Ap + static_cast<int64_t>(m0 + i) * K + 32 * (s0 + j * NW) + 8 * g) =
              to_pair_order(av[j]);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][lane * 4 + r] = acc[r];
  __syncthreads();
  if (wave == 0) {
    // D layout of 16x16 MFMA: column = lane%16, row = 4*(lane/16) + r; the
    // column's bias is loaded once (before the stores, which could alias it)
    const int col = n0 + i;
    const float bv = bias && col < N ? bf2f(bias[col]) : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = red[0][lane * 4 + r];
#pragma unroll
      for (int w = 1; w < NW; ++w) v = v + red[w][lane * 4 + r];
      const int row = m0 + 4 * g + r;
      if (row < M && col < N) C[static_cast<int64_t>(row) * N + col] = f2bf(bias ? v + bv : v);
    }
  }
}

// Router projection of a small batch (T <= kRouterPartialMaxT) as fp32 partial
// sums over KS slices of H, spread over many workgroups so that the router
// weight streams from HBM through many CUs at once: workgroup (tile, ks, tt)
// computes the 16-expert tile `tile` over H range [ks*H/KS, (ks+1)*H/KS) for
// the 16-token tile tt (MFMA rows past T read row T-1 and are never stored),
// its four waves taking interleaved 32-wide steps with every load of a wave
// issued before its MFMAs.  part[ks][t][e] is summed in ks order by
// route_bucket_small_kernel.  The workgroups of expert tile 0 also write x in
// pair K order (xp).
// NORM: x is the RMSNorm of a + b (NormIn), formed here -- the step before
// the block in the same launch.  Each wave first loads the leading chunks of
// its first token row, then its one batch (a, b and norm-weight chunks and
// the router rows of its steps), and finds the scales of the workgroup's rows
// (one wave per row, add_rms_norm_kernel's lane order and arithmetic, so each
// scale is bit-identical to that kernel's) while the batch is in flight; it
// then builds every 8-value operand chunk as that kernel does (bf16(a + b),
// times the scale, times the weight).  The workgroups of expert tile 0 also
// write the chunks of sum_out and of normed, the block's input.
constexpr int kNormRowChunks = 16;  // 16-byte chunks of a row per lane: H <= 8192 (add_rms_norm's limit)
constexpr int kPartialBatch = 8;    // 32-wide steps per wave per batch of loads
template <bool NORM>
__global__ __launch_bounds__(256) void router_partial_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ wg,
                                                             float* __restrict__ part, int T, int E, int H,
                                                             uint16_t* __restrict__ xp, NormIn nin) {
  constexpr int kMaxSteps = kPartialBatch;
  __shared__ float red[4][256];
  __shared__ float rscale[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tile = blockIdx.x, ks = blockIdx.y, KS = gridDim.y, m0 = 16 * blockIdx.z;
  const int n0 = tile * 16, i = lane & 15, g = lane >> 4;
  const int span = H / KS, k0 = ks * span;
  const int arow = min(m0 + i, T - 1);  // this lane's operand row (rows past T repeat row T - 1)
  const int64_t aoff = static_cast<int64_t>(arow) * H + k0 + 8 * g;
  const uint16_t* bp = wg + static_cast<int64_t>(min(n0 + i, E - 1)) * H + k0 + 8 * g;
  const int steps = span / 32;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const bool writer = tile == 0 && m0 + i < T;  // expert tile 0 writes the row's chunks of its K slice
  if constexpr (NORM) {
    // one batch per wave (the host keeps steps <= 4 * kMaxSteps), in straight
    // code so that each wait covers only what it needs
    const int s0 = wave;
    const int nch = H >> 3;
    const bool own_row = m0 + wave < T;  // (wave-uniform)
    const int64_t frow = min(m0 + wave, T - 1);
    u32x4 ra0[4], rb0[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int ch = min(lane + 64 * c, nch - 1);
      ra0[c] = reinterpret_cast<const u32x4*>(nin.a + frow * H)[ch];
      rb0[c] = reinterpret_cast<const u32x4*>(nin.b + frow * H)[ch];
    }
    u32x4 va[kMaxSteps], vb[kMaxSteps], vw[kMaxSteps], bv[kMaxSteps];
#pragma unroll
    for (int j = 0; j < kMaxSteps; ++j) {
      const int st = min(s0 + 4 * j, steps - 1);
      va[j] = *reinterpret_cast<const u32x4*>(nin.a + aoff + 32 * st);
      vb[j] = *reinterpret_cast<const u32x4*>(nin.b + aoff + 32 * st);
      vw[j] = *reinterpret_cast<const u32x4*>(nin.w + k0 + 8 * g + 32 * st);
      bv[j] = *reinterpret_cast<const u32x4*>(bp + 32 * st);
    }
    // sum of squares over chunks c0 .. c0+3 of a row, in add_rms_norm_kernel's
    // order (a chunk past the row was loaded clamped and is not added)
    auto add_group = [&](const u32x4(&ra)[4], const u32x4(&rb)[4], int c0, float ss) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (lane + 64 * (c0 + c) < nch) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float t0 = __uint_as_float(ra[c][q] << 16) + __uint_as_float(rb[c][q] << 16);
            const float t1 = __uint_as_float(ra[c][q] & 0xffff0000u) + __uint_as_float(rb[c][q] & 0xffff0000u);
            ss = fmaf(t0, t0, ss);
            ss = fmaf(t1, t1, ss);
          }
        }
      }
      return ss;
    };
    // the rest of row `row` from chunk group cstart on, then its scale
    auto row_scale = [&](int64_t row, int cstart, float ss) {
      for (int c0 = cstart; c0 < kNormRowChunks && 64 * c0 < nch; c0 += 4) {
        u32x4 ra[4], rb[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int ch = min(lane + 64 * (c0 + c), nch - 1);
          ra[c] = reinterpret_cast<const u32x4*>(nin.a + row * H)[ch];
          rb[c] = reinterpret_cast<const u32x4*>(nin.b + row * H)[ch];
        }
        ss = add_group(ra, rb, c0, ss);
      }
      ss = wave_sum(ss);
      return 1.0f / sqrtf(ss / static_cast<float>(H) + nin.eps);
    };
    if (own_row) {
      const float sc = row_scale(frow, 4, add_group(ra0, rb0, 0, 0.0f));
      if (lane == 0) rscale[wave] = sc;
    }
    for (int r = wave + 4; r < 16 && m0 + r < T; r += 4) {  // (wave-uniform)
      const float sc = row_scale(m0 + r, 0, 0.0f);
      if (lane == 0) rscale[r] = sc;
    }
    __syncthreads();
    const float ascale = rscale[arow - m0];
#pragma unroll
    for (int j = 0; j < kMaxSteps; ++j) {
      if (s0 + 4 * j < steps) {  // (wave-uniform)
        u32x4 sv, av;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float t0 = __uint_as_float(va[j][q] << 16) + __uint_as_float(vb[j][q] << 16);
          const float t1 = __uint_as_float(va[j][q] & 0xffff0000u) + __uint_as_float(vb[j][q] & 0xffff0000u);
          sv[q] = pack_bf16x2(t0, t1);
          av[q] = pack_bf16x2(__uint_as_float(sv[q] << 16) * ascale * __uint_as_float(vw[j][q] << 16),
                              __uint_as_float(sv[q] & 0xffff0000u) * ascale * __uint_as_float(vw[j][q] & 0xffff0000u));
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv[j]),
                                                      acc, 0, 0, 0);
        if (writer) {
          const int64_t o = static_cast<int64_t>(m0 + i) * H + k0 + 32 * (s0 + 4 * j) + 8 * g;
          *reinterpret_cast<u32x4*>(nin.sum_out + o) = sv;
          *reinterpret_cast<u32x4*>(nin.normed + o) = av;
          if (xp) *reinterpret_cast<u32x4*>(xp + o) = to_pair_order(av);
        }
      }
    }
  } else {
    const uint16_t* ap = x + aoff;
    for (int s0 = wave; s0 < steps; s0 += 4 * kMaxSteps) {
      u32x4 av[kMaxSteps], bv[kMaxSteps];
#pragma unroll
      for (int j = 0; j < kMaxSteps; ++j) {
        const int st = min(s0 + 4 * j, steps - 1);
        av[j] = *reinterpret_cast<const u32x4*>(ap + 32 * st);
        bv[j] = *reinterpret_cast<const u32x4*>(bp + 32 * st);
      }
#pragma unroll
      for (int j = 0; j < kMaxSteps; ++j)
        if (s0 + 4 * j < steps)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[j]),
                                                        __builtin_bit_cast(bf16x8, bv[j]), acc, 0, 0, 0);
      if (xp && writer) {
#pragma unroll
        for (int j = 0; j < kMaxSteps; ++j)
          if (s0 + 4 * j < steps)
            *reinterpret_cast<u32x4*>(xp + static_cast<int64_t>(m0 + i) * H + k0 + 32 * (s0 + 4 * j) + 8 * g) =
                to_pair_order(av[j]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) red[wave][lane * 4 + r] = acc[r];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = ((red[0][lane * 4 + r] + red[1][lane * 4 + r]) + red[2][lane * 4 + r]) + red[3][lane * 4 + r];
      // D layout of 16x16 MFMA: column (expert) = lane%16, row (token) = 4*(lane/16) + r
      const int row = m0 + 4 * g + r, col = n0 + i;
      if (row < T && col < E) part[(static_cast<int64_t>(ks) * T + row) * E + col] = v;
    }
  }
}

// Router projection for many tokens (prefill), optionally with the group sums
// of x that the large-bucket expert GEMM consumes.  One workgroup = 32 tokens x
// 128 experts; wave w owns experts 32w..32w+31 over the whole of K, on the
// 32x32x16 bf16 MFMA.  Each 64-wide K step (128 bytes per row) of the token and
// expert rows is staged in LDS by direct-to-LDS loads, 8 lanes per row (whole
// 128-byte lines), the 16-byte chunk c of row r at slot c ^ (r & 7), in a ring
// of kRStages steps.  A lane (row r = lane%32, half h = lane/32) feeds MFMA i
// with chunk 4h + i of its token row and of its expert row: one permutation of
// the step's k for A and B, so the dot products are unchanged.
struct RouterGemmArgs {
  const uint16_t* x;
  const uint16_t* wg;
  const uint16_t* bias;  // [E] or NULL, added before the one rounding
  uint16_t* out;
  int T, E, H;
  // group sums (xhl != nullptr): xhl[t] in 16-group chunks [hi(16) | lo(16)],
  // groups of gs along H, groups G..16*nch-1 zero (the layout the expert GEMM
  // reads)
  uint16_t* xhl;
  int gs, nch;
  // optional: x in pair K order, written from the staged token rows by the
  // workgroups of the first expert block
  uint16_t* xp;
  // K split over gridDim.z workgroups (> 1): fp32 partial sums [KS][T][E]
  // (no bias) instead of out; workgroup ks takes K steps [ks S, (ks+1) S)
  float* part;
};

constexpr int kRStages = 4;
constexpr int kRABytes = 32 * 128;                 // token rows of one step
constexpr int kRStageBytes = kRABytes + 128 * 128;  // + expert rows
constexpr int kRLoads = 5;                          // DMA instructions per wave per step

__global__ __launch_bounds__(256) void router_gemm_tile32(RouterGemmArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kRStages * kRStageBytes];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.x * 32, nb = blockIdx.y * 128;
  const int ks = blockIdx.z;
  const int S = a.H / 64 / gridDim.z, s0 = ks * S;  // this workgroup's K steps: s0 .. s0 + S - 1

  // producer: lane -> row 8*blk + lane/8, slot lane%8 (global chunk slot ^ (row & 7));
  // rows past T or E read a clamped, valid row and are never stored
  const int prow = lane >> 3, pslot = lane & 7;
  const int ar = 8 * wave + prow;
  const uint8_t* asrc = reinterpret_cast<const uint8_t*>(a.x + static_cast<int64_t>(min(m0 + ar, a.T - 1)) * a.H) +
                        128 * s0 + 16 * (pslot ^ (ar & 7));
  const uint8_t* bsrc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int br = 32 * wave + 8 * j + prow;
    bsrc[j] = reinterpret_cast<const uint8_t*>(a.wg + static_cast<int64_t>(min(nb + br, a.E - 1)) * a.H) +
              128 * s0 + 16 * (pslot ^ (br & 7));
  }
  auto issue = [&](int s, int st) {
    s = min(s, S - 1);  // past the end: re-read the last step (in bounds, never consumed)
    uint8_t* sb = lds + st * kRStageBytes;
    load_lds16(asrc + 128 * s, sb + wave * 1024);
#pragma unroll
    for (int j = 0; j < 4; ++j) load_lds16(bsrc[j] + 128 * s, sb + kRABytes + (32 * wave + 8 * j) * 128);
  };
  // consumer offsets within a stage
  int aoff[4], boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    aoff[i] = r * 128 + 16 * ((4 * h + i) ^ (r & 7));
    boff[i] = kRABytes + (32 * wave + r) * 128 + 16 * ((4 * h + i) ^ (r & 7));
  }
  // the first expert block's workgroups also copy x in pair order and take
  // its group sums, both from the staged token rows: thread (row t/8, unit
  // t%8) reads one 16-byte unit per step, sums its 8 values as a tree, and
  // the row's 8 lanes add theirs on DPP (every wave does an equal share; the
  // sums on one wave's MFMA operands held that wave ~8 us longer at T = 8192)
  const bool sums = a.xhl != nullptr && blockIdx.y == 0;
  const bool copy = sums || (a.xp != nullptr && blockIdx.y == 0);
  const int spg = a.gs / 64;  // steps per group
  const int crow = threadIdx.x >> 3, cu = threadIdx.x & 7;

  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  float gsum = 0.0f, gmine = 0.0f;

#pragma unroll
  for (int i = 0; i < kRStages - 1; ++i) issue(i, i);
  for (int s = 0; s < S; ++s) {
    wait_vmcnt<(kRStages - 2) * kRLoads>();  // this wave's loads of step s landed
    lds_barrier();                           // every wave's did; step s-1's stage is free
    issue(s + kRStages - 1, (s + kRStages - 1) % kRStages);
    const uint8_t* sb = lds + (s % kRStages) * kRStageBytes;
    if (copy) {  // step s of the 32 token rows, one 16-byte unit per thread
      const u32x4 v = *reinterpret_cast<const u32x4*>(sb + crow * 128 + 16 * (cu ^ (crow & 7)));
      if (a.xp && m0 + crow < a.T)
        *reinterpret_cast<u32x4*>(a.xp + static_cast<int64_t>(m0 + crow) * a.H + 64 * (s0 + s) + 8 * cu) =
            to_pair_order(v);
      if (sums) {
        float p[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = __uint_as_float(v[q] << 16) + __uint_as_float(v[q] & 0xffff0000u);
        float su = (p[0] + p[1]) + (p[2] + p[3]);
        // the row's 8 units (lanes 8*(row%8) .. +7): every lane ends with the same value
        su += dpp_f<kDppQuadXor1>(su);
        su += dpp_f<kDppQuadXor2>(su);
        su += dpp_f<kDppHalfMirror>(su);
        gsum += su;
        if ((s + 1) % spg == 0) {
          // lane cu keeps the sum of the group gi with gi % 8 == cu; after every
          // 8 groups (and at the slice's last one) the row's 8 lanes store 8
          // consecutive bf16 of the hi half and of the lo half (one store
          // instruction each per 8 groups instead of two per group)
          const int gi = (s0 + s) / spg;  // (s0 is a multiple of spg: the host checks)
          gmine = (gi & 7) == cu ? gsum : gmine;
          gsum = 0.0f;
          if ((gi & 7) == 7 || s == S - 1) {
            const int g = (gi & ~7) + cu;  // groups of this slice only: [s0 / spg, gi]
            if (m0 + crow < a.T && g <= gi && g >= s0 / spg) {
              const uint16_t hi = f2bf(gmine), lo = f2bf(gmine - bf2f(hi));
              uint16_t* c = a.xhl + static_cast<int64_t>(m0 + crow) * a.nch * 32 + (g >> 4) * 32 + (g & 15);
              c[0] = hi;
              c[16] = lo;
            }
          }
        }
      }
    }
    u32x4 fa[4], fb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[i] = *reinterpret_cast<const u32x4*>(sb + aoff[i]);
      fb[i] = *reinterpret_cast<const u32x4*>(sb + boff[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[i]),
                                                    __builtin_bit_cast(bf16x8, fb[i]), acc, 0, 0, 0);
  }
  wait_vmcnt<0>();  // no DMA write into LDS outstanding when the workgroup ends

  // D layout of 32x32 MFMA: column (expert) = lane%32, row (token) =
  // 8*(j/4) + 4*(lane/32) + j%4 for accumulator j
  const int e = nb + 32 * wave + r;
  if (a.part) {  // partial sums of this K slice, summed with the bias by the routing
    if (e < a.E) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int t = m0 + 8 * (j >> 2) + 4 * h + (j & 3);
        if (t < a.T) a.part[(static_cast<int64_t>(ks) * a.T + t) * a.E + e] = acc[j];
      }
    }
  } else if (e < a.E) {
    const float bv = a.bias ? bf2f(a.bias[e]) : 0.0f;  // once, before the stores (which could alias it)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int t = m0 + 8 * (j >> 2) + 4 * h + (j & 3);
      if (t < a.T) a.out[static_cast<int64_t>(t) * a.E + e] = f2bf(a.bias ? acc[j] + bv : acc[j]);
    }
  }
  if (sums && wave == 0 && ks == 0 && h == 0 && m0 + r < a.T) {
    uint16_t* row = a.xhl + static_cast<int64_t>(m0 + r) * a.nch * 32;
    for (int gi = a.H / a.gs; gi < 16 * a.nch; ++gi)
#pragma unroll
      for (int q = 0; q < 2; ++q) row[(gi >> 4) * 32 + 16 * q + (gi & 15)] = 0;
  }
}

template <int VPL>
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= a.T) return;
  route_token<VPL>(a, t, threadIdx.x & 63);
}

// The same from the router's partial sums part [KS][T][E]: the wave of token
// t forms its logits (slice order, the router bias rbias or none before the
// one rounding; written to logits_out [T][E]) in registers, then routes.
template <int VPL>
__global__ __launch_bounds__(256) void route_partial_kernel(RouteArgs a, const float* __restrict__ part, int KS,
                                                            const uint16_t* __restrict__ rbias,
                                                            uint16_t* __restrict__ logits_out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= a.T) return;
  const int lane = threadIdx.x & 63;
  float lv[VPL];
  token_logits_from_partials<VPL>(part + t * a.E, KS, a.T * a.E, a.E, rbias, lane, lv, logits_out + t * a.E);
  route_token_lv<VPL>(a, t, lane, lv);
}

// Small batches: routing and bucketing in one workgroup of NW waves (wave w
// routes tokens w, w + NW, ...; the bucketing then reads the routed experts
// the workgroup just wrote), one launch and no round trip between them.
template <int VPL, int NW>
__global__ __launch_bounds__(NW * 64) void route_bucket_kernel(RouteArgs a, int nbits, BucketOut o) {
  extern __shared__ int lds[];
  // the selected experts also go to LDS (after the bucketing's ints), so the
  // bucketing reads them without a round trip through L2
  uint32_t* inds_lds = reinterpret_cast<uint32_t*>(lds + bucket_fused_lds_ints<NW>(a.E));
  for (int64_t t = threadIdx.x >> 6; t < a.T; t += NW) route_token<VPL>(a, t, threadIdx.x & 63, inds_lds);
  __syncthreads();  // every token's experts are written
  bucket_fused_body<NW>(inds_lds, a.T * a.k, a.E, a.k, nbits, o, lds);
}

constexpr int kPartialMaxFloats = 1 << 16;  // the router's partial sums, at most 256 KB (router_partial_ks)

// threads of route_bucket_small_kernel for T tokens
__host__ __device__ constexpr int route_small_threads(int64_t T) {
  return 64 * (T <= 4 ? 4 : T <= 8 ? 8 : 16);
}

// dynamic LDS of route_bucket_small_kernel: counts and offsets over E + 1
// experts, the T*k expert indices, the T x E bf16 logits
size_t route_small_lds(int64_t T, int E, int k) {
  return sizeof(int) * (2 * (static_cast<size_t>(E) + 1) + static_cast<size_t>(T) * k) +
         sizeof(uint16_t) * static_cast<size_t>(T) * E;
}
constexpr size_t kRouteSmallMaxLds = 64 << 10;  // without raising the kernel's dynamic-LDS limit

// Small batches (T <= kRouteSmallMaxT, T*k <= kSmallMaxP, E <= 512, no
// token-tile table): one workgroup of NW >= max(T, 4) waves.  The logits are
// formed first -- from the router's partial sums (part != NULL: KS slices, a
// power of two, summed in slice order by the thread that owns the logit,
// every load of a thread issued before the first sum; the router bias rbias
// (or NULL) added before the one rounding to bf16; also written to
// logits_out) or read from a.logits -- into LDS; wave w routes token w; then
// one wave buckets the T*k pairs (T = 1: the routing wave itself, from its
// registers), so no workgroup barrier runs after the routing.  (Measured at
// T = 64, 16 waves routing 4 tokens each and one wave bucketing 512 pairs:
// 29.7 µs against 13.4 for the route and bucket launches.)
template <int VPL, int NW>
__global__ __launch_bounds__(NW * 64) void route_bucket_small_kernel(RouteArgs a, const float* __restrict__ part,
                                                                     int KS, const uint16_t* __restrict__ rbias,
                                                                     uint16_t* __restrict__ logits_out,
                                                                     int nbits, BucketOut o) {
  static_assert(NW >= 4, "route_small_threads");
  constexpr int NT = NW * 64;
  extern __shared__ int lds[];
  const int T = static_cast<int>(a.T), E = a.E, k = a.k;
  int* cnt = lds;                                                       // [E + 1]
  int* offs = cnt + E + 1;                                              // [E + 1]
  uint32_t* inds_lds = reinterpret_cast<uint32_t*>(offs + E + 1);       // [T * k]
  uint16_t* lg = reinterpret_cast<uint16_t*>(inds_lds + T * k);         // [T * E]
  const int n = T * E;
  if (part) {
    logits_from_partials<NT>(part, KS, n, E, rbias, lg, logits_out);
  } else {
    for (int x = threadIdx.x; x < n; x += NT) lg[x] = a.logits[x];
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (T == 1) {  // one token: routed and bucketed by wave 0 from its registers
    if (wave == 0) bucket_one_token(route_token<VPL>(a, 0, lane, nullptr, lg), k, E, o);
    return;
  }
  if (wave < T) route_token<VPL>(a, wave, lane, inds_lds, lg + wave * E);
  __syncthreads();
  if (wave == 0) bucket_small_wave(inds_lds, T * k, E, k, nbits, o, cnt, offs);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool router_tile32(int64_t T, int32_t H) { return T >= kRouterTile32MinT && H % 64 == 0; }

int router_logits(const uint16_t* x, const uint16_t* wg, const uint16_t* bias, int64_t T, int32_t H, int32_t E,
                  uint16_t* logits, hipStream_t stream, const RouterGroupSums* sums, uint16_t* xp) {
  if (!x || !wg || !logits || T < 0 || H <= 0 || E <= 0) return MOE_E_INVALID_ARG;
  if (H % 32 != 0 || !aligned16(x) || !aligned16(wg)) return MOE_E_UNSUPPORTED;
  if (T == 0) return MOE_OK;
  if (T > 0x7fffffffLL - 32) return MOE_E_UNSUPPORTED;
  if (router_tile32(T, H)) {
    RouterGemmArgs a{x, wg, bias, logits, static_cast<int>(T), E, H, nullptr, 64, 0, xp, nullptr};
    if (sums) {
      if (sums->gs % 64 != 0 || H % sums->gs != 0 || sums->nch * 16 < H / sums->gs) return MOE_E_INVALID_ARG;
      a.xhl = sums->xhl;
      a.gs = sums->gs;
      a.nch = sums->nch;
    }
    dim3 grid(static_cast<unsigned>((T + 31) / 32), (E + 127) / 128);
    MOE_LAUNCH("router_logits", router_gemm_tile32, grid, dim3(256), 0, stream, a);
  } else {
    if (sums) return MOE_E_INVALID_ARG;  // group sums come with the many-token kernel only
    dim3 grid((E + 15) / 16, static_cast<unsigned>((T + 15) / 16));
    MOE_LAUNCH("router_logits", gemm_nt_bf16_tile16<8>, grid, dim3(512), 0, stream, x, wg, bias, logits,
               static_cast<int>(T), E, H, xp);
  }
  MOE_CHECK_LAUNCH("router_logits");
  return MOE_OK;
}

// K slices of the many-token projection (router_partials_tile32): two where
// the grid is at most one workgroup per CU (the kernel's 80 KB of LDS lets two
// share a CU), K is at least 64 steps and each slice is whole groups of the
// group sums' size.  Measured (same box, T = 8192 / 4096, projection + routing
// from the partials against the one-slice projection + routing from logits):
// Mixtral-8x7B (H 4096) 65.3 -> 56.4 us, DeepSeek-V3 (H 7168) 118.6 -> 102.1
// us, Qwen3-30B-A3B (H 2048) 45.8 -> 46.3 us (so H 2048 keeps one slice).
constexpr int64_t kTile32OneRound = 256;  // workgroups that fill the MI355X's CUs once
constexpr int kTile32MinSteps = 64;
int router_tile32_ks(int64_t T, int32_t E, int32_t H, int gs) {
  if (!router_tile32(T, H) || gs < 64 || gs % 64 != 0) return 1;
  const int64_t wgs = (T + 31) / 32 * ((E + 127) / 128);
  const int steps = H / 64;
  if (wgs > kTile32OneRound || steps < kTile32MinSteps || steps % 2 != 0 || (steps / 2) % (gs / 64) != 0) return 1;
  return 2;
}

int router_partials_tile32(const uint16_t* x, const uint16_t* wg, int64_t T, int32_t H, int32_t E, float* part,
                           int ks, const RouterGroupSums* sums, uint16_t* xp, hipStream_t stream) {
  if (!x || !wg || !part || ks < 2 || T < 1 || E <= 0 || !router_tile32(T, H)) return MOE_E_INVALID_ARG;
  if (!aligned16(x) || !aligned16(wg) || (xp && !aligned16(xp))) return MOE_E_UNSUPPORTED;
  if (T > 0x7fffffffLL - 32 || (H / 64) % ks != 0) return MOE_E_UNSUPPORTED;
  RouterGemmArgs a{x, wg, nullptr, nullptr, static_cast<int>(T), E, H, nullptr, 64, 0, xp, part};
  if (sums) {
    if (sums->gs % 64 != 0 || H % sums->gs != 0 || sums->nch * 16 < H / sums->gs) return MOE_E_INVALID_ARG;
    if ((H / 64 / ks) % (sums->gs / 64) != 0) return MOE_E_UNSUPPORTED;  // each slice holds whole groups
    a.xhl = sums->xhl;
    a.gs = sums->gs;
    a.nch = sums->nch;
  }
  dim3 grid(static_cast<unsigned>((T + 31) / 32), (E + 127) / 128, ks);
  MOE_LAUNCH("router_logits", router_gemm_tile32, grid, dim3(256), 0, stream, a);
  MOE_CHECK_LAUNCH("router_partials_tile32");
  return MOE_OK;
}

int route_validate(const moe_router_params* p) {
  if (!p) return MOE_E_INVALID_ARG;
  const int E = p->num_experts, k = p->top_k;
  if (E <= 0 || k <= 0 || k > E) return MOE_E_INVALID_ARG;
  if (E > 1024 || k > 16) return MOE_E_UNSUPPORTED;
  switch (p->variant) {
    case MOE_ROUTE_TOPK_LOGITS:
    case MOE_ROUTE_TOPK_PROBS:
    case MOE_ROUTE_SOFTMAX_TOPK:
    case MOE_ROUTE_SIGMOID:
      return MOE_OK;
    case MOE_ROUTE_SIGMOID_CORRECTED:
    case MOE_ROUTE_GLM4_SIGMOID:
    case MOE_ROUTE_GLM4_SOFTMAX:
      return MOE_OK;  // their group scores are not applied
    case MOE_ROUTE_LFM2:
      return MOE_OK;  // (the expert bias is optional)
    case MOE_ROUTE_SIGMOID_GROUP:
    case MOE_ROUTE_SIGMOID_GROUP_DROP_BEST:
      if (p->n_group <= 1) return MOE_OK;
      if (p->n_group > 64 || E % p->n_group != 0 || E / p->n_group < 2) return MOE_E_UNSUPPORTED;
      if (p->topk_group < 1 || p->topk_group > p->n_group) return MOE_E_INVALID_ARG;
      return MOE_OK;
    default:
      return MOE_E_INVALID_ARG;
  }
}

int route(const uint16_t* logits, const float* bias, int64_t T, const moe_router_params* p,
          uint32_t* inds, float* scores, hipStream_t stream) {
  int st = route_validate(p);
  if (st != MOE_OK) return st;
  if (!logits || !inds || !scores || T < 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if ((T + 3) / 4 > 0x7fffffff) return MOE_E_UNSUPPORTED;
  RouteArgs a{logits, bias, inds, scores, T, p->num_experts, p->top_k, p->variant,
              p->norm_topk_prob, p->n_group, p->topk_group, p->routed_scaling_factor};
  dim3 grid(static_cast<unsigned>((T + 3) / 4));
  const int vpl = (p->num_experts + 63) / 64;
  if (vpl <= 1)
    MOE_LAUNCH("route", route_kernel<1>, grid, dim3(256), 0, stream, a);
  else if (vpl <= 2)
    MOE_LAUNCH("route", route_kernel<2>, grid, dim3(256), 0, stream, a);
  else if (vpl <= 4)
    MOE_LAUNCH("route", route_kernel<4>, grid, dim3(256), 0, stream, a);
  else if (vpl <= 8)
    MOE_LAUNCH("route", route_kernel<8>, grid, dim3(256), 0, stream, a);
  else
    MOE_LAUNCH("route", route_kernel<16>, grid, dim3(256), 0, stream, a);
  MOE_CHECK_LAUNCH("route");
  return MOE_OK;
}

int router_partial_ks(int64_t T, int32_t E, int32_t H) {
  if (T < 1 || T > kRouterPartialMaxT || H % 128 != 0 || E <= 0) return 0;
  const int tiles = (E + 15) / 16, units = H / 128;
  int ks = 1;
  // the most slices (a power of two) that keep <= 128 workgroups per 16-token
  // tile, <= 256 KB of partials and the loads of the consumer in registers:
  // route_bucket_small <= kPartialLoads per thread, route_from_partials
  // <= 32 per lane (slices x candidates per lane)
  const int64_t per_thread = T <= kRouteSmallMaxT
                                 ? (T * E + route_small_threads(T) - 1) / route_small_threads(T)
                                 : (E + 63) / 64;
  for (int c = 1; c <= units; c *= 2)
    if (units % c == 0 && tiles * c <= 128 && c * T * E <= kPartialMaxFloats && c * per_thread <= kPartialLoads)
      ks = c;
  return ks;
}

bool route_from_partials_fits_any(const moe_router_params* p) { return p && p->num_experts <= kFusedMaxE; }

bool route_from_partials_fits(int64_t T, const moe_router_params* p) {
  return p && T > kRouteSmallMaxT && T <= kRouterPartialMaxT && p->num_experts <= kFusedMaxE;
}

int route_from_partials(const float* part, int ks, const uint16_t* rbias, uint16_t* logits_out, const float* bias,
                        int64_t T, const moe_router_params* p, uint32_t* inds, float* scores, hipStream_t stream,
                        bool any_t) {
  int st = route_validate(p);
  if (st != MOE_OK) return st;
  if (!part || !logits_out || !inds || !scores || T < 1) return MOE_E_INVALID_ARG;
  if (any_t ? (p->num_experts > kFusedMaxE || (T + 3) / 4 > 0x7fffffffLL) : !route_from_partials_fits(T, p))
    return MOE_E_UNSUPPORTED;
  const int vpl = (p->num_experts + 63) / 64;
  if (ks < 1 || ks * (vpl <= 1 ? 1 : vpl <= 2 ? 2 : vpl <= 4 ? 4 : 8) > 32) return MOE_E_INVALID_ARG;
  RouteArgs a{logits_out, bias, inds, scores, T, p->num_experts, p->top_k, p->variant,
              p->norm_topk_prob, p->n_group, p->topk_group, p->routed_scaling_factor};
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  if (vpl <= 1)
    MOE_LAUNCH("route", route_partial_kernel<1>, grid, dim3(256), 0, stream, a, part, ks, rbias, logits_out);
  else if (vpl <= 2)
    MOE_LAUNCH("route", route_partial_kernel<2>, grid, dim3(256), 0, stream, a, part, ks, rbias, logits_out);
  else if (vpl <= 4)
    MOE_LAUNCH("route", route_partial_kernel<4>, grid, dim3(256), 0, stream, a, part, ks, rbias, logits_out);
  else
    MOE_LAUNCH("route", route_partial_kernel<8>, grid, dim3(256), 0, stream, a, part, ks, rbias, logits_out);
  MOE_CHECK_LAUNCH("route_from_partials");
  return MOE_OK;
}

int router_partials(const uint16_t* x, const uint16_t* wg, int64_t T, int32_t H, int32_t E, float* part, int ks,
                    uint16_t* xp, hipStream_t stream) {
  if (!x || !wg || !part || ks < 1 || T < 1 || T > kRouterPartialMaxT || H % (128 * ks) != 0) return MOE_E_INVALID_ARG;
  if (!aligned16(x) || !aligned16(wg) || (xp && !aligned16(xp))) return MOE_E_UNSUPPORTED;
  MOE_LAUNCH("router_logits", router_partial_kernel<false>,
             dim3((E + 15) / 16, ks, static_cast<unsigned>((T + 15) / 16)), dim3(256), 0, stream, x, wg, part,
             static_cast<int>(T), E, H, xp, NormIn{});
  MOE_CHECK_LAUNCH("router_partials");
  return MOE_OK;
}

bool router_partials_norm_fits(int64_t T, int32_t H, int ks) {
  // one batch per wave: a K slice of at most 4 * kPartialBatch steps of 32
  return T >= 1 && T <= kNormFuseMaxT && H % 8 == 0 && H <= 64 * 8 * kNormRowChunks && ks >= 1 &&
         H / ks <= 4 * kPartialBatch * 32;
}

int router_partials_norm(const NormIn& nin, const uint16_t* wg, int64_t T, int32_t H, int32_t E, float* part,
                         int ks, uint16_t* xp, hipStream_t stream) {
  if (!nin.a || !nin.b || !nin.w || !nin.sum_out || !nin.normed || !(nin.eps >= 0.0f) || !wg || !part || ks < 1 ||
      T < 1 || H % (128 * ks) != 0)
    return MOE_E_INVALID_ARG;
  if (!router_partials_norm_fits(T, H, ks)) return MOE_E_UNSUPPORTED;
  for (const void* p : {static_cast<const void*>(nin.a), static_cast<const void*>(nin.b),
                        static_cast<const void*>(nin.w), static_cast<const void*>(nin.sum_out),
                        static_cast<const void*>(nin.normed), static_cast<const void*>(wg)})
    if (!aligned16(p)) return MOE_E_UNSUPPORTED;
  if (xp && !aligned16(xp)) return MOE_E_UNSUPPORTED;
  MOE_LAUNCH("router_logits", router_partial_kernel<true>,
             dim3((E + 15) / 16, ks, static_cast<unsigned>((T + 15) / 16)), dim3(256), 0, stream, nullptr, wg, part,
             static_cast<int>(T), E, H, xp, nin);
  MOE_CHECK_LAUNCH("router_partials_norm");
  return MOE_OK;
}

bool route_bucket_small_fits(int64_t T, const moe_router_params* p, const BucketOut& o) {
  return p && T >= 1 && T <= kRouteSmallMaxT && p->num_experts <= kFusedMaxE && T * p->top_k <= kSmallMaxP &&
         route_small_lds(T, p->num_experts, p->top_k) <= kRouteSmallMaxLds && !o.tiles;
}

template <int NW>
static int launch_route_small(const RouteArgs& a, const float* part, int ks, const uint16_t* rbias,
                              uint16_t* logits_out, int nbits, const BucketOut& o, size_t lds, hipStream_t stream) {
  const int vpl = (a.E + 63) / 64;
  if (vpl <= 1)
    MOE_LAUNCH("route_bucket", (route_bucket_small_kernel<1, NW>), dim3(1), dim3(NW * 64), lds, stream, a, part, ks,
               rbias, logits_out, nbits, o);
  else if (vpl <= 2)
    MOE_LAUNCH("route_bucket", (route_bucket_small_kernel<2, NW>), dim3(1), dim3(NW * 64), lds, stream, a, part, ks,
               rbias, logits_out, nbits, o);
  else if (vpl <= 4)
    MOE_LAUNCH("route_bucket", (route_bucket_small_kernel<4, NW>), dim3(1), dim3(NW * 64), lds, stream, a, part, ks,
               rbias, logits_out, nbits, o);
  else
    MOE_LAUNCH("route_bucket", (route_bucket_small_kernel<8, NW>), dim3(1), dim3(NW * 64), lds, stream, a, part, ks,
               rbias, logits_out, nbits, o);
  return launch_status("route_bucket_small");
}

int route_bucket_small(const uint16_t* logits, const float* part, int ks, const uint16_t* rbias,
                       uint16_t* logits_out, const float* bias, int64_t T, const moe_router_params* p, uint32_t* inds,
                       float* scores, const BucketOut& o, hipStream_t stream) {
  int st = route_validate(p);
  if (st != MOE_OK) return st;
  if (!inds || !scores || !o.offsets || !o.active || (part ? (!logits_out || ks < 1) : !logits))
    return MOE_E_INVALID_ARG;
  if (!route_bucket_small_fits(T, p, o)) return MOE_E_UNSUPPORTED;
  RouteArgs a{part ? logits_out : logits, bias, inds, scores, T, p->num_experts, p->top_k, p->variant,
              p->norm_topk_prob, p->n_group, p->topk_group, p->routed_scaling_factor};
  const int E = p->num_experts, k = p->top_k;
  if (part && (ks & (ks - 1)) != 0) return MOE_E_INVALID_ARG;
  if (part && ks * ((T * E + route_small_threads(T) - 1) / route_small_threads(T)) > kPartialLoads)
    return MOE_E_INVALID_ARG;
  const size_t lds = route_small_lds(T, E, k);
  const int nbits = bits_for(E);
  if (T <= 4) return launch_route_small<4>(a, part, ks, rbias, logits_out, nbits, o, lds, stream);
  if (T <= 8) return launch_route_small<8>(a, part, ks, rbias, logits_out, nbits, o, lds, stream);
  return launch_route_small<16>(a, part, ks, rbias, logits_out, nbits, o, lds, stream);
}

bool route_bucket_fits(int64_t T, const moe_router_params* p) {
  return p && T >= 1 && T <= kRouteBucketMaxT && p->num_experts <= kFusedMaxE &&
         T * p->top_k <= kFusedMaxP;
}

int route_bucket(const uint16_t* logits, const float* bias, int64_t T, const moe_router_params* p,
                 uint32_t* inds, float* scores, const BucketOut& o, hipStream_t stream) {
  int st = route_validate(p);
  if (st != MOE_OK) return st;
  if (!logits || !inds || !scores || !o.offsets) return MOE_E_INVALID_ARG;
  if (!route_bucket_fits(T, p)) return MOE_E_UNSUPPORTED;
  RouteArgs a{logits, bias, inds, scores, T, p->num_experts, p->top_k, p->variant,
              p->norm_topk_prob, p->n_group, p->topk_group, p->routed_scaling_factor};
  constexpr int NW = 16;
  const int E = p->num_experts;
  const size_t lds = sizeof(int) * (bucket_fused_lds_ints<NW>(E) + static_cast<size_t>(T) * p->top_k);
  const int nbits = bits_for(E);
  const int vpl = (E + 63) / 64;
  if (vpl <= 1)
    MOE_LAUNCH("route_bucket", (route_bucket_kernel<1, NW>), dim3(1), dim3(NW * 64), lds, stream, a, nbits, o);
  else if (vpl <= 2)
    MOE_LAUNCH("route_bucket", (route_bucket_kernel<2, NW>), dim3(1), dim3(NW * 64), lds, stream, a, nbits, o);
  else if (vpl <= 4)
    MOE_LAUNCH("route_bucket", (route_bucket_kernel<4, NW>), dim3(1), dim3(NW * 64), lds, stream, a, nbits, o);
  else
    MOE_LAUNCH("route_bucket", (route_bucket_kernel<8, NW>), dim3(1), dim3(NW * 64), lds, stream, a, nbits, o);
  MOE_CHECK_LAUNCH("route_bucket");
  return MOE_OK;
}

}  // namespace moe
