// qmm_prefill.hip -- grouped affine-dequant GEMM for large token counts
// (prefill), gfx950.  Same contract as the grouped kernel in qmm.hip: rows are
// the expert buckets of the sorted (token, expert) pairs.  Weights stay exact.
//
// Arithmetic.  For output row m and weight row n, with quantization groups g:
//     y[m][n] = sum_k x[m][k] * (s[n,g(k)] q[n][k])  +  sum_g b[n,g] * X[m,g]
//     X[m,g]  = sum_{k in g} x[m][k]                   (group sums, fp32)
// The scaled code s*q is exact in fp32 (8 significant bits of the bf16 scale
// times 4 or 8 bits of code) and is split exactly into two bf16 values,
// hi = bf16(s*q) and lo = s*q - hi (lo has at most 4 / 8 significant bits), so
// the first sum is two bf16 MFMAs per operand pair accumulating straight into
// fp32.  The second sum is a small GEMM over the groups run on the MFMA after
// the K loop, with X and b split into bf16 hi + lo parts (hi*hi + hi*lo +
// lo*hi; the dropped lo*lo term is ~2^-18 relative).  No weight is rounded.
//
// Tiling.  A workgroup of 8 waves computes a BM x 128 output tile of one
// expert: BM = 4*MW token rows by 128 weight rows (GLU: 64 gate rows and the 64
// matching up rows); waves are 4 along M (MW rows each) by 2 along N (two
// 32-row weight tiles each; with GLU a gate tile and its up tile).  K advances
// 64 at a time.  The 128x64 code tile is read once per workgroup, expanded to
// the hi and lo bf16 planes by all 512 threads into a padded, double-buffered
// LDS tile shared by the eight waves.  Activation rows are loaded from global
// memory straight into registers, two K steps ahead; a fragment register is
// refilled as soon as its substep has used it.
//
// K order.  Within a 64-wide K step, lane half h (= lane/32) of the A and B
// operands of substep s carries K = 32h + 8s + [0, 8): each lane's four A
// fragments are one contiguous 64-byte read of its row.
//
// Scheduling.  Blocks are numbered so that consecutive virtual tiles land on
// the same XCD (the hardware deals workgroups round-robin over 8 XCDs): the N
// tiles of one token tile, and the token tiles of one expert, share an L2.

#include <type_traits>

#include "internal.hpp"

namespace moe {

struct PArgs {
  const uint16_t* x;        // input rows [*, K]
  const int32_t* row_in;    // sorted pos -> input row (NULL: pos)
  const int32_t* row_out;   // sorted pos -> output row (NULL: pos)
  const float* gsum;        // [*, gstride] group sums of the input rows
  int gstride;              // >= G rounded up to 16
  int gsum_by_pos;          // gsum rows: 1 = sorted position, 0 = input row (as x)
  const int32_t* offsets;   // [E+1] bucket starts
  const int32_t* tile_off;  // [E+1] first token tile of each expert
  int E;
  int n_tiles;              // 128-row (GLU: 64-column) tiles along N
  const uint32_t* w[2];
  const uint16_t* s[2];
  const uint16_t* b[2];
  int N, K, gs;
  int ldo;                  // output row stride (elements)
  uint16_t* out;
};

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBN = 128;
constexpr int kLdsRow = 72;  // bf16 per LDS row: 64 + 8 padding (144 bytes)

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

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

// hi = bf16(v) (round to nearest even), lo = bf16(v - hi); v - hi is exact in fp32.
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  hi = f2bf(v);
  lo = f2bf(v - bf2f(hi));
}

// byte N of a word as fp32 (one v_cvt_f32_ubyteN)
template <int N>
__device__ __forceinline__ float ubyte_f32(uint32_t w) {
  return static_cast<float>((w >> (8 * N)) & 0xFFu);
}

__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  bf16x2 v;
  v[0] = static_cast<__bf16>(a);
  v[1] = static_cast<__bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

template <int BITS, bool GLU, int MW>
__global__ __launch_bounds__(512, 1) void grouped_gemm_prefill_kernel(PArgs a) {
  constexpr int MT = MW / 32;  // 32-row MFMA tiles per wave along M
  constexpr int BM = 4 * MW;
  constexpr int CPT = 16;      // codes per producer thread per K step (128 x 64 / 512)
  constexpr int QW = CPT * BITS / 32;  // packed words per producer thread
  constexpr int kPlane = kBN * kLdsRow;
  __shared__ __attribute__((aligned(16))) uint16_t bl[2][2 * kPlane];  // [buf][hi | lo]

  // ---- tile lookup (XCD-aware virtual numbering) ----
  const int total = gridDim.x;
  const int bid = blockIdx.x;
  const int v = (bid & 7) * (total >> 3) + (bid >> 3);
  const int mslot = v / a.n_tiles;
  const int ntile = v - mslot * a.n_tiles;
  if (mslot >= a.tile_off[a.E]) return;
  int lo = 0, hi = a.E;  // largest e with tile_off[e] <= mslot
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.tile_off[mid] <= mslot) lo = mid; else hi = mid;
  }
  const int e = lo;
  const int row0 = a.offsets[e] + (mslot - a.tile_off[e]) * BM;
  const int rows = min(BM, a.offsets[e + 1] - row0);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;       // 4 waves along M x 2 along N
  const int h = lane >> 5, l32 = lane & 31;
  const int KS = a.K >> 6;
  const int gdiv = a.gs >> 6;
  const int G = a.K / a.gs;
  const int64_t wpr = static_cast<int64_t>(a.K) * BITS / 32;
  // the wave's two 32-row tiles of the 128-row weight tile; with GLU they are
  // a gate tile and the up tile of the same 32 output columns
  const int nt0 = GLU ? wn : 2 * wn;
  const int nt1 = GLU ? wn + 2 : 2 * wn + 1;

  // weight row of LDS tile row r (GLU: rows 0-63 gate, 64-127 up)
  auto weight_row = [&](int r, int& mat) -> int64_t {
    int wr;
    if (GLU) {
      mat = r >> 6;
      wr = ntile * 64 + (r & 63);
    } else {
      mat = 0;
      wr = ntile * kBN + r;
    }
    return static_cast<int64_t>(e) * a.N + wr;
  };

  // ---- B producer role: thread -> (tile row, K quarter) ----
  const int brow = tid >> 2, bq4 = tid & 3;
  int bmat;
  const int64_t bwrow = weight_row(brow, bmat);
  const uint32_t* wsrc = a.w[bmat] + bwrow * wpr + bq4 * QW;
  const uint16_t* ssrc = a.s[bmat] + bwrow * G;

  // ---- A consumer role: this lane's rows (rows past the tile are clamped to a
  //      valid row; their results are never stored) ----
  const uint16_t* arow[MT];
  int64_t xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = min(wm * MW + mt * 32 + l32, rows - 1);
    const int pos = row0 + r;
    xrow[mt] = a.row_in ? a.row_in[pos] : pos;
    arow[mt] = a.x + xrow[mt] * a.K + 32 * h;
  }

  auto load_codes = [&](int ks, uint32_t* q, uint32_t& sc) {
    const uint32_t* src = wsrc + ks * (64 * BITS / 32);
    if constexpr (QW == 2) {
      const uint2 v2 = *reinterpret_cast<const uint2*>(src);
      q[0] = v2.x;
      q[1] = v2.y;
    } else {
      const u32x4 v4 = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
      for (int i = 0; i < 4; ++i) q[i] = v4[i];
    }
    sc = ssrc[ks / gdiv];  // raw bf16 bits: converted where used, so no wait lands early
  };
  // 4 codes (as fp32) -> 4 hi + 4 lo bf16, packed in K order
  auto split4 = [&](float f0, float f1, float f2, float f3, uint2& ph, uint2& pl) {
    ph.x = pk_bf16(f0, f1);
    ph.y = pk_bf16(f2, f3);
    pl.x = pk_bf16(f0 - __uint_as_float(ph.x << 16), f1 - __uint_as_float(ph.x & 0xffff0000u));
    pl.y = pk_bf16(f2 - __uint_as_float(ph.y << 16), f3 - __uint_as_float(ph.y & 0xffff0000u));
  };
  auto store_codes = [&](int buf, const uint32_t* q, uint32_t sc_bits) {
    // pins the conversion here: hoisted next to its load it would force a full
    // wait on the loads in flight
    asm volatile("" : "+v"(sc_bits));
    const float sc = __uint_as_float(sc_bits << 16);
    uint16_t* dh = &bl[buf][brow * kLdsRow + bq4 * CPT];
    uint16_t* dl = dh + kPlane;
    if constexpr (BITS == 4) {
#pragma unroll
      for (int i = 0; i < QW; ++i) {
        const uint32_t w = q[i];
        const uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;  // codes 0,2,4,6 / 1,3,5,7
        uint2 h0, l0, h1, l1;
        split4(sc * ubyte_f32<0>(ev), sc * ubyte_f32<0>(od),
               sc * ubyte_f32<1>(ev), sc * ubyte_f32<1>(od), h0, l0);
        split4(sc * ubyte_f32<2>(ev), sc * ubyte_f32<2>(od),
               sc * ubyte_f32<3>(ev), sc * ubyte_f32<3>(od), h1, l1);
        *reinterpret_cast<u32x4*>(dh + 8 * i) = u32x4{h0.x, h0.y, h1.x, h1.y};
        *reinterpret_cast<u32x4*>(dl + 8 * i) = u32x4{l0.x, l0.y, l1.x, l1.y};
      }
    } else {
#pragma unroll
      for (int i = 0; i < QW; i += 2) {
        uint2 h0, l0, h1, l1;
        split4(sc * ubyte_f32<0>(q[i]), sc * ubyte_f32<1>(q[i]),
               sc * ubyte_f32<2>(q[i]), sc * ubyte_f32<3>(q[i]), h0, l0);
        split4(sc * ubyte_f32<0>(q[i + 1]), sc * ubyte_f32<1>(q[i + 1]),
               sc * ubyte_f32<2>(q[i + 1]), sc * ubyte_f32<3>(q[i + 1]), h1,
               l1);
        *reinterpret_cast<u32x4*>(dh + 4 * i) = u32x4{h0.x, h0.y, h1.x, h1.y};
        *reinterpret_cast<u32x4*>(dl + 4 * i) = u32x4{l0.x, l0.y, l1.x, l1.y};
      }
    }
  };
  auto load_a = [&](int ks, int mt, int s) -> u32x4 {
    return *reinterpret_cast<const u32x4*>(arow[mt] + ks * 64 + 8 * s);
  };

  f32x16 acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][j][r] = 0.0f;

  // prologue: codes of steps 0 and 1 in flight, step 0 expanded into LDS;
  // activations of steps 0 and 1 in flight
  uint32_t q0[QW], q1[QW];
  uint32_t sc0, sc1;
  load_codes(0, q0, sc0);
  load_codes(min(1, KS - 1), q1, sc1);
  u32x4 af[2][MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      af[0][mt][s] = load_a(0, mt, s);
      af[1][mt][s] = load_a(KS > 1 ? 1 : 0, mt, s);
    }
  store_codes(0, q0, sc0);
  lds_barrier();

  // one K step; AB (the activation register set) is a compile-time constant so
  // the fragment arrays stay in registers (the loop below is unrolled by two)
  auto step = [&](int ks, auto ab_c) {
    constexpr int ab = decltype(ab_c)::value;
    const int buf = ks & 1;
    // codes of step ks+2 into the register slot step ks used; past the end the
    // last step is re-read (in bounds, never used) so every wave issues the same
    // loads and the wait counts stay static
    const int ks2 = min(ks + 2, KS - 1);
    load_codes(ks2, q0, sc0);
    const uint16_t* bh = &bl[buf][l32 * kLdsRow + 32 * h];
    const uint16_t* blo = bh + kPlane;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 h0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(bh + nt0 * 32 * kLdsRow + 8 * s));
      const bf16x8 l0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(blo + nt0 * 32 * kLdsRow + 8 * s));
      const bf16x8 h1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(bh + nt1 * 32 * kLdsRow + 8 * s));
      const bf16x8 l1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(blo + nt1 * 32 * kLdsRow + 8 * s));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bf16x8 av = __builtin_bit_cast(bf16x8, af[ab][mt][s]);
        acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, h0, acc[mt][0], 0, 0, 0);
        acc[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, h1, acc[mt][1], 0, 0, 0);
        acc[mt][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, l0, acc[mt][0], 0, 0, 0);
        acc[mt][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, l1, acc[mt][1], 0, 0, 0);
        // this fragment is consumed: refill it with step ks+2's
        af[ab][mt][s] = load_a(ks2, mt, s);
      }
    }
    // expand step ks+1 into the other buffer (after the last step this writes a
    // buffer no wave reads again: harmless)
    store_codes(buf ^ 1, q1, sc1);
    // rotate the code slots: q1 <- step ks+2 (just loaded into q0)
#pragma unroll
    for (int i = 0; i < QW; ++i) {
      const uint32_t t = q0[i];
      q0[i] = q1[i];
      q1[i] = t;
    }
    const uint32_t t = sc0;
    sc0 = sc1;
    sc1 = t;
    lds_barrier();
  };
  int ks = 0;
  for (; ks + 1 < KS; ks += 2) {
    step(ks, std::integral_constant<int, 0>{});
    step(ks + 1, std::integral_constant<int, 1>{});
  }
  if (ks < KS) step(ks, std::integral_constant<int, 0>{});

  // ---- zero-point term: acc += X . b'^T over the groups (16 per MFMA) ----
  for (int g0 = 0; g0 < G; g0 += 16) {
    bf16x8 xh[MT], xl[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      uint16_t hh[8], ll[8];
      const int64_t grow =
          a.gsum_by_pos ? static_cast<int64_t>(row0 + min(wm * MW + mt * 32 + l32, rows - 1)) : xrow[mt];
      const float* gp = a.gsum + grow * a.gstride + g0 + 8 * h;
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(gp);
      const f32x4 v1 = *reinterpret_cast<const f32x4*>(gp + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        split_bf16(v0[i], hh[i], ll[i]);
        split_bf16(v1[i], hh[4 + i], ll[4 + i]);
      }
      xh[mt] = __builtin_bit_cast(bf16x8, u32x4{hh[0] | (uint32_t(hh[1]) << 16), hh[2] | (uint32_t(hh[3]) << 16),
                                               hh[4] | (uint32_t(hh[5]) << 16), hh[6] | (uint32_t(hh[7]) << 16)});
      xl[mt] = __builtin_bit_cast(bf16x8, u32x4{ll[0] | (uint32_t(ll[1]) << 16), ll[2] | (uint32_t(ll[3]) << 16),
                                               ll[4] | (uint32_t(ll[5]) << 16), ll[6] | (uint32_t(ll[7]) << 16)});
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int mat;
      const int64_t wr = weight_row((j ? nt1 : nt0) * 32 + l32, mat);
      const uint16_t* bp = a.b[mat] ? a.b[mat] + wr * G : nullptr;
      uint16_t hh[8], ll[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int g = g0 + 8 * h + i;
        const float bpv = (g < G && bp) ? bf2f(bp[g]) : 0.0f;
        split_bf16(bpv, hh[i], ll[i]);
      }
      const bf16x8 bh = __builtin_bit_cast(bf16x8, u32x4{hh[0] | (uint32_t(hh[1]) << 16), hh[2] | (uint32_t(hh[3]) << 16),
                                                         hh[4] | (uint32_t(hh[5]) << 16), hh[6] | (uint32_t(hh[7]) << 16)});
      const bf16x8 blw = __builtin_bit_cast(bf16x8, u32x4{ll[0] | (uint32_t(ll[1]) << 16), ll[2] | (uint32_t(ll[3]) << 16),
                                                          ll[4] | (uint32_t(ll[5]) << 16), ll[6] | (uint32_t(ll[7]) << 16)});
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh[mt], bh, acc[mt][j], 0, 0, 0);
        acc[mt][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh[mt], blw, acc[mt][j], 0, 0, 0);
        acc[mt][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl[mt], bh, acc[mt][j], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: D layout of the 32x32 MFMA: column = lane%32,
  //      row = 8*(r/4) + 4*(lane/32) + r%4 ----
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = wm * MW + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
      if (m >= rows) continue;
      const int64_t op = a.row_out ? a.row_out[row0 + m] : row0 + m;
      uint16_t* orow = a.out + op * a.ldo;
      if constexpr (GLU) {
        const float g = bfr(acc[mt][0][r]), u = bfr(acc[mt][1][r]);
        orow[ntile * 64 + wn * 32 + l32] = f2bf(silu(g) * u);
      } else {
        orow[ntile * kBN + nt0 * 32 + l32] = f2bf(acc[mt][0][r]);
        orow[ntile * kBN + nt1 * 32 + l32] = f2bf(acc[mt][1][r]);
      }
    }
  }
}

// gsum[r][g] = sum of the gs inputs of group g of row src(r) (fp32, in K
// order), src(r) = row_in ? row_in[r] : r; columns G..gstride-1 are zero.  One
// wave per row.
__global__ __launch_bounds__(256) void group_sums_kernel(const uint16_t* __restrict__ x,
                                                         const int32_t* __restrict__ row_in, int64_t R, int K,
                                                         int gs, int gstride, float* __restrict__ gsum) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const int lane = threadIdx.x & 63;
  const int G = K / gs;
  const uint16_t* xr = x + (row_in ? static_cast<int64_t>(row_in[r]) : r) * K;
  for (int g = lane; g < gstride; g += 64) {
    float s = 0.0f;
    if (g < G)
      for (int i = 0; i < gs; i += 8) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(xr + static_cast<int64_t>(g) * gs + i);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s += __uint_as_float(v[q] << 16);
          s += __uint_as_float(v[q] & 0xffff0000u);
        }
      }
    gsum[r * gstride + g] = s;
  }
}

// tile_off[e] = sum over e' < e of ceil(count(e') / BM)
__global__ __launch_bounds__(1024) void make_tiles_kernel(const int32_t* __restrict__ offsets, int E,
                                                          int BM, int32_t* __restrict__ tile_off) {
  __shared__ int tmp[1025];
  const int e = threadIdx.x;
  int c = 0;
  if (e < E) c = (offsets[e + 1] - offsets[e] + BM - 1) / BM;
  tmp[e] = c;
  __syncthreads();
  if (e == 0) {
    int run = 0;
    for (int i = 0; i < E; ++i) {
      const int t = tmp[i];
      tmp[i] = run;
      run += t;
    }
    tmp[E] = run;
  }
  __syncthreads();
  for (int i = e; i <= E; i += 1024) tile_off[i] = tmp[i];
}

template <int BITS, bool GLU>
int launch_mw(const PArgs& a, int mw, unsigned grid, hipStream_t stream) {
  if (mw == 64)
    MOE_LAUNCH(GLU ? "gemm_gate_up_swiglu" : "gemm_down", (grouped_gemm_prefill_kernel<BITS, GLU, 64>), dim3(grid),
               dim3(512), 0, stream, a);
  else
    MOE_LAUNCH(GLU ? "gemm_gate_up_swiglu" : "gemm_down", (grouped_gemm_prefill_kernel<BITS, GLU, 32>), dim3(grid),
               dim3(512), 0, stream, a);
  return launch_status("grouped_gemm_prefill");
}

}  // namespace

int prefill_gsum_stride(const moe_qweight* w) { return (w->K / w->group_size + 15) / 16 * 16; }

bool prefill_supported(const moe_qweight* w0, const moe_qweight* w1) {
  if (w0->group_size % 64 != 0) return false;
  if (w1) return w0->N % 64 == 0;
  return w0->N % kBN == 0;
}

// offsets [E+1] on device; tile_off [E+1] scratch; gsum scratch of
// max(x_rows, P) * prefill_gsum_stride(w0) floats.  x_rows = rows of x when
// known (group sums are then taken once per input row), -1 otherwise (sums of
// the gathered rows, one per sorted position).  P = total rows, slots = number
// of non-empty experts at most (bounds the partial tiles).
int grouped_gemm_prefill(const uint16_t* x, int64_t x_rows, const int32_t* row_in,
                         const int32_t* row_out, float* gsum, const int32_t* offsets, int32_t* tile_off,
                         int E, int64_t P, int slots, const moe_qweight* w0, const moe_qweight* w1,
                         uint16_t* out, hipStream_t stream) {
  if (E > 1024) return MOE_E_UNSUPPORTED;
  const int gstride = prefill_gsum_stride(w0);
  const bool by_pos = x_rows < 0;
  const int64_t R = by_pos ? P : x_rows;
  if (R > 0) {
    MOE_LAUNCH("group_sums", group_sums_kernel, dim3(static_cast<unsigned>((R + 3) / 4)), dim3(256), 0, stream, x,
               by_pos ? row_in : nullptr, R, w0->K, w0->group_size, gstride, gsum);
    MOE_CHECK_LAUNCH("group_sums");
  }
  const int64_t avg = slots > 0 ? P / slots : P;
  const int BM = avg >= 192 ? 256 : 128;
  MOE_LAUNCH("make_tiles", make_tiles_kernel, dim3(1), dim3(1024), 0, stream, offsets, E, BM, tile_off);
  MOE_CHECK_LAUNCH("make_tiles");
  PArgs a{};
  a.x = x;
  a.row_in = row_in;
  a.row_out = row_out;
  a.gsum = gsum;
  a.gstride = gstride;
  a.gsum_by_pos = by_pos ? 1 : 0;
  a.offsets = offsets;
  a.tile_off = tile_off;
  a.E = E;
  a.w[0] = w0->w;
  a.s[0] = w0->scales;
  a.b[0] = w0->biases;
  if (w1) {
    a.w[1] = w1->w;
    a.s[1] = w1->scales;
    a.b[1] = w1->biases;
  }
  a.N = w0->N;
  a.K = w0->K;
  a.gs = w0->group_size;
  a.n_tiles = w1 ? w0->N / 64 : w0->N / kBN;
  a.ldo = w0->N;
  a.out = out;
  const int64_t mslots = (P + BM - 1) / BM + slots;
  int64_t grid = mslots * a.n_tiles;
  grid = (grid + 7) / 8 * 8;
  if (grid > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  const int mw = BM / 4;
  if (w0->bits == 4)
    return w1 ? launch_mw<4, true>(a, mw, static_cast<unsigned>(grid), stream)
              : launch_mw<4, false>(a, mw, static_cast<unsigned>(grid), stream);
  return w1 ? launch_mw<8, true>(a, mw, static_cast<unsigned>(grid), stream)
            : launch_mw<8, false>(a, mw, static_cast<unsigned>(grid), stream);
}

}  // namespace moe
