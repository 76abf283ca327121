// qmm.hip -- grouped affine-dequant matmul (the gather_qmm of the reference,
// src/common/switch_layers.cpp:94-102) for the MoE experts at decode sizes,
// plus SwiGLU and the weighted combine, gfx950.
//
// Work unit: one wave = (one expert, 16 output rows) over a K range; with GLU
// the gate rows and the up rows of the same 16 columns, so SwiGLU is applied
// in registers.  The expert's tokens are its bucket [offsets[e], offsets[e+1])
// in chunks of 16.  Large buckets (prefill) go to qmm_prefill.hip instead.
//
// Per 64-wide K block and 16x16 (token x row) tile, one wave runs two
// v_mfma_f32_16x16x32_bf16.  The weight operand is exact: a 4-bit code q
// becomes the bf16 value 128 + q by OR-ing it under the exponent pattern
// 0x4300 (bf16 has 7 mantissa bits, so 128..143 are exact), an 8-bit code is
// converted through fp32 (0..255 is exact in bf16).  Scale and bias are
// applied per group in fp32 outside the MFMA:
//     sum_k x_k (s q_k + b) = s * sum_k x_k q'_k + (b - 128 s) * sum_k x_k
// with q' = q + 128 (4-bit) or q' = q (8-bit).  No weight is rounded to bf16.
//
// Lane layout (wave64, 16x16x32 MFMA): lane = 16*g + i.  The A operand
// (tokens) takes row i, K slots 8g..8g+7; B (weights) takes column (row of W)
// i, K slots 8g..8g+7; D holds rows 4g..4g+3 of column i.  A 64-wide K block
// is split so that lane group g owns K [16g, 16g+16) of the block: slots of
// MFMA step s are K 16g + 8s + [0, 8).  For 4-bit weights the 8 codes of one
// uint32 are placed as (q0,q4,q1,q5,q2,q6,q3,q7) -- the order a shift-and-mask
// produces -- and the activations are permuted the same way.

#include <algorithm>
#include <cmath>

#include "internal.hpp"
#include "route_impl.hpp"

namespace moe {
namespace {

struct GQArgs {
  const uint16_t* x;        // input rows [*, K] bf16
  const int32_t* row_in;    // sorted pos -> input row (NULL: pos)
  const int32_t* row_out;   // sorted pos -> output row (NULL: pos)
  const int32_t* offsets;   // [E+1]
  const int32_t* active;    // [E][4] slot records {expert, first row, rows, 0} (NULL: the slot is the expert)
  const int32_t* num_active;
  const uint32_t* w[2];
  const uint16_t* s[2];
  const uint16_t* b[2];
  int N, K, gs;
  uint16_t* out;            // [*, N] bf16
  int out_pairs;            // GLU: write h in pair K order (pair_pos within 8 columns)
  // SwitchLinear biases [E, N] or NULL: gate (and, with GLU, up); without GLU
  // lb[0] covers every output column (a DUO wave's second tile too)
  const uint16_t* lb[2];
  // > 0: the rows of one expert (expert 0), slot s = rows [one_per s,
  // one_per (s + 1)) clamped to one_rows (no slot records are read)
  int one_rows;
  int one_per;              // rows per slot: a multiple of 16
  int act;                  // GLU: moe_activation of h = act(gate, up)
  // one token routed in the kernel (RVPL > 0; see FusedRoute): the router's
  // partial sums [rks][E], its bias, and the outputs workgroup 0 writes
  const float* rpart;
  int rks;
  const uint16_t* rbias;
  uint16_t* rlogits;
  RouteArgs ra;             // ra.inds / ra.scores: written by workgroup 0 only
  BucketOut rbo;
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));  // 16 bytes at a dword boundary

// A dword as a bf16 pair, taken by value: hipcc compiled __builtin_bit_cast
// applied directly to a vector element (v[j] of a u32x4) as a cast of element
// 0 for every j, so the element is copied out first
__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2, v); }

__device__ __forceinline__ uint32_t pick4(const u32x4& v, int d) {
  return d & 2 ? (d & 1 ? v.w : v.z) : (d & 1 ? v.y : v.x);
}

// (v & m) | k in one v_and_or_b32; m and k are passed in registers (a VOP3
// instruction takes no literal here), which the compiler hoists out of loops
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t m, uint32_t k) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(m), "v"(k));
  return r;
}

// 8 nibbles of one word -> bf16 (128 + q) in the order (q0,q4,q1,q5,q2,q6,q3,q7)
__device__ __forceinline__ u32x4 nibbles_to_bf16(uint32_t w, uint32_t m, uint32_t k) {
  u32x4 r;
  r.x = and_or(w, m, k);
  r.y = and_or(w >> 4, m, k);
  r.z = and_or(w >> 8, m, k);
  r.w = and_or(w >> 12, m, k);
  return r;
}

// 4 bytes of one word -> 2 packed bf16 pairs, natural order (exact: q < 256)
__device__ __forceinline__ u32x2 bytes_to_bf16(uint32_t w) {
  const uint32_t f0 = __float_as_uint(static_cast<float>(w & 0xffu));
  const uint32_t f1 = __float_as_uint(static_cast<float>((w >> 8) & 0xffu));
  const uint32_t f2 = __float_as_uint(static_cast<float>((w >> 16) & 0xffu));
  const uint32_t f3 = __float_as_uint(static_cast<float>(w >> 24));
  u32x2 r;
  r.x = (f0 >> 16) | (f1 & 0xffff0000u);
  r.y = (f2 >> 16) | (f3 & 0xffff0000u);
  return r;
}

// 16 six-bit codes = bits [6c, 6c+6) of w2:w1:w0 (the LSB-first stream) ->
// bf16 (128 + code c) in natural order: lo = codes 0..7, hi = codes 8..15.
// Pair j (codes 2j, 2j+1) is the 12-bit field at bit 12j.
__device__ __forceinline__ void q6_to_bf16(uint32_t w0, uint32_t w1, uint32_t w2, u32x4& lo, u32x4& hi) {
  uint32_t f[8];
  f[0] = w0;
  f[1] = w0 >> 12;
  f[2] = __builtin_amdgcn_alignbit(w1, w0, 24);
  f[3] = w1 >> 4;
  f[4] = w1 >> 16;
  f[5] = __builtin_amdgcn_alignbit(w2, w1, 28);
  f[6] = w2 >> 8;
  f[7] = w2 >> 20;
  uint32_t d[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) d[j] = 0x43004300u | (f[j] & 0x3fu) | ((f[j] << 10) & 0x003f0000u);
  lo = u32x4{d[0], d[1], d[2], d[3]};
  hi = u32x4{d[4], d[5], d[6], d[7]};
}

// 16 BITS-bit codes (BITS = 2, 3, 5) of the LSB-first stream, starting at
// bit `sh` (0 or 16) of w[0] -> bf16 (128 + code c) in natural order: lo =
// codes 0..7, hi = codes 8..15.  The field is first shifted down to bit 0
// of f[] (v_alignbit); pair j (codes 2j, 2j+1) is then the 2*BITS-bit field
// at bit 2j*BITS of f[].
template <int BITS>
__device__ __forceinline__ void qn_to_bf16(const uint32_t (&w)[BITS == 2 ? 1 : BITS == 3 ? 2 : 3], uint32_t sh,
                                           u32x4& lo, u32x4& hi) {
  constexpr int ND = BITS == 2 ? 1 : BITS == 3 ? 2 : 3;
  constexpr uint32_t M = (1u << BITS) - 1u;
  uint32_t f[ND];
#pragma unroll
  for (int t = 0; t < ND; ++t) f[t] = t + 1 < ND ? __builtin_amdgcn_alignbit(w[t + 1], w[t], sh) : w[t] >> sh;
  uint32_t d[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    constexpr int kB = 2 * BITS;
    const int pos = kB * j, k = pos >> 5, s = pos & 31;
    const uint32_t fj = s + kB <= 32 || k + 1 >= ND ? f[k] >> s : __builtin_amdgcn_alignbit(f[k + 1], f[k], s);
    d[j] = 0x43004300u | (fj & M) | ((fj << (16 - BITS)) & (M << 16));
  }
  lo = u32x4{d[0], d[1], d[2], d[3]};
  hi = u32x4{d[4], d[5], d[6], d[7]};
}

// 8 BITS-bit codes (BITS = 2, 3, 5, 6) of the LSB-first stream starting at
// bit `sh` (a multiple of 8) of w0 -> 4 packed bf16 pairs (128 + code), natural order
template <int BITS>
__device__ __forceinline__ u32x4 qn8_to_bf16(uint32_t w0, uint32_t w1, uint32_t sh) {
  constexpr uint32_t M = (1u << BITS) - 1u;
  const uint32_t f0 = __builtin_amdgcn_alignbit(w1, w0, sh), f1 = w1 >> sh;
  u32x4 d;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    constexpr int kB = 2 * BITS;
    const int pos = kB * j, k = pos >> 5, sft = pos & 31;
    const uint32_t fj = k ? f1 >> sft : sft + kB <= 32 ? f0 >> sft : __builtin_amdgcn_alignbit(f1, f0, sft);
    d[j] = 0x43004300u | (fj & M) | ((fj << (16 - BITS)) & (M << 16));
  }
  return d;
}

// Group size 32: the bf16 operand of the 8 codes K k0 .. k0+7 of stage row lr
// (128-byte LDS rows of XOR-swizzled 16-byte chunks; 4 bits: 128 + q in the
// pair order of nibbles_to_bf16, 8 bits: q, else 128 + q in natural order)
template <int BITS>
__device__ __forceinline__ bf16x8 g32_operand(const uint8_t* sb, int lr, int k0, uint32_t nib_mask, uint32_t magic) {
  const uint8_t* row = sb + lr * 128;
  auto dword = [&](int D) {
    return *reinterpret_cast<const uint32_t*>(row + 16 * ((D >> 2) ^ (lr & 7)) + 4 * (D & 3));
  };
  if constexpr (BITS == 4) {
    return __builtin_bit_cast(bf16x8, nibbles_to_bf16(dword(k0 >> 3), nib_mask, magic));
  } else if constexpr (BITS == 8) {
    const u32x2 p0 = bytes_to_bf16(dword(k0 >> 2)), p1 = bytes_to_bf16(dword((k0 >> 2) + 1));
    return __builtin_bit_cast(bf16x8, u32x4{p0.x, p0.y, p1.x, p1.y});
  } else {
    const int boff = k0 * BITS / 8;  // (k0 a multiple of 8: a whole byte)
    return __builtin_bit_cast(bf16x8, qn8_to_bf16<BITS>(dword(boff >> 2), dword((boff >> 2) + 1),
                                                        static_cast<uint32_t>((boff & 3) * 8)));
  }
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// One wave = one 16-row tile of one expert (with GLU: the gate tile and the
// up tile of the same 16 output columns) over a K range.  KSPLIT waves of a
// workgroup share a tile and split K (summed through LDS); with KSPLIT = 1
// the four waves of a workgroup are independent tiles (no barrier runs unless
// they share the activation ring, XLDS below).
//
// A wave streams its codes, scales and biases through a private two-stage LDS
// ring by DMA.  A stage is NB 64-wide K blocks: 128 bytes of every code row
// (one DMA instruction moves 8 whole rows, so HBM sees full lines; 16-byte
// chunk c of stage row r sits at slot c ^ (r & 7)) plus the two scale and two
// bias dwords of every row that cover the stage's groups.  The activations of
// a stage are read from global memory (they are shared by every tile of the
// expert and stay in L2; XLDS: through a ring in LDS); their per-group sums
// come from an MFMA against an all-ones operand, already in the accumulator
// layout.
// PAIRS (4-bit): the activation rows are stored in pair K order already (the
// order of the code operand), else each 16-byte unit is reordered in registers.
// SREG: the scales and biases of the K part are held in registers 32 groups
// at a time (lane group g holds groups 8g..8g+7 of the period for its row:
// 16 bytes of a row per lane, half a line per row per instruction) and moved
// to the lanes that need them with ds_bpermute; with SROLL (a K part longer
// than 32 groups) the next period's are loaded after a period's last stage.
// Without SREG the two scale and two bias dwords of every row ride with each
// stage's DMA (32 partly used lines per instruction).
// DUO (without GLU): a wave takes two adjacent 16-row tiles of the expert
// (the host passes w/s/b[1] = rows 16.. of w/s/b[0] and counts 32-row tiles),
// so a short K range still moves 8 code rows per DMA instruction and the
// per-wave set-up is paid once per 32 rows.
// XLDS (K not split, tiles per expert a multiple of 4, so the four waves of a
// workgroup serve the same expert and token chunk): the activations of a stage
// come through a two-stage LDS ring shared by the workgroup, filled by DMA one
// stage ahead (each wave moves 1/4 of a stage: 16 token rows x 128 bytes per
// block, 16-byte chunk c of row t at slot c ^ (t & 7)), so no global load is
// awaited in the step that issues it; one barrier per stage orders the ring.
// RVPL > 0 (GLU, one token): the workgroup first routes the token itself
// (route_token with RVPL candidates per lane, from the router's partial sums)
// and takes slot s = the token's s-th expert in ascending order, one row;
// workgroup 0 also writes what route_bucket_small would (FusedRoute).
template <int BITS, bool GLU, int KSPLIT, int GS, bool PAIRS, bool SREG, bool DUO = false, bool XLDS = false,
          bool SROLL = false, int RVPL = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(PAIRS || !SREG ? 3 : 2))) void grouped_qmm_kernel(GQArgs a, int tiles16, int slots) {
  static_assert(RVPL == 0 || (GLU && !XLDS), "routing in the kernel: gate|up, input row 0");
  static_assert(!(GLU && DUO), "DUO pairs tiles of one projection");
  static_assert(!XLDS || KSPLIT == 1, "the shared activation ring needs whole-K waves");
  constexpr int NMAT = GLU || DUO ? 2 : 1;
  // 64-wide K blocks per stage, NB * 8 * BITS code bytes of each row (of its
  // 128-byte LDS row: 2 bits 64, 3 bits 96, 5 bits 80, 6 bits 96); group
  // size 32 (G32): two blocks, four groups
  constexpr bool G32 = GS == 32;
  constexpr int NB = G32 ? 2 : BITS <= 4 ? 4 : 2;
  constexpr int ROWS = 16 * NMAT;                 // code rows per wave
  constexpr int kBlockBytes = 8 * BITS;           // code bytes per row per 64-wide block
  constexpr int kCodes = ROWS * 128;              // code bytes per stage
  constexpr int kStage = kCodes + (SREG ? 0 : 512);  // + 2 scale and 2 bias dwords per row (as 32 rows)
  constexpr int kWave = 2 * kStage;
  constexpr int kXStage = NB * 16 * 128;          // XLDS: activations of a stage (NB blocks x 16 rows)
  constexpr int kXI = 2 * NB / 4;                 // XLDS: DMA instructions per wave per stage (1 KB each)
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * kWave + (XLDS ? 2 * kXStage : 0)];
  uint8_t* const xring = lds + 4 * kWave;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kp = wave % KSPLIT;                        // this wave's K part
  const int tile = blockIdx.x * (4 / KSPLIT) + wave / KSPLIT;
  const int slot = tile / tiles16;
  const int n0 = (tile - slot * tiles16) * (DUO ? 32 : 16);
  bool valid = slot < slots;
  int e = slot;
  int beg = 0, cnt = 0;
  if constexpr (RVPL > 0) {
    // wave 0: the logits from the partial sums in its registers (slice order,
    // as route_bucket_small), the token routed, its experts sorted into the
    // slot records (the weights only in workgroup 0)
    __shared__ int rexp[16];
    const bool wg0 = blockIdx.x == 0;
    if (wave == 0) {
      float lv[RVPL];
      token_logits_from_partials<RVPL>(a.rpart, a.rks, a.ra.E, a.ra.E, a.rbias, lane, lv, wg0 ? a.rlogits : nullptr);
      RouteArgs ra = a.ra;
      if (!wg0) {
        ra.inds = nullptr;
        ra.scores = nullptr;
      }
      const int idx = route_token_lv<RVPL>(ra, 0, lane, lv);
      // sorted position of slot `lane`: its experts below it (they are distinct)
      int pos = 0;
#pragma unroll
      for (int r = 0; r < 16; ++r) pos += r < ra.k && __builtin_amdgcn_readlane(idx, r) < idx ? 1 : 0;
      if (lane < ra.k) rexp[pos] = idx;
      if (wg0) bucket_one_token(idx, ra.k, ra.E, a.rbo);
    }
    __syncthreads();
    e = valid ? rexp[slot] : 0;  // (slots = k <= 16)
    beg = slot;
    cnt = valid ? 1 : 0;
  } else if (valid && a.one_rows > 0) {
    e = 0;
    beg = a.one_per * slot;
    cnt = min(a.one_per, a.one_rows - beg);
    valid = cnt > 0;
  } else if (valid && a.active) {  // the slot's record: one load
    const int4 rec = reinterpret_cast<const int4*>(a.active)[slot];
    e = rec.x;
    beg = rec.y;
    cnt = rec.z;
    valid = cnt > 0;
  } else if (valid) {
    beg = a.offsets[e];
    cnt = a.offsets[e + 1] - beg;
  }

  const int g = lane >> 4, i16 = lane & 15;
  const int KB = a.K >> 6;
  // whole stages per K part, so every stage starts at a multiple of NB blocks
  // (its groups then sit in the two scale dwords the stage loads)
  const int per = ((KB + KSPLIT - 1) / KSPLIT + NB - 1) / NB * NB;
  const int jb = min(KB, kp * per);
  const int je = min(KB, jb + per);
  const int G = a.K / GS;
  constexpr int gdiv = G32 ? 1 : GS / 64;  // blocks per group (G32: two groups a block, handled apart)
  const int64_t rbytes = static_cast<int64_t>(a.K) * BITS / 8;
  uint8_t* ring = lds + wave * kWave;

  // DMA roles.  Codes: block d (rows 8d..8d+7) of a stage; stage row
  // lr = 16*mt + r16.  Scales/biases: lane -> (row lane%32, dword lane/32).
  const uint8_t* crow[ROWS / 8];
  int cblk[ROWS / 8], coff[ROWS / 8];
#pragma unroll
  for (int d = 0; d < ROWS / 8; ++d) {
    const int lr = 8 * d + (lane >> 3);
    const int mt = lr >> 4, r16 = lr & 15;
    const int64_t row = static_cast<int64_t>(e) * a.N + min(n0 + r16, a.N - 1);  // (a partial last tile re-reads row N-1)
    const int c = (lane & 7) ^ (lr & 7);
    crow[d] = reinterpret_cast<const uint8_t*>(a.w[mt]) + row * rbytes;
    if constexpr (kBlockBytes % 16 == 0) {
      cblk[d] = c / (kBlockBytes / 16);
      coff[d] = 16 * (c % (kBlockBytes / 16));
    } else {  // 3, 5 bits: chunk c of the stage's contiguous bytes
      cblk[d] = 0;
      coff[d] = 16 * c;
    }
  }
  const int sr = lane & 31, sd = lane >> 5;  // scale role: stage row, dword
  const uint16_t* ssrc;
  const uint16_t* bsrc;
  {
    const int mt = (sr >> 4) % NMAT;
    const int64_t row = static_cast<int64_t>(e) * a.N + min(n0 + (sr & 15), a.N - 1);
    ssrc = a.s[mt] + row * G;
    bsrc = a.b[mt] ? a.b[mt] + row * G : nullptr;
  }
  // stage st for the batch starting at block j0: every lane issues the same
  // number of DMA instructions (3 + ROWS/8), so the wait counts are static
  auto issue = [&](int j0, int st) {
    uint8_t* sb = ring + st * kStage;
#pragma unroll
    for (int d = 0; d < ROWS / 8; ++d) {
      if constexpr (kBlockBytes % 16 == 0) {
        const int blk = min(j0 + cblk[d], KB - 1);  // a partial batch re-reads block KB-1 (unused)
        load_lds16(crow[d] + static_cast<int64_t>(blk) * kBlockBytes + coff[d], sb + d * 1024);
      } else {  // chunks past the stage or the row re-read the row's last 16 bytes (unused)
        const int64_t off = min(static_cast<int64_t>(j0) * kBlockBytes + coff[d], rbytes - 16);
        load_lds16(crow[d] + off, sb + d * 1024);
      }
    }
    if constexpr (!SREG) {
      const int dw = min((G32 ? j0 : (j0 / gdiv) / 2) + sd, G / 2 - 1);  // (G32: block j, groups 2j, 2j + 1)
      load_lds4(ssrc + 2 * dw, sb + kCodes);
      load_lds4((bsrc ? bsrc : ssrc) + 2 * dw, sb + kCodes + 256);
      // (ROWS = 16 without GLU: lanes 16..31 of each half repeat rows 0..15)
    }
  };
  constexpr int kIssue = ROWS / 8 + (SREG ? 0 : 2);
  // SREG: groups g0 + 32 per + 8g .. +7 of row (mt, i16), scales and biases,
  // for period per of 32 groups of the K part (reloaded after each period)
  const int g0 = jb / gdiv;
  u32x4 sreg[NMAT], breg[NMAT];
  auto load_sreg = [&](int per) {
    const int s0 = g0 + 32 * per + 8 * g;
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt) sreg[mt] = breg[mt] = u32x4{0u, 0u, 0u, 0u};
    if (32 * per + 8 * g >= (je - jb) / gdiv) return;  // none of this lane group's groups is in the part
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt) {
      const int64_t row = static_cast<int64_t>(e) * a.N + min(n0 + i16, a.N - 1);
      const uint16_t* sp = a.s[mt] + row * G;
      const uint16_t* bp = a.b[mt] ? a.b[mt] + row * G : sp;
      if (s0 + 8 <= G) {  // 16 bytes inside the row (dword aligned)
        sreg[mt] = *reinterpret_cast<const u32x4a*>(sp + s0);
        breg[mt] = *reinterpret_cast<const u32x4a*>(bp + s0);
      } else {  // the row ends inside: a dword past it is clamped (its groups are not used)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int gi = min(s0 + 2 * d, G - 2);
          sreg[mt][d] = *reinterpret_cast<const uint32_t*>(sp + gi);
          breg[mt][d] = *reinterpret_cast<const uint32_t*>(bp + gi);
        }
      }
      if (!a.b[mt]) breg[mt] = u32x4{0u, 0u, 0u, 0u};  // no biases: b = 0 (no select per block)
    }
  };

  // constants of the nibble expansion, kept in VGPRs
  uint32_t kNibMask = 0x000F000Fu, kMagic = 0x43004300u;
  asm volatile("" : "+v"(kNibMask), "+v"(kMagic));
  f32x4 acc[NMAT];
  const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});

  // SwitchLinear's bias (switch_layers.cpp:111-114) of this lane's output
  // feature n0 + i16 (a DUO wave's second tile: + 16), indexed by the feature,
  // not the stored column; loaded once per tile, before any store (the
  // compiler would otherwise reload it after each store, which might alias it)
  const int64_t fb = static_cast<int64_t>(e) * a.N + n0 + i16;
  float lbv[2] = {0.0f, 0.0f};
  if (valid && n0 + i16 < a.N) {
    if constexpr (GLU) {
      if (a.lb[0]) lbv[0] = bf2f(a.lb[0][fb]);
      if (a.lb[1]) lbv[1] = bf2f(a.lb[1][fb]);
    } else {
#pragma unroll
      for (int mt = 0; mt < NMAT; ++mt)
        if (a.lb[0]) lbv[mt] = bf2f(a.lb[0][fb + 16 * mt]);
    }
  }

  for (int tc = 0; tc < cnt || (tc == 0 && KSPLIT > 1); tc += 16) {
    const int mcount = max(0, min(16, cnt - tc));
    const bool mval = i16 < mcount;
    const int pos_m = beg + tc + max(0, min(i16, mcount - 1));
    const int64_t xrow = RVPL > 0 || !valid ? 0 : a.row_in ? a.row_in[pos_m] : pos_m;  // (RVPL: the one token)
    // output rows of this lane's four results, loaded with the input row
    int orow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * g + r;
      const int pos = beg + tc + min(m, max(mcount - 1, 0));
      orow[r] = valid && kp == 0 && a.row_out && m < mcount ? a.row_out[pos] : pos;
    }
    // this lane's K values of a block: 16g .. 16g+15 (G32: 8g .. 8g+7 and 32 + 8g ..)
    const uint16_t* xp = a.x + xrow * a.K + (G32 ? 8 : 16) * g;
#pragma unroll
    for (int mt = 0; mt < NMAT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // XLDS: this lane's source rows for the ring, token rows lane/8 and
    // 8 + lane/8 of the chunk (clamped to its last token: every ring row holds
    // a real row, the rows past the chunk are never stored)
    const uint16_t* xsrc[2];
    if constexpr (XLDS) {
#pragma unroll
      for (int rg = 0; rg < 2; ++rg) {
        const int t = 8 * rg + (lane >> 3);
        const int pos = beg + tc + min(t, max(mcount - 1, 0));
        const int64_t r = valid ? (a.row_in ? a.row_in[pos] : pos) : 0;
        xsrc[rg] = a.x + r * a.K + 8 * ((lane & 7) ^ (t & 7));
      }
    }
    // XLDS: wave w moves instructions kXI*w .. of the stage at block j0 into
    // ring slot xs (instruction i: block i/2, token rows 8*(i%2) .. +7)
    auto issue_x = [&](int j0, int xs) {
#pragma unroll
      for (int q = 0; q < kXI; ++q) {
        const int ins = wave * kXI + q;
        const int p = ins >> 1, rg = ins & 1;
        const int blk = min(j0 + p, KB - 1);  // past the end: re-read the last block (unused)
        load_lds16(xsrc[rg] + 64 * blk, xring + xs * kXStage + p * 2048 + rg * 1024);
      }
    };

    if (valid && jb < je) {
      if constexpr (SREG) load_sreg(0);  // awaited with the first stage
      issue(jb, 0);
      if constexpr (XLDS) {
        lds_barrier();  // every wave has finished reading the ring (previous token chunk)
        issue_x(jb, 0);
      }
      // activations: only the lanes of the bucket's tokens load (the others
      // keep zeros, so their MFMA rows are zero)
      u32x4 xa[NB][2];
#pragma unroll
      for (int p = 0; p < NB; ++p) xa[p][0] = xa[p][1] = u32x4{0u, 0u, 0u, 0u};
      // one stage: blocks j0 .. j0+NB-1 from ring slot st; u = the stage's
      // index modulo kUnroll (compile time with SREG)
      auto stage = [&](const int j0, const int st, const int u) __attribute__((always_inline)) {
        if constexpr (!XLDS) {
#pragma unroll
          for (int p = 0; p < NB; ++p) {
            const int j = min(j0 + p, je - 1);
            if (mval) {
              xa[p][0] = *reinterpret_cast<const u32x4*>(xp + 64 * j);
              xa[p][1] = *reinterpret_cast<const u32x4*>(xp + 64 * j + (G32 ? 32 : 8));
            }
          }
        }
        issue(min(j0 + NB, je - 1), st ^ 1);  // next stage (past the end: re-read, unused)
        // this stage's codes and activations have landed (XLDS: the ring's part
        // of this wave, issued before the DMA above); the next stage may be in flight
        wait_vmcnt<kIssue>();
        if constexpr (XLDS) {
          // every wave's part of this stage's activations has landed, and every
          // wave has finished the previous stage, whose ring slot is refilled now
          lds_barrier();
          issue_x(j0 + NB, st ^ 1);
        }
        const uint8_t* sb = ring + st * kStage;
        // the stage's scale and bias dwords of this lane's rows (two groups each)
        uint32_t sdw[NMAT][2], bdw[NMAT][2];
        const int D = SREG ? ((j0 - jb) / gdiv) >> 1 : 0;
        if constexpr (SREG) {
          // dword D + q of the part's groups (D: the stage's first group / 2)
          // sits in lane group (D + q) / 4 of the row, register (D + q) % 4;
          // (D + q) % 4 is a compile-time constant: the stages are unrolled
          // kUnroll at a time and kUnroll stages advance D by a multiple of 4
          const int Ds = (u * (NB / gdiv)) >> 1;
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const int Dq = min((D & 15) + q, 15);  // (within the period; a dword past the part's last: not used)
            const int src = (16 * (Dq >> 2) + i16) * 4;
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt) {
              sdw[mt][q] = __builtin_amdgcn_ds_bpermute(src, pick4(sreg[mt], (Ds + q) & 3));
              bdw[mt][q] = __builtin_amdgcn_ds_bpermute(src, pick4(breg[mt], (Ds + q) & 3));
            }
          }
        } else {
#pragma unroll
          for (int mt = 0; mt < NMAT; ++mt)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              sdw[mt][q] = *reinterpret_cast<const uint32_t*>(sb + kCodes + 4 * (32 * q + 16 * mt + i16));
              bdw[mt][q] = *reinterpret_cast<const uint32_t*>(sb + kCodes + 256 + 4 * (32 * q + 16 * mt + i16));
            }
        }
#pragma unroll
        for (int p = 0; p < NB; ++p) {
          if (j0 + p >= je) break;
          u32x4 xa0 = xa[p][0], xa1 = xa[p][1];
          if constexpr (XLDS) {  // row i16 of block p: chunks 2g and 2g + 1 (G32: g and g + 4)
            const uint8_t* xb = xring + st * kXStage + p * 2048 + i16 * 128;
            xa0 = *reinterpret_cast<const u32x4*>(xb + 16 * ((G32 ? g : 2 * g) ^ (i16 & 7)));
            xa1 = *reinterpret_cast<const u32x4*>(xb + 16 * ((G32 ? g + 4 : 2 * g + 1) ^ (i16 & 7)));
          }
          const bf16x8 A0 = __builtin_bit_cast(bf16x8, BITS == 4 && !PAIRS ? to_pair_order(xa0) : xa0);
          const bf16x8 A1 = __builtin_bit_cast(bf16x8, BITS == 4 && !PAIRS ? to_pair_order(xa1) : xa1);
          if constexpr (G32) {
            // group size 32: A0/B0 hold K 8g .. 8g+7 of the block (group
            // 2(j0+p), the low half of the stage's scale dword p), A1/B1 K 32 +
            // 8g .. (group 2(j0+p) + 1, the high half): one MFMA per group
            const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
            const f32x4 xr0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, ones, zero4, 0, 0, 0);
            const f32x4 xr1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, ones, zero4, 0, 0, 0);
#pragma unroll
            for (int mt = 0; mt < NMAT; ++mt) {
              const int lr = 16 * mt + i16;
              const bf16x8 B0 = g32_operand<BITS>(sb, lr, 64 * p + 8 * g, kNibMask, kMagic);
              const bf16x8 B1 = g32_operand<BITS>(sb, lr, 64 * p + 32 + 8 * g, kNibMask, kMagic);
              const uint32_t sdwv = p ? sdw[mt][1] : sdw[mt][0];
              const uint32_t bdwv = p ? bdw[mt][1] : bdw[mt][0];
              const float s0 = __uint_as_float(sdwv << 16), s1 = __uint_as_float(sdwv & 0xffff0000u);
              const float b0 = a.b[mt] ? __uint_as_float(bdwv << 16) : 0.0f;
              const float b1 = a.b[mt] ? __uint_as_float(bdwv & 0xffff0000u) : 0.0f;
              const float bp0 = BITS == 8 ? b0 : b0 - 128.0f * s0, bp1 = BITS == 8 ? b1 : b1 - 128.0f * s1;
              const f32x4 c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, B0, zero4, 0, 0, 0);
              const f32x4 c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, B1, zero4, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[mt][r] = fmaf(s1, c1[r], fmaf(bp1, xr1[r], fmaf(s0, c0[r], fmaf(bp0, xr0[r], acc[mt][r]))));
            }
            continue;
          }
          f32x4 xr = {0.f, 0.f, 0.f, 0.f};
          xr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, ones, xr, 0, 0, 0);
          xr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, ones, xr, 0, 0, 0);
          // group of block j0+p, its dword in the stage (0 or 1) and half; with
          // four blocks a stage (2, 3, 4 bits: j0 a multiple of 4) both are
          // compile-time constants
          const int grp = (j0 + p) / gdiv;
          const int q = NB == 4 ? (p / gdiv) >> 1
                        : SREG  ? ((grp - g0) >> 1) - D
                                : grp / 2 - min((j0 / gdiv) / 2, G / 2 - 1);
          const int hsel = NB == 4 ? (p / gdiv) & 1 : SREG ? (grp - g0) & 1 : grp & 1;
#pragma unroll
          for (int mt = 0; mt < NMAT; ++mt) {
            const int lr = 16 * mt + i16;
            bf16x8 B0, B1;
            if constexpr (BITS == 4) {
              // 16 codes = bytes 32p + 8g .. +7 of the row: chunk 2p + g/2, half g%2
              const int c = 2 * p + (g >> 1);
              const u32x2 wq = *reinterpret_cast<const u32x2*>(sb + lr * 128 + 16 * (c ^ (lr & 7)) + 8 * (g & 1));
              B0 = __builtin_bit_cast(bf16x8, nibbles_to_bf16(wq.x, kNibMask, kMagic));
              B1 = __builtin_bit_cast(bf16x8, nibbles_to_bf16(wq.y, kNibMask, kMagic));
            } else if constexpr (BITS == 2 || BITS == 3 || BITS == 5) {
              // 16 codes = 2*BITS bytes at byte (8p + 2g)*BITS of the stage
              // row (even: at bit 0 or 16 of its dword), in the dwords from
              // there: dword D sits in chunk D/4
              constexpr int ND = BITS == 2 ? 1 : BITS == 3 ? 2 : 3;
              const int boff = (8 * p + 2 * g) * BITS;
              uint32_t wq[ND];
#pragma unroll
              for (int t = 0; t < ND; ++t) {
                const int D = (boff >> 2) + t;
                wq[t] = *reinterpret_cast<const uint32_t*>(sb + lr * 128 + 16 * ((D >> 2) ^ (lr & 7)) + 4 * (D & 3));
              }
              u32x4 lo, hi;
              qn_to_bf16<BITS>(wq, static_cast<uint32_t>((boff & 3) * 8), lo, hi);
              B0 = __builtin_bit_cast(bf16x8, lo);
              B1 = __builtin_bit_cast(bf16x8, hi);
            } else if constexpr (BITS == 6) {
              // 16 codes = 12 bytes, dwords 12p + 3g .. +2 of the stage row
              // (96 of its 128 bytes hold codes): dword D sits in chunk D/4
              uint32_t wq[3];
#pragma unroll
              for (int t = 0; t < 3; ++t) {
                const int D = 12 * p + 3 * g + t;
                wq[t] = *reinterpret_cast<const uint32_t*>(sb + lr * 128 + 16 * ((D >> 2) ^ (lr & 7)) + 4 * (D & 3));
              }
              u32x4 lo, hi;
              q6_to_bf16(wq[0], wq[1], wq[2], lo, hi);
              B0 = __builtin_bit_cast(bf16x8, lo);
              B1 = __builtin_bit_cast(bf16x8, hi);
            } else {
              // 16 codes = bytes 64p + 16g .. +15: chunk 4p + g
              const int c = 4 * p + g;
              const u32x4 wq = *reinterpret_cast<const u32x4*>(sb + lr * 128 + 16 * (c ^ (lr & 7)));
              const u32x2 p0 = bytes_to_bf16(wq.x), p1 = bytes_to_bf16(wq.y);
              const u32x2 p2 = bytes_to_bf16(wq.z), p3 = bytes_to_bf16(wq.w);
              B0 = __builtin_bit_cast(bf16x8, u32x4{p0.x, p0.y, p1.x, p1.y});
              B1 = __builtin_bit_cast(bf16x8, u32x4{p2.x, p2.y, p3.x, p3.y});
            }
            const uint32_t sdwv = q ? sdw[mt][1] : sdw[mt][0];
            const uint32_t bdwv = q ? bdw[mt][1] : bdw[mt][0];
            const float sc = __uint_as_float(hsel ? (sdwv & 0xffff0000u) : (sdwv << 16));
            const float bv = __uint_as_float(hsel ? (bdwv & 0xffff0000u) : (bdwv << 16));
            const float bi = SREG || a.b[mt] ? bv : 0.0f;  // (SREG: the registers hold 0 without biases)
            const float bp = BITS == 8 ? bi : bi - 128.0f * sc;  // 4, 6 bits: the operand is 128 + q
            f32x4 c4 = {0.f, 0.f, 0.f, 0.f};
            c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, B0, c4, 0, 0, 0);
            c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, B1, c4, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][r] = fmaf(sc, c4[r], fmaf(bp, xr[r], acc[mt][r]));
          }
        }
      };
      if constexpr (SREG) {
        constexpr int kUnroll = 8 / (NB / gdiv);  // stages after which D has advanced by a multiple of 4
        constexpr int kPer = 4 * kUnroll;         // stages per period of 32 groups
        for (int i0 = 0; jb + i0 * NB < je; i0 += kUnroll) {
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            const int j0 = jb + (i0 + u) * NB;
            if (j0 >= je) break;
            __builtin_amdgcn_sched_barrier(0);  // one stage at a time (registers)
            stage(j0, u & 1, u);
          }
          // after a period's last stage (its scales already moved out of the
          // registers): the next period's, awaited with the next stage
          if constexpr (SROLL)
            if ((i0 + kUnroll) % kPer == 0 && jb + (i0 + kUnroll) * NB < je) load_sreg((i0 + kUnroll) / kPer);
        }
      } else {
        for (int j0 = jb, st = 0; j0 < je; j0 += NB, st ^= 1) stage(j0, st, 0);
      }
      wait_vmcnt<0>();  // no DMA into this wave's ring outstanding
    }

    if constexpr (KSPLIT > 1) {
      // sum the K parts: the ring of the tile's first wave holds the partials
      __syncthreads();
      f32x4* red = reinterpret_cast<f32x4*>(lds + (wave - kp) * kWave);
      if (kp > 0)
#pragma unroll
        for (int mt = 0; mt < NMAT; ++mt) red[((kp - 1) * NMAT + mt) * 64 + lane] = acc[mt];
      __syncthreads();
      if (kp == 0)
        for (int q = 1; q < KSPLIT; ++q)
#pragma unroll
          for (int mt = 0; mt < NMAT; ++mt) acc[mt] += red[((q - 1) * NMAT + mt) * 64 + lane];
      __syncthreads();
    }
    if (valid && kp == 0) {
      // the output-row loads have landed on every path (a wave without K work
      // skipped the loop's final wait): no store below waits for the one
      // before it (stores and loads share one counter)
      wait_vmcnt<0>();
      const int col = n0 + (GLU && a.out_pairs ? (i16 & ~7) | pair_pos(i16 & 7) : i16);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r;
        if (m >= mcount || col >= a.N) continue;  // (columns past N: a partial last tile)
        uint16_t* orp = a.out + static_cast<int64_t>(orow[r]) * a.N + col;
        // the bias is added to the bf16 projection output
        if constexpr (GLU) {
          float gg = bfr(acc[0][r]), uu = bfr(acc[1][r]);
          if (a.lb[0]) gg = bfr(gg + lbv[0]);
          if (a.lb[1]) uu = bfr(uu + lbv[1]);
          *orp = f2bf(glu_act(a.act, gg, uu, silu(gg)));
        } else {
#pragma unroll
          for (int mt = 0; mt < NMAT; ++mt)
            orp[16 * mt] = f2bf(a.lb[0] ? bfr(acc[mt][r]) + lbv[mt] : acc[mt][r]);
        }
      }
    }
  }
}

// relu_squared (include/mlx-lm/common/activations.h:45-55): bf16(max(v, 0)^2).
// Runs in place (in == out) in moe_switch_mlp_relu2, so the pointers are not
// __restrict__; each element is read and written by the same thread.
__global__ void relu2_kernel(const uint16_t* in, int64_t n, uint16_t* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) {
    const float r = fmaxf(bf2f(in[i]), 0.0f);
    out[i] = f2bf(r * r);
  }
}

// y[t] = bf16(x[t] . dequant(w)^T) (+ SwitchLinear bias) for one quantized
// row w [1, K] (a projection with N = 1: the quantized shared-expert gate).
// One wave per token; lane l takes the 8 K values 8l + 512j of each step,
// fp32 products with s*q + b of their group, summed over the wave.
template <int BITS>
__global__ __launch_bounds__(256) void qrow_kernel(const uint16_t* __restrict__ x, int64_t T, int K,
                                                   const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                                   const uint16_t* __restrict__ b, int gs,
                                                   const uint16_t* __restrict__ lb, uint16_t* __restrict__ y) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* xr = x + t * K;
  float acc = 0.0f;
  for (int c0 = 8 * lane; c0 < K; c0 += 512) {
    const u32x4 xv = *reinterpret_cast<const u32x4*>(xr + c0);
    const int g = c0 / gs;
    const float sc = bf2f(s[g]), bi = b ? bf2f(b[g]) : 0.0f;
    uint32_t q[8];
    if constexpr (BITS == 4) {
      const uint32_t wd = w[c0 / 8];
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = (wd >> (4 * j)) & 15u;
    } else if constexpr (BITS != 8) {
      // 8 codes = 8*BITS bits at bit BITS*c0 (a multiple of 8): within two
      // words (the second clamped to the row: a field that ends in the first
      // word does not use it)
      const int64_t bit = static_cast<int64_t>(BITS) * c0;
      const int64_t wi = bit >> 5, last = static_cast<int64_t>(K) * BITS / 32 - 1;
      const uint64_t v = (static_cast<uint64_t>(w[wi + 1 <= last ? wi + 1 : last]) << 32 | w[wi]) >> (bit & 31);
#pragma unroll
      for (int j = 0; j < 8; ++j) q[j] = static_cast<uint32_t>(v >> (BITS * j)) & ((1u << BITS) - 1u);
    } else {
      const uint32_t w0 = w[c0 / 4], w1 = w[c0 / 4 + 1];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        q[j] = (w0 >> (8 * j)) & 255u;
        q[4 + j] = (w1 >> (8 * j)) & 255u;
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float xj = __uint_as_float(j & 1 ? xv[j >> 1] & 0xffff0000u : xv[j >> 1] << 16);
      acc += xj * (sc * static_cast<float>(q[j]) + bi);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) y[t] = f2bf(lb ? bfr(acc) + bf2f(lb[0]) : acc);
}

__global__ void swiglu_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                              int64_t n, uint16_t* __restrict__ h) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) h[i] = f2bf(silu(bf2f(g[i])) * bf2f(u[i]));
}

// GPT-OSS's clipped SwiGLU (gptoss.cpp:50-58) of x_linear and x_glu.
__global__ void gptoss_swiglu_kernel(const uint16_t* __restrict__ xl, const uint16_t* __restrict__ xg,
                                     int64_t n, uint16_t* __restrict__ h) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) h[i] = f2bf(gptoss_glu(bf2f(xl[i]), bf2f(xg[i])));
}

// y[t] = bf16(sum_j scores[t, j] * Y[row(t, j)] (+ gate * Ys[t])), 8 columns
// per thread.  KC > 0: k == KC at compile time, so the k row indices and the
// k row loads are all issued before the sums (in j order); KC == 0: any k.
template <int KC>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ Y,
                                                      const int32_t* __restrict__ inv_perm,
                                                      const float* __restrict__ scores, int64_t T, int k, int H,
                                                      const uint16_t* __restrict__ Ys,
                                                      const uint16_t* __restrict__ sgl, uint16_t* __restrict__ y) {
  const int cpr = H >> 3;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= T * cpr) return;
  const int64_t t = idx / cpr;
  const int c = static_cast<int>(idx % cpr) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto add = [&](float s, const u32x4& v) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += s * __uint_as_float(v[q] << 16);
      acc[2 * q + 1] += s * __uint_as_float(v[q] & 0xffff0000u);
    }
  };
  if constexpr (KC > 0) {
    int64_t row[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) row[j] = inv_perm ? inv_perm[t * KC + j] : t * KC + j;
    u32x4 v[KC];
    float sc[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(Y + row[j] * H + c));  // read once
      sc[j] = scores[t * KC + j];
    }
#pragma unroll
    for (int j = 0; j < KC; ++j) add(sc[j], v[j]);
  } else {
    for (int j = 0; j < k; ++j) {
      const int64_t f = t * k + j;
      const int64_t row = inv_perm ? inv_perm[f] : f;
      add(scores[f], *reinterpret_cast<const u32x4*>(Y + row * H + c));
    }
  }
  if (Ys) {
    const float gate = sgl ? 1.0f / (1.0f + __expf(-bf2f(sgl[t]))) : 1.0f;
    add(gate, *reinterpret_cast<const u32x4*>(Ys + t * H + c));
  }
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(y + t * H + c));
}

template <int BITS, bool GLU, int GS, bool PAIRS, bool SREG, bool DUO = false, bool SROLL = false>
int launch_ks(const GQArgs& a, int ksplit, int tiles16, int slots, hipStream_t stream) {
  const char* name = GLU ? "qmm_gate_up_swiglu" : "qmm_down";
  const int64_t tiles = static_cast<int64_t>(tiles16) * slots;
  // ksplit: 4 or 1 (gqmm_ksplit)
  if (DUO && ksplit == 4) {
    MOE_LAUNCH(name, (grouped_qmm_kernel<BITS, GLU, 4, GS, PAIRS, SREG, DUO>), dim3(static_cast<unsigned>(tiles)),
               dim3(256), 0, stream, a, tiles16, slots);
  } else if (SREG || DUO || ksplit == 1) {  // (DUO: no K split, or the four-way split above)
    // whole-K waves: the four waves of a workgroup share one expert when its
    // tiles come in fours (then the activations go through the shared ring)
    if (tiles16 % 4 == 0)
      MOE_LAUNCH(name, (grouped_qmm_kernel<BITS, GLU, 1, GS, PAIRS, SREG, DUO, true, SROLL>),
                 dim3(static_cast<unsigned>(tiles / 4)), dim3(256), 0, stream, a, tiles16, slots);
    else
      MOE_LAUNCH(name, (grouped_qmm_kernel<BITS, GLU, 1, GS, PAIRS, SREG, DUO, false, SROLL>),
                 dim3(static_cast<unsigned>((tiles + 3) / 4)), dim3(256), 0, stream, a, tiles16, slots);
  } else if constexpr (!SREG && !DUO) {
    MOE_LAUNCH(name, (grouped_qmm_kernel<BITS, GLU, 4, GS, PAIRS, false>), dim3(static_cast<unsigned>(tiles)),
               dim3(256), 0, stream, a, tiles16, slots);
  }
  return launch_status("grouped_qmm");
}

// Groups of one wave's K part (the kernel's split: whole stages of NB blocks)
int part_groups(int K, int bits, int gs, int ksplit) {
  const int NB = bits <= 4 ? 4 : 2, KB = K / 64;
  const int per = ((KB + ksplit - 1) / ksplit + NB - 1) / NB * NB;
  return per / (gs / 64);
}

// Scales in registers: gate|up, and down when its K part spans at least 32
// groups (measured slower for Qwen3's 12-group rows, whose stage DMA of scales
// touches few lines); whole-K waves only (measured: at T = 1 with four parts
// slower), the part's scales 16 bytes per lane per 32 groups, every
// part starting at an even group (its dwords are whole pairs of groups: in the
// row or unused).
bool gqmm_sreg(const moe_qweight* w0, bool glu, int ksplit) {
  const int pg = part_groups(w0->K, w0->bits, w0->group_size, ksplit);
  return (glu || pg >= 32) && ksplit == 1 && pg % 2 == 0;
}

// mode: 1 = scales in registers, 3 = the same over more than 32 groups
// (reloaded per 32), 2 = two tiles per wave (down), 4 / 5 = two tiles per wave
// with scales in registers (/ reloaded), else 0
template <int BITS, bool GLU, int GS, bool PAIRS>
int launch_mode(const GQArgs& a, int ksplit, int mode, int tiles16, int slots, hipStream_t stream) {
  if constexpr (BITS == 2 || BITS == 3 || BITS == 5 || GS == 32) {
    (void)mode;  // staged scales, one tile per wave (grouped_qmm picks mode 0 for these and for group size 32)
    return launch_ks<BITS, GLU, GS, PAIRS, false>(a, ksplit, tiles16, slots, stream);
  } else {
    if constexpr (GLU) {
      if (mode == 1) return launch_ks<BITS, GLU, GS, PAIRS, true>(a, ksplit, tiles16, slots, stream);
      if (mode == 3) return launch_ks<BITS, GLU, GS, PAIRS, true, false, true>(a, ksplit, tiles16, slots, stream);
    } else {
      if (mode == 2) return launch_ks<BITS, GLU, GS, PAIRS, false, true>(a, ksplit, tiles16, slots, stream);
      if (mode == 4) return launch_ks<BITS, GLU, GS, PAIRS, true, true>(a, ksplit, tiles16, slots, stream);
      if (mode == 5) return launch_ks<BITS, GLU, GS, PAIRS, true, true, true>(a, ksplit, tiles16, slots, stream);
    }
    return launch_ks<BITS, GLU, GS, PAIRS, false>(a, ksplit, tiles16, slots, stream);
  }
}

// One token (T = 1): the down projection of its k expert rows and the
// weighted combine (plus the shared expert) in one launch, so no second
// dependent kernel runs after down.  A workgroup owns 8 output columns
// n0 .. n0+7 for every expert: wave s takes slot s (the token's experts in
// sorted order, slot records as the grouped kernel reads them) over the whole
// of K.  Each load instruction covers whole lines: lane (row r = lane / 8,
// part c = lane % 8) reads 16 bytes of codes at c in every 128-byte block of
// row n0 + r (32 4-bit or 16 8-bit codes), with the matching activations,
// and sums s * (x . q) + b * sum(x) per block in fp32, every load issued
// before the first sum.  The 8 lanes of a row add their sums in a fixed
// order; each expert's output is rounded to bf16 (plus its SwitchLinear bias,
// rounded again), and the combine then adds score_j * Y_j over the pairs j in
// flat order and the gated shared expert, rounding once -- the arithmetic of
// combine_kernel, so only the GEMV's summation order differs from the
// two-launch path.
struct DCArgs {
  const uint16_t* h;        // [k, K] expert inputs in sorted order, natural K order
  const int32_t* perm;      // sorted position -> flat pair index
  const int32_t* active;    // [k][4] slot records {expert, sorted position, 1, 0}
  const float* scores;      // [k] flat pair order
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;        // or NULL
  const uint16_t* lb;       // [E, N] or NULL
  const uint16_t* Ys;       // [N] or NULL
  const uint16_t* sgl;      // [1] or NULL
  uint16_t* out;            // [N]
  int k, blocks, N, K, gs;  // blocks: 128-byte code blocks per row
};

// NB: blocks per row rounded up (2 or 4: every load of a lane is in
// flight at once); MAXT: 512 threads (k <= 8, 256 VGPRs a wave) or 1024
template <int BITS, int NB, int MAXT>
__global__ __launch_bounds__(MAXT) void down_combine_one_kernel(DCArgs a) {
  constexpr int kVals = 128 * 8 / BITS;  // K values per 128-byte code block
  constexpr int kLaneVals = kVals / 8;   // per lane (16 code bytes)
  __shared__ float part[16][8];               // slot -> column
  __shared__ int slot_of[16], expert_of[16];  // pair -> slot, slot -> expert
  __shared__ float score_of[16];              // pair -> score
  const int lane = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 8;
  const int r = lane >> 3, c = lane & 7;
  // the combine's inputs, loaded first (their latency overlaps the GEMV's):
  // thread t < k, as slot t and as pair t; threads 0 .. 7 the shared
  // expert's columns
  if (threadIdx.x < a.k) {
    const int t = threadIdx.x;
    slot_of[a.perm[t]] = t;
    expert_of[t] = a.active[4 * t];
    score_of[t] = a.scores[t];
  }
  float ys = 0.0f, gate = 1.0f;
  if (threadIdx.x < 8 && a.Ys) {
    if (a.sgl) gate = 1.0f / (1.0f + __expf(-bf2f(a.sgl[0])));
    ys = bf2f(a.Ys[n0 + threadIdx.x]);
  }
  float acc = 0.0f;
  {
    const int4 rec = reinterpret_cast<const int4*>(a.active)[sl];
    const int e = rec.x, pos = rec.y;
    const int K = a.K, G = K / a.gs;
    const int64_t row = static_cast<int64_t>(e) * a.N + n0 + r;
    const uint16_t* xr = a.h + static_cast<int64_t>(pos) * K + kLaneVals * c;
    const uint8_t* wr = reinterpret_cast<const uint8_t*>(a.w) + row * (static_cast<int64_t>(K) * BITS / 8) + 16 * c;
    const uint16_t* sr = a.s + row * G;
    const uint16_t* br = a.b ? a.b + row * G : nullptr;
    u32x4 cv[NB];
    u32x4 xv[NB][kLaneVals / 8];
    float sv[NB], bv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (i < a.blocks) {
        cv[i] = *reinterpret_cast<const u32x4*>(wr + 128 * i);
#pragma unroll
        for (int v = 0; v < kLaneVals / 8; ++v) xv[i][v] = *reinterpret_cast<const u32x4*>(xr + kVals * i + 8 * v);
        const int g = (kVals * i + kLaneVals * c) / a.gs;  // the lane's values lie in one group
        sv[i] = bf2f(sr[g]);
        bv[i] = br ? bf2f(br[g]) : 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (i < a.blocks) {
        float dot = 0.0f, sx = 0.0f;
        if constexpr (BITS == 4) {
          // two K values per instruction: each pair of codes becomes the bf16
          // pair (128 + q) (exact), dotted with the activation pair in fp32
          // (v_dot2c_f32_bf16), and the pair's sum of x likewise against ones;
          // acc = s * dot + (b - 128 s) * sx
          const bf16x2 ones2 = __builtin_bit_cast(bf16x2, 0x3f803f80u);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t w = cv[i][d], hw = w >> 4;  // codes 8d .. 8d+7 of the lane's 32
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              // byte 0: code 8d+2j (low nibble of byte j), byte 2: code 8d+2j+1
              const uint32_t sel = 0x0c040c00u + 0x00010001u * static_cast<uint32_t>(j);
              const uint32_t qp = (__builtin_amdgcn_perm(hw, w, sel) & 0x000f000fu) | 0x43004300u;
              const bf16x2 xp2 = as_bf16x2(xv[i][d][j]);  // x 8d+2j, 8d+2j+1
              dot = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(qp), xp2, dot, false);
              sx = __builtin_amdgcn_fdot2_f32_bf16(xp2, ones2, sx, false);
            }
          }
          acc = __builtin_fmaf(sv[i], dot, __builtin_fmaf(bv[i] - 128.0f * sv[i], sx, acc));
        } else {
#pragma unroll
          for (int v = 0; v < kLaneVals; ++v) {
            const uint32_t xw = xv[i][v >> 3][(v >> 1) & 3];
            const float x = __uint_as_float(v & 1 ? xw & 0xffff0000u : xw << 16);
            const uint32_t cw = cv[i][(v * BITS) >> 5];
            const uint32_t q = (cw >> ((v * BITS) & 31)) & ((1u << BITS) - 1u);
            dot = __builtin_fmaf(x, static_cast<float>(q), dot);
            sx += x;
          }
          acc = __builtin_fmaf(sv[i], dot, __builtin_fmaf(bv[i], sx, acc));
        }
      }
    }
  }
  // the 8 lanes of a row, then one value per (slot, column)
  acc += __shfl_xor(acc, 1);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 4);
  if (c == 0) part[sl][r] = acc;
  __syncthreads();
  if (threadIdx.x < 8) {  // one column each (the lanes that loaded the shared expert's)
    const int cc = threadIdx.x, n = n0 + cc;
    float lbv[16];
#pragma unroll
    for (int t = 0; t < 16; ++t)  // the experts' SwitchLinear biases of this column, all loads first
      lbv[t] = a.lb && t < a.k ? bf2f(a.lb[static_cast<int64_t>(expert_of[t]) * a.N + n]) : 0.0f;
    float o = 0.0f;
    for (int j = 0; j < a.k; ++j) {  // pairs in flat order, as combine_kernel
      const int sj = slot_of[j];
      float y = bfr(part[sj][cc]);
      if (a.lb) {
        float bb = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; ++t) bb = t == sj ? lbv[t] : bb;
        y = bfr(y + bb);
      }
      o += score_of[j] * y;
    }
    if (a.Ys) o += gate * ys;
    a.out[n] = f2bf(o);
  }
}

template <int BITS, bool GLU, bool PAIRS>
int launch_gs(const GQArgs& a, int ksplit, int mode, int tiles16, int slots, hipStream_t stream) {
  return a.gs == 64    ? launch_mode<BITS, GLU, 64, PAIRS>(a, ksplit, mode, tiles16, slots, stream)
         : a.gs == 128 ? launch_mode<BITS, GLU, 128, PAIRS>(a, ksplit, mode, tiles16, slots, stream)
                       : launch_mode<BITS, GLU, 32, PAIRS>(a, ksplit, mode, tiles16, slots, stream);
}

// gate|up of one token that routes it in the kernel (4-bit, x in pair K
// order, K split over the four waves of a workgroup: one 16-row tile each)
template <int GS>
int launch_routed(const GQArgs& a, int tiles16, int slots, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(tiles16) * slots));
  const int vpl = (a.ra.E + 63) / 64;
  if (vpl <= 1)
    MOE_LAUNCH("qmm_gate_up_swiglu", (grouped_qmm_kernel<4, true, 4, GS, true, false, false, false, false, 1>), grid,
               dim3(256), 0, stream, a, tiles16, slots);
  else if (vpl <= 2)
    MOE_LAUNCH("qmm_gate_up_swiglu", (grouped_qmm_kernel<4, true, 4, GS, true, false, false, false, false, 2>), grid,
               dim3(256), 0, stream, a, tiles16, slots);
  else if (vpl <= 4)
    MOE_LAUNCH("qmm_gate_up_swiglu", (grouped_qmm_kernel<4, true, 4, GS, true, false, false, false, false, 4>), grid,
               dim3(256), 0, stream, a, tiles16, slots);
  else
    MOE_LAUNCH("qmm_gate_up_swiglu", (grouped_qmm_kernel<4, true, 4, GS, true, false, false, false, false, 8>), grid,
               dim3(256), 0, stream, a, tiles16, slots);
  return launch_status("grouped_qmm");
}

}  // namespace

// Validates one stacked quantized projection for the grouped kernel.
int qweight_check(const moe_qweight* w) {
  if (!w || !w->w || !w->scales) return MOE_E_INVALID_ARG;
  if (w->experts <= 0 || w->N <= 0 || w->K <= 0) return MOE_E_INVALID_ARG;
  if (w->bits < 2 || w->bits > 8 || w->bits == 7) return MOE_E_UNSUPPORTED;
  // 3 and 5 bits: rows of whole 16-byte units (the stage DMA moves 16-byte chunks of a row)
  if ((w->bits == 3 || w->bits == 5) && w->K % 128 != 0) return MOE_E_UNSUPPORTED;
  if (w->group_size != 32 && w->group_size != 64 && w->group_size != 128) return MOE_E_UNSUPPORTED;
  if (w->K % w->group_size != 0) return MOE_E_UNSUPPORTED;
  // scales and biases are read as aligned dwords (two groups each)
  if ((w->K / w->group_size) % 2 != 0) return MOE_E_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(w->w) & 15u) != 0) return MOE_E_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(w->scales) & 3u) != 0) return MOE_E_UNSUPPORTED;
  if (w->biases && (reinterpret_cast<uintptr_t>(w->biases) & 3u) != 0) return MOE_E_UNSUPPORTED;
  return MOE_OK;
}

// K-split threshold of the grouped kernel, in expected busy 16-row tiles
constexpr double kGqmmSplit4Tiles = 1536;

// K split per tile (4 waves or none) from the tiles that expect work: the
// grid covers `slots` experts, of which about E (1 - (1 - 1/E)^P) are routed
// a token (the count itself is known only on the device).  Below the
// threshold four waves share each tile's K; from it on whole-K waves, whose
// workgroups serve one expert with a shared activation ring.  (A two-way
// split between 1536 and 4096 tiles measured slower than whole-K waves at
// every size tried: Qwen3 T = 4 46.7 -> 44.2 us, T = 6 51.4 -> 48.4, T = 16
// 78.6 -> 75.0; Mixtral T = 16 392 -> 341; DeepSeek-V3 T = 1 101.6 -> 95.5.)
int gqmm_ksplit(int64_t P, int slots, const moe_qweight* w0) {
  const double E = w0->experts;
  // (one expert: every slot is a record of its rows, all busy)
  const double busy =
      (E == 1 ? slots : std::min<double>(slots, E * (1.0 - std::pow(1.0 - 1.0 / E, static_cast<double>(P))))) *
      (w0->N / 16);
  return busy < kGqmmSplit4Tiles ? 4 : 1;
}

// Workgroups the large-bucket GEMM gets at most: P/128 token tiles of 128
// rows plus two shorter ones per non-empty expert, times the column tiles
// (GLU: 128 output columns each, else 256).
constexpr int kPrefillMinWgs = 64;
int64_t prefill_wgs(int64_t P, int slots, const moe_qweight* w0, bool glu) {
  const int64_t ntiles = glu ? (w0->N + 127) / 128 : (w0->N + 255) / 256;
  return (P / 128 + 2 * std::min<int64_t>(slots, P)) * ntiles;
}

// The large-bucket GEMM from 16 rows per non-empty expert on average (Qwen3
// shape, measured: at 8 rows both paths take the same time, at 16 the GEMM
// takes 0.6x the per-16-row kernel's, at 64 rows 0.42x), unless it would get
// so few workgroups that most CUs idle (a shared expert at a few dozen tokens:
// one expert's token tile times a handful of column tiles).
bool use_prefill(int64_t P, int slots, const moe_qweight* w0, const moe_qweight* w1) {
  return P >= 16 * static_cast<int64_t>(slots) && prefill_supported(w0, w1) &&
         prefill_wgs(P, slots, w0, w1 != nullptr) >= kPrefillMinWgs;
}

bool gate_up_route_fits(int64_t P, int slots, const PrefillScratch& pf, const moe_qweight* gate,
                        const moe_qweight* up, const moe_router_params& rp, int ks) {
  if (!gate || !up || pf.gemv_only || !pf.xp || !pf.xp_ready) return false;
  if (gate->bits != 4 || (gate->group_size != 64 && gate->group_size != 128)) return false;
  const int E = rp.num_experts, k = rp.top_k;
  if (P != k || slots != k || k > 16 || E > 512 || E != gate->experts) return false;
  // the partial sums of the logits: every load of a lane at once (token_logits_from_partials)
  if (ks < 1 || ks * ((E + 63) / 64) > 32) return false;
  if (use_prefill(P, slots, gate, up)) return false;
  const int ksplit = gqmm_ksplit(P, slots, gate);
  return ksplit == 4 && !gqmm_sreg(gate, true, ksplit);
}

int grouped_qmm(const uint16_t* x, const int32_t* row_in, const int32_t* row_out,
                const int32_t* offsets, const int32_t* active, const int32_t* num_active,
                int slots, int64_t P, const PrefillScratch* pf, const moe_qweight* w0,
                const moe_qweight* w1, uint16_t* out, hipStream_t stream) {
  int st = qweight_check(w0);
  if (st != MOE_OK) return st;
  if (w1) {
    st = qweight_check(w1);
    if (st != MOE_OK) return st;
    if (w0->N % 16 != 0) return MOE_E_UNSUPPORTED;  // gate|up: whole 16-row tiles (any N without GLU)
    if (w1->N != w0->N || w1->K != w0->K || w1->bits != w0->bits || w1->group_size != w0->group_size ||
        w1->experts != w0->experts)
      return MOE_E_INVALID_ARG;
  }
  if (!x || !offsets || !out || slots < 0) return MOE_E_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return MOE_E_UNSUPPORTED;
  if (slots == 0) return MOE_OK;
  // Large buckets (prefill): the LDS-staged GEMM.  Small buckets (decode):
  // the per-16-row kernel below.
  if (pf && !pf->gemv_only && use_prefill(P, slots, w0, w1))
    return grouped_gemm_prefill(x, row_in, row_out, *pf, offsets, w0->experts, P, slots, w0, w1, out, stream);
  // 4-bit: activations already in pair K order (gate|up: the copy the router
  // projection wrote; down: h written in that order by gate|up)
  const bool pairs = w0->bits == 4 && pf && (w1 ? pf->xp && pf->xp_ready : pf->in_p8);
  GQArgs a{};
  a.x = pairs && w1 ? pf->xp : x;
  a.out_pairs = w1 && pf && pf->out_p8 ? 1 : 0;
  a.row_in = row_in;
  a.row_out = row_out;
  a.offsets = offsets;
  a.active = active;
  a.num_active = num_active;
  // one expert's rows spread evenly over the slots, a multiple of 16 rows
  // each (their records follow from P)
  a.one_rows = pf && pf->gemv_only ? static_cast<int>(P) : 0;
  if (a.one_rows > 0) {
    if (w0->experts != 1 || slots != one_expert_slots(P)) return MOE_E_INVALID_ARG;
    a.one_per = static_cast<int>((P + slots - 1) / slots + 15) / 16 * 16;
  }
  a.w[0] = w0->w;
  a.s[0] = w0->scales;
  a.b[0] = w0->biases;
  a.lb[0] = w0->linear_bias;
  if (w1) {
    a.w[1] = w1->w;
    a.s[1] = w1->scales;
    a.b[1] = w1->biases;
    a.lb[1] = w1->linear_bias;
  }
  a.N = w0->N;
  a.K = w0->K;
  a.gs = w0->group_size;
  a.out = out;
  a.act = w1 && pf ? pf->act : MOE_ACT_SWIGLU;

  const int ksplit = gqmm_ksplit(P, slots, w0);
  // 2, 3 and 5 bits, and group size 32: one tile per wave, scales staged with the codes
  const bool plain = w0->bits == 2 || w0->bits == 3 || w0->bits == 5 || w0->group_size == 32;
  const bool sreg = !plain && gqmm_sreg(w0, w1 != nullptr, ksplit);
  // down: two 16-row tiles per wave without a K split (T = 8, 64: -9 %, -21 %) and with the four-way
  // split (T = 1: K = 768 is 12 blocks, so one wave in four has none; -2 %)
  const bool duo = !plain && !w1 && (ksplit == 1 || ksplit == 4) && a.N % 32 == 0;
  if (duo) {
    const int64_t rows16 = 16;
    a.w[1] = w0->w + rows16 * w0->K * w0->bits / 32;
    a.s[1] = w0->scales + rows16 * (w0->K / w0->group_size);
    a.b[1] = w0->biases ? w0->biases + rows16 * (w0->K / w0->group_size) : nullptr;
  }
  const bool roll = !plain && part_groups(w0->K, w0->bits, w0->group_size, ksplit) > 32;
  const int mode = duo ? (sreg ? (roll ? 5 : 4) : 2) : sreg && w1 ? (roll ? 3 : 1) : 0;
  const int tiles16 = duo ? a.N / 32 : (a.N + 15) / 16;  // tiles of one wave (per K part)
  const int64_t tiles = static_cast<int64_t>(tiles16) * slots;
  if (tiles > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  if (pf && pf->route) {  // one token, routed by the gate|up kernel itself
    const FusedRoute& fr = *pf->route;
    const moe_router_params& rp = fr.params;
    if (!w1 || !gate_up_route_fits(P, slots, *pf, w0, w1, rp, fr.ks) || !fr.part || !fr.logits_out || !fr.inds ||
        !fr.scores || !fr.o.offsets || !fr.o.active)
      return MOE_E_INVALID_ARG;
    a.rpart = fr.part;
    a.rks = fr.ks;
    a.rbias = fr.rbias;
    a.rlogits = fr.logits_out;
    a.ra = RouteArgs{nullptr, fr.score_bias, fr.inds, fr.scores, 1, rp.num_experts, rp.top_k, rp.variant,
                     rp.norm_topk_prob, rp.n_group, rp.topk_group, rp.routed_scaling_factor};
    a.rbo = fr.o;
    return a.gs == 64 ? launch_routed<64>(a, tiles16, slots, stream) : launch_routed<128>(a, tiles16, slots, stream);
  }
  if (w0->bits == 4) {
    if (pairs)
      return w1 ? launch_gs<4, true, true>(a, ksplit, mode, tiles16, slots, stream)
                : launch_gs<4, false, true>(a, ksplit, mode, tiles16, slots, stream);
    return w1 ? launch_gs<4, true, false>(a, ksplit, mode, tiles16, slots, stream)
              : launch_gs<4, false, false>(a, ksplit, mode, tiles16, slots, stream);
  }
  if (w0->bits == 6)
    return w1 ? launch_gs<6, true, false>(a, ksplit, mode, tiles16, slots, stream)
              : launch_gs<6, false, false>(a, ksplit, mode, tiles16, slots, stream);
  if (w0->bits == 2)
    return w1 ? launch_gs<2, true, false>(a, ksplit, mode, tiles16, slots, stream)
              : launch_gs<2, false, false>(a, ksplit, mode, tiles16, slots, stream);
  if (w0->bits == 3)
    return w1 ? launch_gs<3, true, false>(a, ksplit, mode, tiles16, slots, stream)
              : launch_gs<3, false, false>(a, ksplit, mode, tiles16, slots, stream);
  if (w0->bits == 5)
    return w1 ? launch_gs<5, true, false>(a, ksplit, mode, tiles16, slots, stream)
              : launch_gs<5, false, false>(a, ksplit, mode, tiles16, slots, stream);
  return w1 ? launch_gs<8, true, false>(a, ksplit, mode, tiles16, slots, stream)
            : launch_gs<8, false, false>(a, ksplit, mode, tiles16, slots, stream);
}


int relu_squared(const uint16_t* in, int64_t n, uint16_t* out, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!in || !out))) return MOE_E_INVALID_ARG;
  if (n == 0) return MOE_OK;
  MOE_LAUNCH("relu_squared", relu2_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, in,
             n, out);
  return launch_status("relu_squared");
}

int qrow(const uint16_t* x, int64_t T, const moe_qweight* w, uint16_t* y, hipStream_t stream) {
  int st = qweight_check(w);
  if (st != MOE_OK) return st;
  if (w->experts != 1 || w->N != 1 || T < 0 || (T > 0 && (!x || !y))) return MOE_E_INVALID_ARG;
  if (w->K % 8 != 0 || (reinterpret_cast<uintptr_t>(x) & 15u)) return MOE_E_UNSUPPORTED;
  if (T == 0) return MOE_OK;
  if ((T + 3) / 4 > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>((T + 3) / 4));
  if (w->bits == 4)
    MOE_LAUNCH("shared_gate", qrow_kernel<4>, grid, dim3(256), 0, stream, x, T, w->K, w->w, w->scales, w->biases,
               w->group_size, w->linear_bias, y);
  else if (w->bits == 2)
    MOE_LAUNCH("shared_gate", qrow_kernel<2>, grid, dim3(256), 0, stream, x, T, w->K, w->w, w->scales, w->biases,
               w->group_size, w->linear_bias, y);
  else if (w->bits == 3)
    MOE_LAUNCH("shared_gate", qrow_kernel<3>, grid, dim3(256), 0, stream, x, T, w->K, w->w, w->scales, w->biases,
               w->group_size, w->linear_bias, y);
  else if (w->bits == 5)
    MOE_LAUNCH("shared_gate", qrow_kernel<5>, grid, dim3(256), 0, stream, x, T, w->K, w->w, w->scales, w->biases,
               w->group_size, w->linear_bias, y);
  else if (w->bits == 6)
    MOE_LAUNCH("shared_gate", qrow_kernel<6>, grid, dim3(256), 0, stream, x, T, w->K, w->w, w->scales, w->biases,
               w->group_size, w->linear_bias, y);
  else
    MOE_LAUNCH("shared_gate", qrow_kernel<8>, grid, dim3(256), 0, stream, x, T, w->K, w->w, w->scales, w->biases,
               w->group_size, w->linear_bias, y);
  return launch_status("qrow");
}

int swiglu(const uint16_t* g, const uint16_t* u, int64_t n, uint16_t* h, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!g || !u || !h))) return MOE_E_INVALID_ARG;
  if (n == 0) return MOE_OK;
  MOE_LAUNCH("swiglu", swiglu_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     stream, g, u, n, h);
  return launch_status("swiglu");
}

int gptoss_swiglu(const uint16_t* xl, const uint16_t* xg, int64_t n, uint16_t* h, hipStream_t stream) {
  if (n < 0 || (n > 0 && (!xl || !xg || !h))) return MOE_E_INVALID_ARG;
  if (n == 0) return MOE_OK;
  if ((n + 255) / 256 > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  MOE_LAUNCH("gptoss_swiglu", gptoss_swiglu_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
             stream, xl, xg, n, h);
  return launch_status("gptoss_swiglu");
}

bool down_combine_one_fits(const moe_qweight* w, int k) {
  if (!w || k < 1 || k > 16 || (w->bits != 4 && w->bits != 8)) return false;
  const int vals = 128 * 8 / w->bits;  // K values per 128-byte code block
  // whole blocks, and a lane's values (an eighth of a block) inside one group
  if (w->N % 8 != 0 || w->K % vals != 0 || w->group_size % (vals / 8) != 0) return false;
  const int blocks = w->K / vals;
  // at most 4 blocks (K <= 1024 at 4 bits): its VALU dot products cost more
  // than the combine launch they save beyond that (DeepSeek-V3's down, K =
  // 2048 and 7168 columns, measured 26 -> 49 us)
  return blocks <= 4;
}

int down_combine_one(const uint16_t* h, const int32_t* perm, const int32_t* active, const float* scores, int k,
                     const moe_qweight* w, const uint16_t* Ys, const uint16_t* sgl, uint16_t* out,
                     hipStream_t stream) {
  if (!h || !perm || !active || !scores || !out || !down_combine_one_fits(w, k)) return MOE_E_INVALID_ARG;
  if ((reinterpret_cast<uintptr_t>(h) & 15u) || (reinterpret_cast<uintptr_t>(w->w) & 15u)) return MOE_E_UNSUPPORTED;
  const int blocks = w->K / (128 * 8 / w->bits);
  DCArgs a{h, perm, active, scores, w->w, w->scales, w->biases, w->linear_bias, Ys, sgl, out,
           k, blocks, w->N, w->K, w->group_size};
  const dim3 grid(w->N / 8), block(64 * k);
#define MOE_DC(BITS, NB, MAXT) \
  MOE_LAUNCH("qmm_down_combine", (down_combine_one_kernel<BITS, NB, MAXT>), grid, block, 0, stream, a)
  if (w->bits == 4) {
    if (k > 8) {
      if (blocks <= 2) MOE_DC(4, 2, 1024); else MOE_DC(4, 4, 1024);
    } else if (blocks <= 2) MOE_DC(4, 2, 512); else MOE_DC(4, 4, 512);
  } else {
    if (k > 8) {
      if (blocks <= 2) MOE_DC(8, 2, 1024); else MOE_DC(8, 4, 1024);
    } else if (blocks <= 2) MOE_DC(8, 2, 512); else MOE_DC(8, 4, 512);
  }
#undef MOE_DC
  return launch_status("down_combine_one");
}

int combine(const uint16_t* Y, const int32_t* inv_perm, const float* scores, int64_t T, int k,
            int H, const uint16_t* Ys, const uint16_t* sgl, uint16_t* y, hipStream_t stream) {
  if (T < 0 || k <= 0 || H <= 0) return MOE_E_INVALID_ARG;
  if (T == 0) return MOE_OK;
  if (!Y || !scores || !y) return MOE_E_INVALID_ARG;
  if (H % 8 != 0 || (reinterpret_cast<uintptr_t>(Y) & 15u) || (reinterpret_cast<uintptr_t>(y) & 15u) ||
      (Ys && (reinterpret_cast<uintptr_t>(Ys) & 15u)))
    return MOE_E_UNSUPPORTED;
  const int64_t n = T * (H / 8);
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  switch (k) {
#define MOE_COMBINE_K(KC)                                                                                   \
  case KC:                                                                                                 \
    MOE_LAUNCH("combine", combine_kernel<KC>, grid, dim3(256), 0, stream, Y, inv_perm, scores, T, k, H, Ys, \
               sgl, y);                                                                                    \
    break;
    MOE_COMBINE_K(1)
    MOE_COMBINE_K(2)
    MOE_COMBINE_K(4)
    MOE_COMBINE_K(6)
    MOE_COMBINE_K(8)
    MOE_COMBINE_K(10)
#undef MOE_COMBINE_K
    default:
      MOE_LAUNCH("combine", combine_kernel<0>, grid, dim3(256), 0, stream, Y, inv_perm, scores, T, k, H, Ys, sgl,
                 y);
  }
  return launch_status("combine");
}

}  // namespace moe
