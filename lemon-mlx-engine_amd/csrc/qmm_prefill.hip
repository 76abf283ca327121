// qmm_prefill.hip -- grouped affine-dequant GEMM for large token counts
// (prefill), gfx950.  Same contract as the grouped kernel in qmm.hip: rows are
// the expert buckets of the sorted (token, expert) pairs.  No weight is
// rounded.
//
// Arithmetic.  For output row m, weight row n and quantization group g:
//     y[m][n] = sum_g s[n,g] P[m,n,g]  +  sum_g b'[n,g] X[m,g]
//     P[m,n,g] = sum_{k in g} x[m][k] (q[n][k] + OFF)    (one MFMA chain per group)
//     X[m,g]   = sum_{k in g} x[m][k]                    (group sums, fp32)
//     b'       = b - OFF * s
// 4-bit codes enter the MFMA as the bf16 value 128 + q (bit pattern 0x4300|q,
// so OFF = 128); 8-bit codes as bf16(q) (exact below 256, OFF = 0).  Both are
// exact, and x * (q + OFF) is exact in the fp32 accumulator.  Each group's
// partial P is folded into the fp32 accumulator with one FMA per output
// (acc += s * P).  (Rounding s*q + b to a bf16 operand instead would cost up
// to a sixth of a quantization step per 8-bit weight and measurably breaks
// the output tolerance at large K.)  The zero point sum is a small GEMM over
// the groups run on the MFMA while the K pipeline fills, written as
// X.b + (-OFF X).s so that its weight-side operands are the checkpoint's own
// bf16 biases and scales; X is split into bf16 hi + lo parts (exact to 2^-16
// relative) and -OFF X is exact.
//
// Tiling.  A workgroup of 4 waves computes a BM x 256 tile of one expert:
// BM = 32*MT token rows by 256 weight rows (GLU: 128 gate rows and the 128
// matching up rows).  Each wave owns all BM rows and 64 weight rows: two
// 32-row weight tiles, with GLU a gate tile and the up tile of the same 32
// output columns, so SwiGLU is applied in registers.
//
// Memory.  Global loads are counted in cache lines touched (a CU's vector
// memory path retires about one line access per two clocks), so every
// instruction reads whole or half lines:
//   * activations: BM rows x 64 bf16 per K step, 8 lanes per 128-byte row,
//     straight to LDS (no VGPR staging) into a ring of 3 (4-bit) / 2 (8-bit)
//     steps, shared by the four waves (one LDS-only barrier per step);
//   * codes: 64 bytes per weight row at a time (two K steps at 4 bits, one at
//     8), 4 lanes per row, straight to LDS into two slots private to each
//     wave, which expands its own rows to bf16 operands in registers (4-bit:
//     one v_perm + one v_and_or per two codes);
//   * scales: 8 groups (16 bytes) of a weight row per lane into registers, the
//     other weight tile's row taken from the lane 32 apart (v_permlane32_swap).
// LDS chunks are XOR-swizzled 16-byte units, so that the 16 lanes a 128-bit
// LDS read serves per clock (64 banks of 4 bytes) never share a bank: keyed on
// row / 2 for the 128-byte activation rows, row / 4 for the 64-byte code rows.
//
// K order.  Within a 64-wide step, lane half h (= lane/32) of the A and B
// operands of substep s carries K = 32h + 8s + [0, 8): a lane's B operands for
// the whole step are one 16-byte (4-bit) or 32-byte (8-bit) run of codes.
//
// Scheduling.  Blocks are numbered so that consecutive virtual tiles land on
// the same XCD (the hardware deals workgroups round-robin over 8 XCDs): the N
// tiles of one token tile, and the token tiles of one expert, share an L2.

#include "internal.hpp"

#include <algorithm>

namespace moe {

struct PArgs {
  const uint16_t* x;        // input rows [*, K]
  const int32_t* row_in;    // sorted pos -> input row (NULL: pos)
  const int32_t* row_out;   // sorted pos -> output row (NULL: pos)
  const uint16_t* xhl;      // [*, nch, 32] group sums X of the input rows: bf16 hi(16) | lo(16) per chunk
  int nch;                  // 16-group chunks per row (G rounded up to 16, / 16)
  int gsum_by_pos;          // xhl rows: 1 = sorted position, 0 = input row (as x)
  const int32_t* tiles;     // [0] = token tile count; entry i at 4+4i: {expert, row0, rows, 0}
  int n_tiles;              // 256-row (GLU: 128-column) tiles along N
  const uint32_t* w[2];
  const uint16_t* s[2];
  const uint16_t* b[2];
  int N, K, gs;
  int wide_scales;          // rows of scales and biases 16-byte aligned (G % 8 == 0): 16-byte loads of 8 groups
  int ldo;                  // output row stride (elements)
  uint16_t* out;
  const uint16_t* lb[2];    // SwitchLinear biases [E, N] of w[0] / w[1] or NULL
  // GLU only, optional: group sums of the output rows (h) for the next
  // projection, in the xhl layout (nch chunks of 2 bf16 planes), groups of gs
  uint16_t* hsum;
  int hsum_nch, hsum_gs, hsum_G;
  int out_p8;               // GLU: write h in the pair K order (see pair_order)
  int act;                  // GLU: moe_activation of h = act(gate, up)
};

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kBN = 256;           // weight rows per workgroup
constexpr int kChunkRow = 64;      // code bytes per weight row in one code chunk
constexpr int kChunkBytes = 4096;  // one wave's 64 rows of a chunk

// g * (1 / (1 + e^-g)) (the checker's form) with the hardware exp and
// reciprocal (v_exp_f32, v_rcp_f32: 1 ulp each; a correctly rounded
// reciprocal costs ten more VALU instructions per output, ~7 % of the gate|up
// kernel's, and its last bit changes the bf16 h in a few outputs only)
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// hi = bf16(v) (round to nearest even), lo = bf16(v - hi); v - hi is exact in fp32.
__device__ __forceinline__ void split_bf16(float v, uint16_t& hi, uint16_t& lo) {
  hi = f2bf(v);
  lo = f2bf(v - bf2f(hi));
}

// (a, b) -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// (v & m) | c as the single v_and_or_b32 (m in an SGPR, c in a VGPR); the
// optimiser otherwise splits it into an AND and an OR
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(m), "v"(c));
  return r;
}

// Pair K order (pair_pos, to_pair_order): the GEMM reads a stored 16-byte
// unit of activations as one MFMA operand of 8 K values, so the codes'
// operand is built in the same order; both orders give the same dot
// products.  In pair order the operand of 8 codes (one word) is 4 AND-ORs of
// the word shifted by 0, 4, 8, 12 bits (codes j and j+4 land in one bf16
// pair) instead of a byte permute and an AND-OR per pair.

// eight 4-bit codes (code j in bits 4j..4j+3) -> bf16 operand [128 + code j]
// in natural order
__device__ __forceinline__ bf16x8 expand_q4(uint32_t w, uint32_t k4300) {
  const uint32_t hw = w >> 4;
  u32x4 o;
  // byte 0 = code 2j (low nibble of byte j), byte 2 = code 2j+1 (low nibble of byte j of w >> 4)
  o[0] = and_or(__builtin_amdgcn_perm(hw, w, 0x0c040c00u), 0x000f000fu, k4300);
  o[1] = and_or(__builtin_amdgcn_perm(hw, w, 0x0c050c01u), 0x000f000fu, k4300);
  o[2] = and_or(__builtin_amdgcn_perm(hw, w, 0x0c060c02u), 0x000f000fu, k4300);
  o[3] = and_or(__builtin_amdgcn_perm(hw, w, 0x0c070c03u), 0x000f000fu, k4300);
  return __builtin_bit_cast(bf16x8, o);
}

// ... in pair order (codes j and j+4 in pair j)
__device__ __forceinline__ bf16x8 expand_q4_pairs(uint32_t w, uint32_t k4300) {
  u32x4 o;
  o[0] = and_or(w, 0x000f000fu, k4300);
  o[1] = and_or(w >> 4, 0x000f000fu, k4300);
  o[2] = and_or(w >> 8, 0x000f000fu, k4300);
  o[3] = and_or(w >> 12, 0x000f000fu, k4300);
  return __builtin_bit_cast(bf16x8, o);
}

// eight 8-bit codes (two words, code j in byte j) -> bf16 operand [code j],
// natural order or (PAIRS) pair order
template <bool PAIRS>
__device__ __forceinline__ bf16x8 expand_q8(uint32_t w0, uint32_t w1) {
  if constexpr (PAIRS) {
    u32x4 o;
    o[0] = pk_bf16(static_cast<float>(w0 & 0xffu), static_cast<float>(w1 & 0xffu));
    o[1] = pk_bf16(static_cast<float>((w0 >> 8) & 0xffu), static_cast<float>((w1 >> 8) & 0xffu));
    o[2] = pk_bf16(static_cast<float>((w0 >> 16) & 0xffu), static_cast<float>((w1 >> 16) & 0xffu));
    o[3] = pk_bf16(static_cast<float>(w0 >> 24), static_cast<float>(w1 >> 24));
    return __builtin_bit_cast(bf16x8, o);
  }
  u32x4 o;
  o[0] = pk_bf16(static_cast<float>(w0 & 0xffu), static_cast<float>((w0 >> 8) & 0xffu));
  o[1] = pk_bf16(static_cast<float>((w0 >> 16) & 0xffu), static_cast<float>(w0 >> 24));
  o[2] = pk_bf16(static_cast<float>(w1 & 0xffu), static_cast<float>((w1 >> 8) & 0xffu));
  o[3] = pk_bf16(static_cast<float>((w1 >> 16) & 0xffu), static_cast<float>(w1 >> 24));
  return __builtin_bit_cast(bf16x8, o);
}

// LDS bytes of one tile body: activation ring + code slots (+ group-sum
// staging with a two-stage ring), or the output tile, whichever is larger
template <int BITS, bool GLU, int MT>
constexpr int prefill_lds_bytes() {
  constexpr int BM = 32 * MT;
  constexpr int kAStages = BITS == 4 ? 3 : 2;
  constexpr int kMain = kAStages * BM * 128 + 4 * 2 * kChunkBytes + (kAStages == 3 ? 0 : BM * 128);
  constexpr int kOut = BM * ((GLU ? 128 : kBN) + 8) * 2;
  return kMain > kOut ? kMain : kOut;
}

// One output tile: token rows row0 .. row0+rows-1 (sorted positions of
// expert e's bucket, rows <= 32*MT) x column tile ntile.  PAIRS: the input
// rows are stored in pair K order.  GACT (GLU): h = glu_act(a.act, ...), the
// activations other than SwiGLU; without it the SwiGLU epilogue alone is
// compiled (the selector's other branches, inlined into every tile height's
// unrolled epilogue, doubled the kernel's code and cost ~4 % of gate|up).
template <int BITS, bool GLU, int MT, bool PAIRS, bool GACT = false>
__device__ __forceinline__ void prefill_tile(const PArgs& a, uint8_t* lds, const int e, const int row0,
                                             const int rows, const int ntile) {
  constexpr int BM = 32 * MT;
  constexpr int OFF = BITS == 4 ? 128 : 0;
  constexpr int kAStages = BITS == 4 ? 3 : 2;  // activation ring (steps)
  constexpr int kLead = kAStages - 1;          // steps the loads run ahead
  constexpr int kABytes = BM * 128;            // activation tile per stage: BM rows x 64 bf16
  constexpr int kSPC = BITS == 4 ? 2 : 1;      // K steps per code chunk
  constexpr int kBSlots = 2;                   // code chunk slots per wave
  constexpr int kLdsA = kAStages * kABytes;
  constexpr int kLdsB = 4 * kBSlots * kChunkBytes;
  constexpr int OW = GLU ? 128 : kBN;  // output columns of the tile
  constexpr int OS = OW + 8;           // LDS row stride of the output tile (elements)
  // group sums of the tile's rows are staged through LDS before the K loop:
  // in the third activation stage (idle until then), or, with a two-stage
  // ring, in a region of their own (BM rows x 128 bytes: two 16-group chunks)
  constexpr int kLdsZ = kAStages == 3 ? 0 : BM * 128;
  constexpr int kLdsMain = kLdsA + kLdsB + kLdsZ;
  static_assert((kLdsMain > BM * OS * 2 ? kLdsMain : BM * OS * 2) == prefill_lds_bytes<BITS, GLU, MT>(), "LDS size");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int KS = a.K >> 6;
  const int NCH = KS / kSPC;  // code chunks along K
  const int gdiv = a.gs >> 6;
  const int G = a.K / a.gs;
  const uint32_t wrow_bytes = static_cast<uint32_t>(a.K) * BITS / 8;

  // weight row (within the expert) and matrix of code row c = 64*wave + 32*nt + l
  // (GLU: nt 0 = gate, 1 = up of the same 32 output columns)
  auto code_row = [&](int c, int& mat) -> int {
    if (GLU) {
      mat = (c >> 5) & 1;
      return ntile * 128 + (c >> 6) * 32 + (c & 31);
    }
    mat = 0;
    return ntile * kBN + c;
  };

  // ---- producers: buffer loads straight to LDS, a 32-bit offset per lane
  //      and the step's offset in a scalar register ----
  // activation block j of this wave = tile rows 8*(wave + 4j) .. +7, 128
  // bytes each; lane -> row + lane/8, LDS slot lane%8 holds 16-byte chunk
  // slot ^ ((row / 2) % 8).  Offsets into x fit 32 bits (checked on the host).
  const __amdgpu_buffer_rsrc_t xrs = raw_rsrc(a.x);
  uint32_t aoff[MT];
  uint32_t zrow[MT];  // group-sum row of the same tile row (input row, or sorted position)
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const int r = 8 * (wave + 4 * j) + (lane >> 3);
    const int pos = row0 + min(r, rows - 1);
    const uint32_t xr = static_cast<uint32_t>(a.row_in ? a.row_in[pos] : pos);
    aoff[j] = xr * static_cast<uint32_t>(a.K) * 2u + 16u * static_cast<uint32_t>((lane & 7) ^ ((r >> 1) & 7));
    zrow[j] = a.gsum_by_pos ? static_cast<uint32_t>(pos) : xr;
  }
  // code chunk q of this wave's 64 rows (bytes 64q .. 64q+63 of each) goes to
  // the wave's own slot q % 2; instruction i covers rows 16i + lane/4 (one
  // matrix: with GLU rows 0-31 of a wave are gate rows, 32-63 up rows), LDS
  // slot lane%4 of a row holds its 16-byte part slot ^ ((row / 4) % 4).
  // Instruction i's weight rows are instruction 0's plus a wave-uniform step
  // (GLU: the same 32 output columns of the up matrix for i >= 2), so one
  // lane offset serves all four with the step in the scalar offset.
  __amdgpu_buffer_rsrc_t wrs[2];
#pragma unroll
  for (int m = 0; m < 2; ++m)
    wrs[m] = raw_rsrc(reinterpret_cast<const uint8_t*>(a.w[GLU ? m : 0]) + static_cast<int64_t>(e) * a.N * wrow_bytes);
  uint32_t coff;
  {
    int mat;
    const int wr = code_row(64 * wave + (lane >> 2), mat);
    coff = static_cast<uint32_t>(wr) * wrow_bytes + 16u * static_cast<uint32_t>((lane & 3) ^ ((lane >> 4) & 3));
  }
  auto crow_step = [&](int i) -> uint32_t {  // byte offset of instruction i's rows from instruction 0's
    return static_cast<uint32_t>(GLU ? (i & 1) * 16 : i * 16) * wrow_bytes;
  };
  uint8_t* bring = lds + kLdsA + wave * (kBSlots * kChunkBytes);

  auto issue_a = [&](int ks, int stage) {  // stage = ks % kAStages; steps past the end re-read the last step (in bounds)
    const uint32_t kc = static_cast<uint32_t>(min(ks, KS - 1));
    uint8_t* sb = lds + stage * kABytes;
#pragma unroll
    for (int j = 0; j < MT; ++j) buffer_load_lds16(xrs, aoff[j], kc * 128u, sb + (wave + 4 * j) * 1024);
  };
  auto issue_b = [&](int q) {
    const uint32_t qc = static_cast<uint32_t>(min(q, NCH - 1));
    uint8_t* dst = bring + (q % kBSlots) * kChunkBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      buffer_load_lds16(wrs[GLU ? i >> 1 : 0], coff, qc * kChunkRow + crow_step(i), dst + i * 1024);
  };

  // ---- scales: lane (l32, h) holds 8 groups of weight row (nt = h, l32) in
  //      registers; the other tile's row comes from lane l32 + 32(1 - h) ----
  const uint16_t* sprow;
  {
    int mat;
    const int wr = code_row(64 * wave + 32 * h + l32, mat);
    sprow = a.s[mat] + (static_cast<int64_t>(e) * a.N + wr) * G;
  }
  const bool wide = a.wide_scales != 0;
  // chunk j holds groups [c0, c0 + 8), c0 = max(min(8j, G - 8), 0); the
  // 4-byte pairs of the narrow form are clamped to the row (G is even)
  auto load_sc = [&](int j, u32x4& sv) {
    const int c0 = max(min(8 * j, G - 8), 0);
    if (wide) {
      sv = *reinterpret_cast<const u32x4*>(sprow + c0);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] = *reinterpret_cast<const uint32_t*>(sprow + min(c0 + 2 * i, G - 2));
    }
  };

  // LDS byte offsets (within a stage / slot) of this lane's operands
  int aread[4];  // A fragment of substep s of m-tile 0 (+ 32*128*mt)
#pragma unroll
  for (int s = 0; s < 4; ++s) aread[s] = l32 * 128 + 16 * ((4 * h + s) ^ ((l32 >> 1) & 7));
  // codes of weight tile 0 (tile 1: rows 32 further, + 2048 bytes): 4-bit,
  // step parity p (part 2p + h); 8-bit, half p (part 2h + p)
  int bread[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int part = BITS == 4 ? 2 * p + h : 2 * h + p;
    bread[p] = l32 * kChunkRow + 16 * (part ^ ((l32 >> 2) & 3));
  }

  f32x16 acc[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][j][r] = 0.0f;
  const f32x16 zero = {};  // an inline-constant accumulator operand

  // ---- prologue: the tile rows' group sums go through LDS, two 16-group
  //      chunks (128 bytes of a row) a round: one DMA instruction per 8 rows,
  //      16-byte units swizzled by row / 2.  Round 0 first, then the scales
  //      of chunk 0 and the first kLead steps ----
  const __amdgpu_buffer_rsrc_t zrs = raw_rsrc(a.xhl);
  uint8_t* zs = lds + (kAStages == 3 ? 2 * kABytes : kLdsA + kLdsB);
  auto issue_z = [&](int c0) {  // units past the row's last chunk re-read unit 0 (in bounds, unused)
    const int nu = min(a.nch - c0, 2) * 4;  // 16-byte units of the round
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int r = 8 * (wave + 4 * j) + (lane >> 3);
      const int u = (lane & 7) ^ ((r >> 1) & 7);
      const uint32_t off = (zrow[j] * static_cast<uint32_t>(a.nch) + static_cast<uint32_t>(c0)) * 64u +
                           (u < nu ? 16u * static_cast<uint32_t>(u) : 0u);
      buffer_load_lds16(zrs, off, 0u, zs + (wave + 4 * j) * 1024);
    }
  };
  // weight side of the zero-point term: the biases and scales of groups
  // 16c + 8h .. +7 of this lane's two weight rows, one 16-byte load each
  // where the 8 groups lie in the row (else per dword, clamped to the row: in
  // bounds, and groups past G meet zero group sums); without biases the
  // scales are read in their place and the bias MFMAs are skipped.  Chunk 0
  // is loaded first of all (its latency overlaps the group sums'), each
  // later chunk one chunk ahead.
  const uint16_t* brow[2];
  const uint16_t* srow[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    int mat;
    const int wr = code_row(64 * wave + 32 * nt + l32, mat);
    const int64_t base = (static_cast<int64_t>(e) * a.N + wr) * G;  // even: G is even
    srow[nt] = a.s[mat] + base;
    brow[nt] = (a.b[mat] ? a.b[mat] : a.s[mat]) + base;
  }
  auto load_bs = [&](int c, u32x4(&bw)[2], u32x4(&sw)[2]) {
    const int g0 = 16 * c + 8 * h;
    if (a.wide_scales && g0 + 8 <= G) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        bw[nt] = *reinterpret_cast<const u32x4*>(brow[nt] + g0);
        sw[nt] = *reinterpret_cast<const u32x4*>(srow[nt] + g0);
      }
    } else {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int d = min(g0 / 2 + q, G / 2 - 1);
          bw[nt][q] = reinterpret_cast<const uint32_t*>(brow[nt])[d];
          sw[nt][q] = reinterpret_cast<const uint32_t*>(srow[nt])[d];
        }
    }
  };
  u32x4 bw[2], sw[2];
  load_bs(0, bw, sw);
  issue_z(0);
  u32x4 sc_cur;
  load_sc(0, sc_cur);
  issue_b(0);
#pragma unroll
  for (int i = 0; i < kLead; ++i) issue_a(i, i);

  // ---- zero-point term first: acc = X . b'^T over the groups, 16 per MFMA
  //      (its loads overlap the pipeline fill) ----
  {
    // round 0 has landed: only the loads issued after it may be in flight
    if (a.wide_scales) wait_vmcnt<1 + 4 + kLead * MT>();
    else wait_vmcnt<4 + 4 + kLead * MT>();
    const bool has_b = a.b[0] != nullptr;
    for (int c = 0; c < a.nch; ++c) {
      if ((c & 1) == 0) {
        if (c > 0) {  // the next round: every earlier load has landed by then
          lds_barrier();  // the previous round's reads are done
          issue_z(c);
          wait_vmcnt<0>();
        }
        lds_barrier();
      }
      u32x4 bwn[2], swn[2];
      if (c + 1 < a.nch) load_bs(c + 1, bwn, swn);
      // -OFF * s: exact (a power-of-two multiple)
      if constexpr (OFF != 0) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            sw[nt][q] = pk_bf16(-static_cast<float>(OFF) * __uint_as_float(sw[nt][q] << 16),
                                -static_cast<float>(OFF) * __uint_as_float(sw[nt][q] & 0xffff0000u));
      }
      // one m-tile's group sums at a time (few registers live beside acc)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        u32x4 xv[2];  // hi, lo of groups 16c + 8h .. +7 of row m
        const int m = mt * 32 + l32;
#pragma unroll
        for (int q = 0; q < 2; ++q)
          xv[q] = *reinterpret_cast<const u32x4*>(zs + m * 128 + 16 * ((4 * (c & 1) + 2 * q + h) ^ ((m >> 1) & 7)));
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const bf16x8 bB = __builtin_bit_cast(bf16x8, bw[nt]);
          const bf16x8 sB = __builtin_bit_cast(bf16x8, sw[nt]);
          if (has_b) {
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xv[0]), bB, acc[mt][nt], 0, 0, 0);
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xv[1]), bB, acc[mt][nt], 0, 0, 0);
          }
          if constexpr (OFF != 0) {
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xv[0]), sB, acc[mt][nt], 0, 0, 0);
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xv[1]), sB, acc[mt][nt], 0, 0, 0);
          }
        }
        // keep the next m-tile's loads below this point (register pressure)
        __builtin_amdgcn_sched_barrier(0);
      }
      if (c + 1 < a.nch) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          bw[nt] = bwn[nt];
          sw[nt] = swn[nt];
        }
      }
    }
  }

  // step 0's tiles and the scales have landed (4-bit: step 1's activations may
  // still be in flight)
  wait_vmcnt<BITS == 4 ? MT : 0>();
  lds_barrier();

  const uint32_t k4300 = 0x43004300u;
  const int sc_period = 8 * gdiv;  // K steps per 8-group scale chunk
  // per-step indices carried from step to step (a runtime division by gdiv
  // or sc_period costs about 15 scalar instructions a step): the step's
  // group g and its K step within the group, the steps since the last scale
  // chunk load, the activation stages of this step and of step ks + kLead
  int g = 0, g_step = 0, sc_step = 0, sc_chunk = 0, stage = 0, stage_lead = kLead % kAStages;
  for (int ks = 0; ks < KS; ++ks) {
    // ---- scale of the step's group for both weight tiles ----
    const int gi = g - max(min(8 * (g >> 3), G - 8), 0);
    const uint32_t sd = gi < 2 ? sc_cur[0] : gi < 4 ? sc_cur[1] : gi < 6 ? sc_cur[2] : sc_cur[3];
    const auto ss = __builtin_amdgcn_permlane32_swap(sd, sd, false, false);  // [nt]: tile nt's row
    const bool odd = gi & 1;
    float sc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) sc[nt] = __uint_as_float(odd ? (ss[nt] & 0xffff0000u) : (ss[nt] << 16));

    // ---- loads for later steps: after the last step of a scale chunk, the
    //      next chunk into the same registers (issued first: the end-of-step
    //      wait covers it); activations of step ks + kLead; at the first step
    //      of a code chunk, the next code chunk ----
    if (++sc_step == sc_period) {
      sc_step = 0;
      if (ks + 1 < KS) load_sc(++sc_chunk, sc_cur);
    }
    if constexpr (BITS == 4) {
      // at the first step of a code chunk the next chunk, first; then the
      // activations kLead steps ahead.  Past the end these re-read the last
      // step's tiles / chunk into a stage / slot that no later step reads, so
      // the wait below is one constant (a branch on it costs the register
      // allocator dearly: spills at four m-tiles)
      if (ks % kSPC == 0) issue_b(ks / kSPC + 1);
      issue_a(ks + kLead, stage_lead);
    } else if (ks + 1 < KS) {
      issue_a(ks + 1, stage_lead);
      issue_b(ks + 1);
    }

    // ---- B operands of the two weight tiles for the four substeps ----
    const uint8_t* cb = bring + ((ks / kSPC) % kBSlots) * kChunkBytes;
    bf16x8 bf[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      if constexpr (BITS == 4) {
        const u32x4 c = *reinterpret_cast<const u32x4*>(cb + bread[ks & 1] + 2048 * nt);
#pragma unroll
        for (int s = 0; s < 4; ++s) bf[nt][s] = PAIRS ? expand_q4_pairs(c[s], k4300) : expand_q4(c[s], k4300);
      } else {
        const u32x4 c0 = *reinterpret_cast<const u32x4*>(cb + bread[0] + 2048 * nt);
        const u32x4 c1 = *reinterpret_cast<const u32x4*>(cb + bread[1] + 2048 * nt);
        bf[nt][0] = expand_q8<PAIRS>(c0[0], c0[1]);
        bf[nt][1] = expand_q8<PAIRS>(c0[2], c0[3]);
        bf[nt][2] = expand_q8<PAIRS>(c1[0], c1[1]);
        bf[nt][3] = expand_q8<PAIRS>(c1[2], c1[3]);
      }
    }

    // ---- per m-tile: the group's partial products of the two weight tiles,
    //      each an MFMA chain over the four substeps, folded in with the
    //      tile's scale ----
    const uint8_t* sa = lds + stage * kABytes;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      bf16x8 af[4];
#pragma unroll
      for (int s = 0; s < 4; ++s)
        af[s] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(sa + mt * 32 * 128 + aread[s]));
      f32x16 p0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0], bf[0][0], zero, 0, 0, 0);
#pragma unroll
      for (int s = 1; s < 4; ++s) p0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s], bf[0][s], p0, 0, 0, 0);
      f32x16 p1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[0], bf[1][0], zero, 0, 0, 0);
#pragma unroll
      for (int s = 1; s < 4; ++s) p1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s], bf[1][s], p1, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][0][r] = __builtin_fmaf(sc[0], p0[r], acc[mt][0][r]);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][1][r] = __builtin_fmaf(sc[1], p1[r], acc[mt][1][r]);
    }

    // step ks+1's tiles, chunk and scales have landed: in flight may stay
    // only this step's activations (4-bit; its code chunk, issued before
    // them, is waited for: one step early at the first step of a chunk).
    // 8-bit runs one step ahead: nothing.
    if constexpr (BITS == 4) wait_vmcnt<MT>();
    else wait_vmcnt<0>();
    lds_barrier();
    if (++g_step == gdiv) {
      g_step = 0;
      ++g;
    }
    stage = stage + 1 == kAStages ? 0 : stage + 1;
    stage_lead = stage_lead + 1 == kAStages ? 0 : stage_lead + 1;
  }
  wait_vmcnt<0>();  // no LDS write outstanding past this point

  // output rows of this thread's 16-byte store chunks and of its h group-sum
  // row, loaded here so that their latency overlaps the staging below
  constexpr int CPR = OW / 8;          // 16-byte chunks per output row
  constexpr int RPP = kThreads / CPR;  // rows per pass of the store loop
  constexpr int NPASS = BM / RPP;
  int orow[NPASS];
#pragma unroll
  for (int j = 0; j < NPASS; ++j) {
    const int m = tid / CPR + RPP * j;
    orow[j] = m < rows ? (a.row_out ? a.row_out[row0 + m] : row0 + m) : 0;
  }
  const int hs_gpt = GLU && a.hsum ? OW / a.hsum_gs : 1;  // h groups per tile: 2 (gs 64) or 1 (gs 128)
  const int hs_m = tid / hs_gpt;
  int hs_row = 0;
  if (GLU && a.hsum && hs_m < rows) hs_row = a.row_out ? a.row_out[row0 + hs_m] : row0 + hs_m;

  // ---- epilogue: the output tile goes through LDS so that global stores
  //      are 16-byte, whole-row-segment writes.  D layout of the 32x32 MFMA:
  //      column = lane%32, row = 8*(r/4) + 4*(lane/32) + r%4.  Rows r and r+1
  //      of a lane pair (columns 2i, 2i+1) are exchanged across the pair (DPP)
  //      so that each lane writes one dword of two adjacent columns: the even
  //      lane row r, the odd lane row r+1 ----
  lds_barrier();  // every wave's DMA writes have landed (vmcnt(0) above)
  uint16_t* ot = reinterpret_cast<uint16_t*>(lds);
  const bool odd_lane = l32 & 1;
  // SwitchLinear's bias of this lane's output features (switch_layers.cpp:111-114),
  // added to the bf16 projection output: GLU, gate and up of feature
  // 128*ntile + 32*wave + l32; otherwise features 256*ntile + 64*wave + l32 (+ 32)
  float lbv[2] = {0.0f, 0.0f};
  bool has_lb[2] = {false, false};
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    int mat;
    const int f = code_row(64 * wave + 32 * nt + l32, mat);
    const uint16_t* lbp = a.lb[GLU ? mat : 0];
    has_lb[nt] = lbp != nullptr;
    if (lbp) lbv[nt] = bf2f(lbp[static_cast<int64_t>(e) * a.N + f]);
  }
  const int hcol = wave * 32 + (a.out_p8 ? (l32 & ~7) | pair_pos(l32 & 7) : l32);  // GLU: this lane's h column
  auto put_pair = [&](int m0, int col0, float v0, float v1) {  // v0: row m0, v1: row m0 + 1, column col0 + l32
    const float partner = dpp_f<kDppQuadXor1>(odd_lane ? v0 : v1);
    const uint32_t w = odd_lane ? pk_bf16(partner, v1) : pk_bf16(v0, partner);
    *reinterpret_cast<uint32_t*>(ot + (m0 + (odd_lane ? 1 : 0)) * OS + col0 + (l32 & ~1)) = w;
  };
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const int m0 = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
      if constexpr (GLU) {
        // SwiGLU of the bf16-rounded gate and up values (the reference's op
        // outputs); rows m0 and m0 + 1 of this lane's column, each a 16-bit
        // store at the column's position (pair K order for a GEMM that reads
        // h in that order)
        const uint32_t gp = pk_bf16(acc[mt][0][r], acc[mt][0][r + 1]);
        const uint32_t up = pk_bf16(acc[mt][1][r], acc[mt][1][r + 1]);
        float g0 = __uint_as_float(gp << 16), g1 = __uint_as_float(gp & 0xffff0000u);
        float u0 = __uint_as_float(up << 16), u1 = __uint_as_float(up & 0xffff0000u);
        if (has_lb[0]) {
          g0 = bfr(g0 + lbv[0]);
          g1 = bfr(g1 + lbv[0]);
        }
        if (has_lb[1]) {
          u0 = bfr(u0 + lbv[1]);
          u1 = bfr(u1 + lbv[1]);
        }
        uint32_t hv;
        if constexpr (GACT) hv = pk_bf16(glu_act(a.act, g0, u0, silu(g0)), glu_act(a.act, g1, u1, silu(g1)));
        else hv = pk_bf16(silu(g0) * u0, silu(g1) * u1);
        ot[m0 * OS + hcol] = static_cast<uint16_t>(hv);
        ot[(m0 + 1) * OS + hcol] = static_cast<uint16_t>(hv >> 16);
      } else {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          float v0 = acc[mt][nt][r], v1 = acc[mt][nt][r + 1];
          if (has_lb[nt]) {
            v0 = bfr(v0) + lbv[nt];
            v1 = bfr(v1) + lbv[nt];
          }
          put_pair(m0, wave * 64 + 32 * nt, v0, v1);
        }
      }
    }
  }
  // the output-row loads above have landed (their latency overlapped the
  // staging): with nothing of this wave's outstanding, no store below waits
  // for the one before it (stores and loads share one counter, and the
  // compiler otherwise waits for all of them before each conditional store)
  wait_vmcnt<0>();
  lds_barrier();
  {
    const int c8 = tid % CPR;
#pragma unroll
    for (int j = 0; j < NPASS; ++j) {
      const int m = tid / CPR + RPP * j;
      if (m < rows)  // streaming (nt) stores: the tile is read by the next launch, not from this L2
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(ot + m * OS + 8 * c8),
                                    reinterpret_cast<u32x4*>(a.out + static_cast<int64_t>(orow[j]) * a.ldo + ntile * OW + 8 * c8));
    }
  }
  if constexpr (GLU) {
    if (a.hsum) {
      // group sums of the bf16 h values of this tile's 128 columns: one
      // (row, group) per thread, written at the row's output index
      const int gpt = hs_gpt;
      const int m = hs_m, q = tid - m * gpt;
      if (m < rows) {
        float sum = 0.0f;
        for (int c = 0; c < a.hsum_gs; c += 8) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(ot + m * OS + q * a.hsum_gs + c);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            sum += __uint_as_float(v[j] << 16);
            sum += __uint_as_float(v[j] & 0xffff0000u);
          }
        }
        uint16_t* dst = a.hsum + static_cast<int64_t>(hs_row) * a.hsum_nch * 32;
        const int g = ntile * gpt + q;
        uint16_t hi, lo;
        split_bf16(sum, hi, lo);
        uint16_t* c = dst + (g >> 4) * 32 + (g & 15);
        c[0] = hi;
        c[16] = lo;
        // groups past the last one are zero (written by the first column tile)
        if (ntile == 0 && q == 0)
          for (int gz = a.hsum_G; gz < 16 * a.hsum_nch; ++gz)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) dst[(gz >> 4) * 32 + 16 * pl + (gz & 15)] = 0;
      }
    }
  }
}

// The grouped GEMM over the token-tile table (see make_tiles_kernel): n4
// tiles of 128 rows, then n3 of 96, n2 of 64 and n1 of 32, each against every
// column tile.  Workgroups go to the 8 XCDs round robin (XCD = bid % 8).  Each
// XCD first takes one contiguous eighth of the 128- and 96-row tiles (tiles
// sharing rows or weights share its L2), then the short tiles, dealt round
// robin, so that the last workgroups to run are short ones.  The grid is sized
// for the most tiles P rows can need; the split follows the real counts.  All
// four bodies share the one LDS allocation (the 128-row body needs the most).
template <int BITS, bool GLU, bool PAIRS, bool GACT = false>
__global__ __launch_bounds__(kThreads, 2) void grouped_gemm_prefill_kernel(PArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[prefill_lds_bytes<BITS, GLU, 4>()];
  const int bid = blockIdx.x;
  const int4 cnt = reinterpret_cast<const int4*>(a.tiles)[0];  // {n4, n3, n2, n1}
  const int nt = a.n_tiles;
  const int xcd = bid & 7, i = bid >> 3;
  const int nlong = cnt.x + cnt.y;
  const int vl = nlong * nt;
  const int perl = (vl + 7) >> 3;
  int slot, ntile;
  if (i < perl) {
    const int v = xcd * perl + i;
    if (v >= vl) return;
    slot = v / nt;
    ntile = v - slot * nt;
  } else {
    const int v = (i - perl) * 8 + xcd;
    if (v >= (cnt.z + cnt.w) * nt) return;
    const int q = v / nt;
    ntile = v - q * nt;
    slot = nlong + q;
  }
  const int4 tinfo = reinterpret_cast<const int4*>(a.tiles)[1 + slot];
  if (slot < cnt.x)
    prefill_tile<BITS, GLU, 4, PAIRS, GACT>(a, lds, tinfo.x, tinfo.y, tinfo.z, ntile);
  else if (slot < nlong)
    prefill_tile<BITS, GLU, 3, PAIRS, GACT>(a, lds, tinfo.x, tinfo.y, tinfo.z, ntile);
  else if (slot < nlong + cnt.z)
    prefill_tile<BITS, GLU, 2, PAIRS, GACT>(a, lds, tinfo.x, tinfo.y, tinfo.z, ntile);
  else
    prefill_tile<BITS, GLU, 1, PAIRS, GACT>(a, lds, tinfo.x, tinfo.y, tinfo.z, ntile);
}

// xhl[r] = the group sums X[g] (fp32) of row src(r) as bf16 hi and lo parts,
// (xp != NULL: also row r of x in pair K order, xp[r] = pairs(x[r]));
// in 16-group chunks [hi(16) | lo(16)]; groups past G are zero.
// src(r) = row_in ? row_in[r] : r.  L = gs/8 consecutive lanes own one group
// (16 bytes each: whole 128-byte lines per 8 lanes) and add their partial
// sums across the DPP row; groups are numbered over rows x 16*nch.
template <int L>
__global__ __launch_bounds__(256) void group_sums_kernel(const uint16_t* __restrict__ x,
                                                         const int32_t* __restrict__ row_in, int64_t R, int K,
                                                         int nch, uint16_t* __restrict__ xhl,
                                                         uint16_t* __restrict__ xp) {
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int part = threadIdx.x & (L - 1);
  const int64_t gid = tid / L;  // wave-aligned: L divides 64
  const int gpr = 16 * nch;
  const int64_t r = gid / gpr;
  const int g = static_cast<int>(gid % gpr);
  const int G = K / (8 * L);
  float s = 0.0f;
  if (r < R && g < G) {
    const uint16_t* xr = x + (row_in ? static_cast<int64_t>(row_in[r]) : r) * K;
    const int64_t off = static_cast<int64_t>(g) * 8 * L + 8 * part;
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + off);
    if (xp) *reinterpret_cast<u32x4*>(xp + r * K + off) = to_pair_order(v);  // row r in pair K order
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      s += __uint_as_float(v[q] << 16);
      s += __uint_as_float(v[q] & 0xffff0000u);
    }
  }
  // every lane of the wave takes part in the row sums (no lane has left)
  s += dpp_f<kDppQuadXor1>(s);
  s += dpp_f<kDppQuadXor2>(s);
  s += dpp_f<kDppHalfMirror>(s);
  if constexpr (L == 16) s += dpp_f<kDppMirror>(s);
  if (part == 0 && r < R) {
    uint16_t hi, lo;
    split_bf16(s, hi, lo);
    uint16_t* c = xhl + r * nch * 32 + (g >> 4) * 32 + (g & 15);
    c[0] = hi;
    c[16] = lo;
  }
}

// Token-tile table (layout: tile_counts / write_tiles) from the offsets.
__global__ __launch_bounds__(1024) void make_tiles_kernel(const int32_t* __restrict__ offsets, int E,
                                                          int32_t* __restrict__ tiles) {
  __shared__ int base[4][1025];
  const int t = threadIdx.x;
  int c4 = 0, c3 = 0, c2 = 0, c1 = 0;
  if (t < E) tile_counts(offsets[t + 1] - offsets[t], c4, c3, c2, c1);
  base[0][t] = c4;
  base[1][t] = c3;
  base[2][t] = c2;
  base[3][t] = c1;
  __syncthreads();
  if (t < 4) {  // exclusive scans of the four counts over experts
    int run = 0;
    for (int i = 0; i < E; ++i) {
      const int n = base[t][i];
      base[t][i] = run;
      run += n;
    }
    base[t][E] = run;
    tiles[t] = run;
  }
  __syncthreads();
  if (t < E)
    write_tiles(tiles, t, offsets[t], offsets[t + 1] - offsets[t], c4, c3, c2, c1, base[0][t], base[1][t], base[2][t],
                base[3][t], base[0][E], base[1][E], base[2][E]);
}

template <int BITS, bool GLU, bool PAIRS, bool GACT = false>
int launch_prefill(const PArgs& a, unsigned grid, hipStream_t stream) {
  MOE_LAUNCH(GLU ? "gemm_gate_up_swiglu" : "gemm_down", (grouped_gemm_prefill_kernel<BITS, GLU, PAIRS, GACT>),
             dim3(grid), dim3(kThreads), 0, stream, a);
  return launch_status("grouped_gemm_prefill");
}

}  // namespace

// 4-byte words per row of the group-sum buffer: 32 bf16 per 16-group chunk
int prefill_gsum_stride(const moe_qweight* w) { return (w->K / w->group_size + 15) / 16 * 16; }

// header + at most P/128 + E' tiles of 128 rows and E' each of 64 and 32
// rows, E' = min(E, P) non-empty experts
int64_t prefill_tile_ints(int64_t P, int E) { return 4 * (1 + P / 128 + 3 * std::min<int64_t>(E, P)); }

bool prefill_supported(const moe_qweight* w0, const moe_qweight* w1) {
  if (w0->bits != 4 && w0->bits != 8) return false;  // 6-bit experts: the per-16-row kernel
  if (w0->group_size % 64 != 0) return false;
  const int G = w0->K / w0->group_size;
  if (G % 2 != 0) return false;  // scale pairs are read as aligned dwords
  // code chunks are 16-byte loads of 64-byte row segments (two K steps at 4 bits)
  if (w0->K % (w0->bits == 4 ? 128 : 64) != 0) return false;
  const moe_qweight* ws[2] = {w0, w1};
  for (const moe_qweight* w : ws) {
    if (!w) continue;
    if (reinterpret_cast<uintptr_t>(w->w) % 16 != 0 || reinterpret_cast<uintptr_t>(w->scales) % 4 != 0) return false;
  }
  // the zero-point MFMAs take the bias operand of both matrices or of neither
  if (w1 && (w0->biases == nullptr) != (w1->biases == nullptr)) return false;
  if (static_cast<int64_t>(w0->N) * w0->K * w0->bits / 8 >= (int64_t{1} << 32)) return false;
  if (w1) return w0->N % (kBN / 2) == 0;
  return w0->N % kBN == 0;
}

// offsets [E+1] on device; tiles: prefill_tile_ints(P, E) ints of scratch
// (tiles_ready: already built from these offsets);
// gsum: scratch of max(x_rows, P) * prefill_gsum_stride(w0) 4-byte words.
// x_rows = rows of x when known (group sums are then taken once per input
// row), -1 otherwise (sums of the gathered rows, one per sorted position).
// P = total rows, slots = number of non-empty experts at most (bounds the
// partial tiles).
int grouped_gemm_prefill(const uint16_t* x, const int32_t* row_in, const int32_t* row_out, const PrefillScratch& pf,
                         const int32_t* offsets, int E, int64_t P, int slots, const moe_qweight* w0,
                         const moe_qweight* w1, uint16_t* out, hipStream_t stream) {
  const int64_t x_rows = pf.x_rows;
  float* gsum = pf.gsum;
  int32_t* tiles = pf.tiles;
  // gate|up reads its input rows in pair K order from pf.xp (written with the
  // group sums here, or by the router projection when gsum_ready)
  if (w1 && (!pf.xp || x_rows < 0)) return MOE_E_INVALID_ARG;
  const uint16_t* xin = w1 ? pf.xp : x;
  if (E > 1024) return MOE_E_UNSUPPORTED;
  // the kernel addresses x with 32-bit byte offsets
  if ((x_rows >= 0 ? x_rows : P) * static_cast<int64_t>(w0->K) * 2 >= (int64_t{1} << 32)) return MOE_E_UNSUPPORTED;
  const int gstride = prefill_gsum_stride(w0);
  const bool by_pos = x_rows < 0;
  const int64_t R = by_pos ? P : x_rows;
  if (R > 0 && !(pf.gsum_ready && !by_pos)) {
    const int L = w0->group_size / 8;  // 8 or 16 lanes per group
    const int64_t threads = R * (gstride / 16) * 16 * L;
    if ((threads + 255) / 256 > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    const int32_t* rin = by_pos ? row_in : nullptr;
    if (L == 8)
      MOE_LAUNCH("group_sums", group_sums_kernel<8>, grid, dim3(256), 0, stream, x, rin, R, w0->K, gstride / 16,
                 reinterpret_cast<uint16_t*>(gsum), w1 ? pf.xp : nullptr);
    else
      MOE_LAUNCH("group_sums", group_sums_kernel<16>, grid, dim3(256), 0, stream, x, rin, R, w0->K, gstride / 16,
                 reinterpret_cast<uint16_t*>(gsum), w1 ? pf.xp : nullptr);
    MOE_CHECK_LAUNCH("group_sums");
  }
  if (!pf.tiles_ready) {
    MOE_LAUNCH("make_tiles", make_tiles_kernel, dim3(1), dim3(1024), 0, stream, offsets, E, tiles);
    MOE_CHECK_LAUNCH("make_tiles");
  }
  PArgs a{};
  a.x = xin;
  a.row_in = row_in;
  a.row_out = row_out;
  a.xhl = reinterpret_cast<const uint16_t*>(gsum);
  a.nch = gstride / 16;
  a.gsum_by_pos = by_pos ? 1 : 0;
  a.tiles = tiles;
  a.w[0] = w0->w;
  a.s[0] = w0->scales;
  a.b[0] = w0->biases;
  a.lb[0] = w0->linear_bias;
  a.lb[1] = w1 ? w1->linear_bias : nullptr;
  auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  bool wide = (w0->K / w0->group_size) % 8 == 0 && al16(w0->scales) && (!w0->biases || al16(w0->biases));
  if (w1) {
    a.w[1] = w1->w;
    a.s[1] = w1->scales;
    a.b[1] = w1->biases;
    wide = wide && al16(w1->scales) && (!w1->biases || al16(w1->biases));
  }
  a.N = w0->N;
  a.K = w0->K;
  a.gs = w0->group_size;
  a.wide_scales = wide ? 1 : 0;
  a.n_tiles = w1 ? w0->N / (kBN / 2) : w0->N / kBN;
  a.ldo = w0->N;
  a.out = out;
  float* next_gsum = pf.next_gsum;
  const moe_qweight* next_w = pf.next_w;
  a.out_p8 = w1 && pf.out_p8 ? 1 : 0;
  a.act = w1 ? pf.act : MOE_ACT_SWIGLU;
  if (w1 && next_gsum && next_w) {
    if (next_w->K != w0->N || kBN / 2 % next_w->group_size != 0) return MOE_E_INVALID_ARG;
    a.hsum = reinterpret_cast<uint16_t*>(next_gsum);
    a.hsum_nch = prefill_gsum_stride(next_w) / 16;
    a.hsum_gs = next_w->group_size;
    a.hsum_G = next_w->K / next_w->group_size;
  }
  // per XCD: an eighth of the 128- and 96-row tiles, then of the short ones
  // (n4 + n3 <= P/128 + slots, n2 + n1 <= slots: one remainder tile per expert)
  const int64_t nt = a.n_tiles;
  const int64_t grid = 8 * ((((P / 128 + slots) * nt + 7) / 8) + (2 * slots * nt + 7) / 8);
  if (grid > 0x7fffffffLL) return MOE_E_UNSUPPORTED;
  const unsigned g = static_cast<unsigned>(grid);
  const bool gact = a.act != MOE_ACT_SWIGLU;
  if (w0->bits == 4) {
    if (w1) return gact ? launch_prefill<4, true, true, true>(a, g, stream) : launch_prefill<4, true, true>(a, g, stream);
    return pf.in_p8 ? launch_prefill<4, false, true>(a, g, stream) : launch_prefill<4, false, false>(a, g, stream);
  }
  if (w1) return gact ? launch_prefill<8, true, true, true>(a, g, stream) : launch_prefill<8, true, true>(a, g, stream);
  return pf.in_p8 ? launch_prefill<8, false, true>(a, g, stream) : launch_prefill<8, false, false>(a, g, stream);
}

}  // namespace moe
