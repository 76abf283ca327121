// synth.cpp -- host-side data formats: the seeded synthetic-input generator and
// the MLX affine quantizer that produces the packed weights the kernels read.
//
// Generator: SplitMix64 (Steele, Lea, Flood 2014; the finalizer published by
// Vigna) gives one 64-bit draw per pair of elements (2i, 2i+1), split into two
// 23-bit uniforms in (0, 1) for a Box-Muller transform in fp32: element 2i takes
// the cosine branch, element 2i+1 the sine branch.  Every element depends only
// on (seed, tensor_id, index), so generation parallelises and any slice can be
// produced alone.
//
// Quantizer: the affine scheme of mx::quantize as used by the reference's
// converter (examples/convert.cpp:225) and read back by gather_qmm
// (src/common/switch_layers.cpp:94-102): per group, the scale spans the group's
// min..max over 2^bits - 1 steps, anchored on whichever edge has the larger
// magnitude; q = clip(round((w - bias)/scale)), packed least significant first:
// code c of a row at bits [c*bits, c*bits + bits) of the row's little-endian
// bit stream (at 6 bits, four codes per three bytes).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "moe_mi355x.h"

namespace {

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t stream_key(uint64_t seed, uint64_t tensor_id) {
  return mix64(seed + kGamma) ^ mix64(tensor_id * 0xD6E8FEB86659FD93ull + 0x632BE59BD9B4E019ull);
}

// Normals of pair p: (radius * cos(angle), radius * sin(angle)).
inline void normal_pair(uint64_t key, int64_t p, float* z0, float* z1) {
  const uint64_t r = mix64(key + static_cast<uint64_t>(p + 1) * kGamma);
  const float u1 = (static_cast<float>(r >> 41) + 0.5f) * (1.0f / 8388608.0f);
  const float u2 = (static_cast<float>((r >> 9) & 0x7FFFFFull) + 0.5f) * (1.0f / 8388608.0f);
  const float rad = std::sqrt(-2.0f * std::log(u1));
  const float ang = 6.28318530717958648f * u2;
  *z0 = rad * std::cos(ang);
  *z1 = rad * std::sin(ang);
}

// Calls f(i, z) for every element i in [b, e) of the stream.
template <class F>
inline void for_normals(uint64_t key, int64_t b, int64_t e, F&& f) {
  for (int64_t p = b >> 1; 2 * p < e; ++p) {
    float z0, z1;
    normal_pair(key, p, &z0, &z1);
    if (2 * p >= b) f(2 * p, z0);
    if (2 * p + 1 < e) f(2 * p + 1, z1);
  }
}

inline uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

inline float bf2f(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

template <class F>
void parallel_for(int64_t n, int64_t grain, F&& f) {
  unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const int64_t chunks = std::min<int64_t>(hw, (n + grain - 1) / grain);
  if (chunks <= 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  const int64_t per = (n + chunks - 1) / chunks;
  for (int64_t c = 0; c < chunks; ++c) {
    const int64_t b = c * per, e = std::min(n, b + per);
    if (b >= e) break;
    th.emplace_back([&f, b, e] { f(b, e); });
  }
  for (auto& t : th) t.join();
}

}  // namespace

extern "C" {

int moe_synth_normal_bf16(uint64_t seed, uint64_t tensor_id, float mean, float std_dev,
                          int64_t first, int64_t n, uint16_t* out) {
  if (n < 0 || first < 0 || (n > 0 && !out)) return MOE_E_INVALID_ARG;
  const uint64_t key = stream_key(seed, tensor_id);
  parallel_for(n, 1 << 16, [&](int64_t b, int64_t e) {
    for_normals(key, first + b, first + e,
                [&](int64_t i, float z) { out[i - first] = f2bf(mean + std_dev * z); });
  });
  return MOE_OK;
}

int moe_synth_normal_f32(uint64_t seed, uint64_t tensor_id, float mean, float std_dev,
                         int64_t first, int64_t n, float* out) {
  if (n < 0 || first < 0 || (n > 0 && !out)) return MOE_E_INVALID_ARG;
  const uint64_t key = stream_key(seed, tensor_id);
  parallel_for(n, 1 << 16, [&](int64_t b, int64_t e) {
    for_normals(key, first + b, first + e,
                [&](int64_t i, float z) { out[i - first] = mean + std_dev * z; });
  });
  return MOE_OK;
}

int moe_quantize_affine(const uint16_t* w, int64_t rows, int32_t K, int32_t group_size,
                        int32_t bits, uint32_t* wq, uint16_t* scales, uint16_t* biases) {
  if (!w || !wq || !scales || !biases || rows < 0 || K <= 0) return MOE_E_INVALID_ARG;
  if (bits < 2 || bits > 8 || bits == 7) return MOE_E_UNSUPPORTED;
  // every group starts on a 32-bit word
  if (group_size <= 0 || K % group_size != 0 || (static_cast<int64_t>(group_size) * bits) % 32 != 0)
    return MOE_E_UNSUPPORTED;
  const int64_t words = static_cast<int64_t>(K) * bits / 32;  // per row
  const int32_t groups = K / group_size;
  const float n_bins = static_cast<float>((1 << bits) - 1);
  parallel_for(rows, 64, [&](int64_t rb, int64_t re) {
    std::vector<uint32_t> q(group_size);
    for (int64_t r = rb; r < re; ++r) {
      const uint16_t* wr = w + r * K;
      uint32_t* qr = wq + r * words;
      for (int32_t g = 0; g < groups; ++g) {
        const uint16_t* wg = wr + static_cast<int64_t>(g) * group_size;
        float wmax = bf2f(wg[0]), wmin = wmax;
        for (int32_t i = 1; i < group_size; ++i) {
          const float v = bf2f(wg[i]);
          wmax = std::max(wmax, v);
          wmin = std::min(wmin, v);
        }
        float scale = std::max((wmax - wmin) / n_bins, 1e-7f);
        float edge;
        if (std::fabs(wmin) > std::fabs(wmax)) {
          edge = wmin;
        } else {
          scale = -scale;
          edge = wmax;
        }
        const float q0 = std::nearbyint(edge / scale);
        if (q0 != 0.0f) scale = edge / q0;
        const float bias = (q0 == 0.0f) ? 0.0f : edge;
        for (int32_t i = 0; i < group_size; ++i) {
          float v = std::nearbyint((bf2f(wg[i]) - bias) / scale);
          v = std::min(std::max(v, 0.0f), n_bins);
          q[i] = static_cast<uint32_t>(v);
        }
        // the group's words: its codes at consecutive bit offsets
        const int64_t w0 = static_cast<int64_t>(g) * group_size * bits / 32;
        const int64_t nw = static_cast<int64_t>(group_size) * bits / 32;
        for (int64_t i = 0; i < nw; ++i) qr[w0 + i] = 0u;
        for (int32_t i = 0; i < group_size; ++i) {
          const int64_t bit = static_cast<int64_t>(i) * bits;
          const uint64_t v = static_cast<uint64_t>(q[i]) << (bit & 31);
          qr[w0 + (bit >> 5)] |= static_cast<uint32_t>(v);
          if ((bit & 31) + bits > 32) qr[w0 + (bit >> 5) + 1] |= static_cast<uint32_t>(v >> 32);
        }
        scales[r * groups + g] = f2bf(scale);
        biases[r * groups + g] = f2bf(bias);
      }
    }
  });
  return MOE_OK;
}

}  // extern "C"
