// synth.cpp — the benchmarks' synthetic weights (host code): seeded N(0, std^2)
// F32 values, counter-based so that any split of the index range over calls
// or threads gives the same numbers. The reference loads trained weights from
// a GGUF file (src/model.cpp:164-311); the benchmark configurations here use
// random-init weights of the same architecture instead.
//
// Sample k of stream `seed`: Box-Muller pair j = k / 2 takes splitmix64
// outputs 2j+1 and 2j+2 (splitmix64 output i mixes seed + i * 0x9E3779B97F4A7C15),
// u1 = ((z1 >> 11) + 1) * 2^-53 in (0, 1], u2 = (z2 >> 11) * 2^-53 in [0, 1),
// r = sqrt(-2 ln u1); sample 2j = r cos(2 pi u2), 2j+1 = r sin(2 pi u2); then
// times std in double and one rounding to float.
#include <cerrno>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

#include "../../include/ikv_model.h"

namespace {

inline uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + i * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void fill(uint64_t seed, uint64_t first, size_t n, double std, float *out) {
  constexpr double kTwoPi = 6.283185307179586476925286766559;
  const double scale = 1.0 / 9007199254740992.0;  // 2^-53
  size_t i = 0;
  while (i < n) {
    const uint64_t k = first + i;
    const uint64_t j = k >> 1;
    const uint64_t z1 = splitmix64_at(seed, 2 * j + 1);
    const uint64_t z2 = splitmix64_at(seed, 2 * j + 2);
    const double u1 = (static_cast<double>(z1 >> 11) + 1.0) * scale;
    const double u2 = static_cast<double>(z2 >> 11) * scale;
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double a = kTwoPi * u2;
    if ((k & 1) == 0) {
      out[i++] = static_cast<float>(r * std::cos(a) * std);
      if (i < n) out[i++] = static_cast<float>(r * std::sin(a) * std);
    } else {
      out[i++] = static_cast<float>(r * std::sin(a) * std);
    }
  }
}

}  // namespace

extern "C" int ikv_synth_normal_f32(uint64_t seed, uint64_t offset, size_t n, double std,
                                    float *out_host, int threads) {
  if (!out_host && n) return -EINVAL;
  if (n == 0) return 0;
  size_t t = threads > 1 ? static_cast<size_t>(threads) : 1;
  if (t > 256) t = 256;
  const size_t min_chunk = 1 << 16;
  if (t > 1 && n / t < min_chunk) t = n / min_chunk > 0 ? n / min_chunk : 1;
  if (t == 1) {
    fill(seed, offset, n, std, out_host);
    return 0;
  }
  const size_t chunk = (n + t - 1) / t;
  std::vector<std::thread> pool;
  for (size_t b = 0; b < n; b += chunk) {
    const size_t len = n - b < chunk ? n - b : chunk;
    pool.emplace_back(fill, seed, offset + b, len, std, out_host + b);
  }
  for (auto &th : pool) th.join();
  return 0;
}
