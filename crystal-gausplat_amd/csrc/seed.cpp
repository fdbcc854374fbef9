// Seeded synthetic data shared by the context and the tests.
//
// The reference draws weights with an unseeded Random + Box-Muller
// (src/core/tensor.cr:116-140); the configurations here need reproducible
// "seed 0" values on any host, so the stream is SplitMix64 keyed by
// (seed, FNV-1a(tensor name)), counter-based so large tensors fill in
// parallel. Value i of a stream = mix64(key + (i+1) * 0x9E3779B97F4A7C15).
// uniform24(x) = (x >> 40) * 2^-24. Normal pair p: u1 = ((x_{2p} >> 40) + 1)
// * 2^-24, u2 = uniform24(x_{2p+1}), r = sqrt(-2 ln u1), z = r cos(2 pi u2),
// r sin(2 pi u2), all in double, rounded once to fp32.
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/gs_hip.h"

namespace {

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t fnv1a(const char* s) {
  uint64_t h = 0xCBF29CE484222325ULL;
  for (; *s; ++s) {
    h ^= (uint8_t)*s;
    h *= 0x100000001B3ULL;
  }
  return h;
}

inline uint64_t stream_key(uint64_t seed, const char* name) {
  return mix64(seed ^ mix64(fnv1a(name)));
}

inline uint64_t draw(uint64_t key, uint64_t i) {
  return mix64(key + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

template <class F>
void parallel_chunks(int64_t n, F&& f) {
  const int64_t chunk = 1 << 20;
  const int64_t nchunks = (n + chunk - 1) / chunk;
  unsigned hw = std::thread::hardware_concurrency();
  int nt = (int)std::min<int64_t>(nchunks, hw ? std::min(hw, 16u) : 4u);
  if (nt <= 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  for (int t = 0; t < nt; ++t)
    th.emplace_back([&, t]() {
      for (int64_t c = t; c < nchunks; c += nt) f(c * chunk, std::min(n, (c + 1) * chunk));
    });
  for (auto& x : th) x.join();
}

}  // namespace

extern "C" void gs_seed_normal(uint64_t seed, const char* name, float mean, float std,
                               float* out, int64_t n) {
  const uint64_t key = stream_key(seed, name);
  const double two_pi = 6.283185307179586476925286766559;
  const int64_t npairs = (n + 1) / 2;
  parallel_chunks(npairs, [&](int64_t p0, int64_t p1) {
    for (int64_t p = p0; p < p1; ++p) {
      const double u1 = (double)((draw(key, 2 * p) >> 40) + 1) * (1.0 / 16777216.0);
      const double u2 = (double)(draw(key, 2 * p + 1) >> 40) * (1.0 / 16777216.0);
      const double r = sqrt(-2.0 * log(u1));
      const double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
      out[2 * p] = (float)((double)mean + (double)std * z0);
      if (2 * p + 1 < n) out[2 * p + 1] = (float)((double)mean + (double)std * z1);
    }
  });
}

extern "C" void gs_seed_uniform(uint64_t seed, const char* name, float lo, float hi,
                                float* out, int64_t n) {
  const uint64_t key = stream_key(seed, name);
  parallel_chunks(n, [&](int64_t i0, int64_t i1) {
    for (int64_t i = i0; i < i1; ++i) {
      const double u = (double)(draw(key, i) >> 40) * (1.0 / 16777216.0);
      out[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
    }
  });
}
