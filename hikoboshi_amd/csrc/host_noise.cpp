// Backbone coordinate noise on the host, in the reference's draw order
// (cpp/algorithms/inverse_fold.cpp:191-207): a 64-bit Mersenne Twister seeded
// with seed ^ 0x4D504E4E76343875 feeds std::normal_distribution<float>(0,
// sigma); every present atom (AtomSource != Missing) gets x, y, z offsets in
// that order. The distribution is the standard library's own, so results
// match the reference when both use the same C++ library; this file is
// compiled without floating-point contraction like the reference.
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <random>

namespace hkbs {

void backbone_noise_host(const float* coords, const uint8_t* atom_sources, int32_t L, float sigma, uint64_t seed,
                         float* out) {
  const size_t n_atoms = static_cast<size_t>(L) * 5;
  std::memmove(out, coords, n_atoms * 3 * sizeof(float));
  std::mt19937_64 rng(seed ^ 0x4D504E4E76343875ull);
  std::normal_distribution<float> normal(0.0F, sigma);
  for (size_t a = 0; a < n_atoms; ++a) {
    if (atom_sources[a] == 0) continue;
    out[a * 3 + 0] += normal(rng);
    out[a * 3 + 1] += normal(rng);
    out[a * 3 + 2] += normal(rng);
  }
}

}  // namespace hkbs
