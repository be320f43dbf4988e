// Counter-based random numbers for the draw's uniforms: Philox4x32-10, the generator of
// J. K. Salmon, M. A. Moraes, R. O. Dror and D. E. Shaw, "Parallel Random Numbers: As Easy
// as 1, 2, 3" (SC 2011), written from the paper: ten rounds of
//   (hi0, lo0) = mulhilo(0xD2511F53, c0); (hi1, lo1) = mulhilo(0xCD9E8D57, c2);
//   c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0);  k += (0x9E3779B9, 0xBB67AE85)
// (the key is bumped between rounds, not after the last).
//
// A sampled row with a seed draws its uniform from the counter (step_lo, step_hi,
// NS_PHILOX_TAG, 0) under the key (seed_lo, seed_hi), step the number of tokens in the
// row's history: the same seed and history give the same uniform on every call, and each
// decode step of a request a fresh one.  The first output word's top 24 bits, times 2^-24,
// is the uniform (a float32 in [0, 1)).
#pragma once

#include <stdint.h>

namespace ns {

constexpr uint32_t PHILOX_M0 = 0xD2511F53u, PHILOX_M1 = 0xCD9E8D57u;
constexpr uint32_t PHILOX_W0 = 0x9E3779B9u, PHILOX_W1 = 0xBB67AE85u;
constexpr uint32_t NS_PHILOX_TAG = 0x4E53534Du;   // "NSSM": the counter word that marks sampler draws

struct Philox4 {
  uint32_t x, y, z, w;
};

__host__ __device__ __forceinline__ Philox4 philox4x32_10(Philox4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)PHILOX_M0 * c.x;
    const uint64_t p1 = (uint64_t)PHILOX_M1 * c.z;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    c = Philox4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    if (r < 9) {
      k0 += PHILOX_W0;
      k1 += PHILOX_W1;
    }
  }
  return c;
}

// The uniform of a seeded row: see the header comment.
__host__ __device__ __forceinline__ float seeded_uniform(uint64_t seed, int64_t step) {
  const uint64_t s = (uint64_t)step;
  const Philox4 o = philox4x32_10(Philox4{(uint32_t)s, (uint32_t)(s >> 32), NS_PHILOX_TAG, 0u}, (uint32_t)seed,
                                  (uint32_t)(seed >> 32));
  return (float)(o.x >> 8) * 0x1.0p-24f;
}

}  // namespace ns
