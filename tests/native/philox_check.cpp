// CPU cross-check of the sampler's Philox4x32-10 (ns::philox4x32_10, csrc/ns_rng.h, a
// __host__ __device__ function) against rocRAND's engine (an independent implementation,
// rocrand_philox4x32_10.h): for key = (seed low, seed high) and counter
// (c0, c1, c2, c3), rocRAND's engine seeded with (seed, subsequence = c2 | c3 << 32,
// offset = 4 * (c0 | c1 << 32)) returns that counter's output first.  Prints
// "seed c0 c1 c2 c3 x0 x1 x2 x3" per case (the test compares them with the numpy
// restatement too) and "mismatches N".
#include <hip/hip_runtime.h>
#include <rocrand/rocrand_philox4x32_10.h>

#include <cstdint>
#include <cstdio>

#include "ns_rng.h"

int main() {
  uint64_t state = 0x9E3779B97F4A7C15ull;
  auto next = [&]() {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return state;
  };
  int bad = 0, n = 0;
  for (int i = 0; i < 2000; ++i) {
    const uint64_t seed = i < 3 ? (i == 0 ? 0ull : (i == 1 ? ~0ull : 42ull)) : next();
    const uint64_t lo = i % 7 == 0 ? (uint64_t)i : next() >> (i % 40);
    const uint64_t hi = i % 5 == 0 ? (uint64_t)ns::NS_PHILOX_TAG : next();
    const ns::Philox4 ctr{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
    const ns::Philox4 mine = ns::philox4x32_10(ctr, (uint32_t)seed, (uint32_t)(seed >> 32));
    if (lo >= (1ull << 62)) continue;   // rocRAND's offset counts words: 4 * lo must not overflow
    rocrand_device::philox4x32_10_engine eng(seed, hi, 4ull * lo);
    const uint4 ref = eng.next4();
    ++n;
    if (ref.x != mine.x || ref.y != mine.y || ref.z != mine.z || ref.w != mine.w) ++bad;
    if (i < 64)
      std::printf("%llu %u %u %u %u %u %u %u %u\n", (unsigned long long)seed, ctr.x, ctr.y, ctr.z, ctr.w, mine.x,
                  mine.y, mine.z, mine.w);
  }
  std::printf("cases %d mismatches %d\n", n, bad);
  return bad != 0;
}
