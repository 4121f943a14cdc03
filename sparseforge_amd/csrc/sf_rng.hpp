// Counter-based random numbers for the sparse-training hot path.
//
// The generator is SplitMix64 (G. Steele, D. Lea, C. Flood, "Fast splittable
// pseudorandom number generators", OOPSLA 2014) used as a stateless hash of
// (seed, counter): value(seed, c) = mix64(seed + (c + 1) * 0x9E3779B97F4A7C15).
// Being a pure function of its counter, it is reproducible on the host (the
// test oracle restates it in numpy) and needs no per-thread state on the GPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sf {

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t counter_hash(uint64_t seed, uint64_t ctr) {
  return mix64(seed + (ctr + 1ull) * 0x9E3779B97F4A7C15ull);
}

// Uniform integer in [0, n) by the multiply-high method (D. Lemire, "Fast
// random integer generation in an interval", 2019) without the rejection
// step; the bias is below n / 2^64.
__host__ __device__ __forceinline__ uint64_t uniform_below(uint64_t x, uint64_t n) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul64hi(x, n);
#else
  return static_cast<uint64_t>((static_cast<unsigned __int128>(x) * n) >> 64);
#endif
}

// Rademacher sign for element i: bit (i % 64) of counter_hash(seed, i / 64).
__host__ __device__ __forceinline__ float rademacher(uint64_t seed, uint64_t i) {
  uint64_t h = counter_hash(seed, i >> 6);
  return ((h >> (i & 63)) & 1ull) ? 1.0f : -1.0f;
}

}  // namespace sf
