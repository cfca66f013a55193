// Threefry-2x32 with 20 rounds (Salmon et al., "Parallel random numbers: as
// easy as 1, 2, 3", SC'11), the block cipher behind jax.random's default key
// type, and the 32-bit random words jax 0.10.2 draws from a key with
// threefry_partitionable on: word i of an array of any shape is out0 ^ out1 of
// threefry2x32(key, (i >> 32, i & 0xffffffff)), i the row-major flat index.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ppo {

__device__ __forceinline__ uint32_t rotl32(uint32_t v, uint32_t r) {
  return (v << r) | (v >> (32u - r));
}

__device__ __forceinline__ void threefry2x32(uint32_t k0, uint32_t k1, uint32_t& x0, uint32_t& x1) {
  const uint32_t ks2 = k0 ^ k1 ^ 0x1BD11BDAu;
  const uint32_t ks[3] = {k0, k1, ks2};
  x0 += k0;
  x1 += k1;
#pragma unroll
  for (uint32_t s = 1; s <= 5; ++s) {
    const uint32_t r0 = (s & 1) ? 13u : 17u;
    const uint32_t r1 = (s & 1) ? 15u : 29u;
    const uint32_t r2 = (s & 1) ? 26u : 16u;
    const uint32_t r3 = (s & 1) ? 6u : 24u;
    x0 += x1; x1 = rotl32(x1, r0); x1 ^= x0;
    x0 += x1; x1 = rotl32(x1, r1); x1 ^= x0;
    x0 += x1; x1 = rotl32(x1, r2); x1 ^= x0;
    x0 += x1; x1 = rotl32(x1, r3); x1 ^= x0;
    x0 += ks[s % 3];
    x1 += ks[(s + 1) % 3] + s;
  }
}

// Word i of jax.random.bits(key, shape, uint32) (flat index i).
__device__ __forceinline__ uint32_t random_word(uint32_t k0, uint32_t k1, uint64_t i) {
  uint32_t x0 = (uint32_t)(i >> 32), x1 = (uint32_t)(i & 0xffffffffu);
  threefry2x32(k0, k1, x0, x1);
  return x0 ^ x1;
}

// A float in [0, 1) from a 32-bit word as jax.random.uniform forms it: the top
// 23 bits become the mantissa of a float in [1, 2), then 1 is subtracted.
__device__ __forceinline__ float unit_float(uint32_t w) {
  return __uint_as_float((w >> 9) | 0x3f800000u) - 1.0f;
}

}  // namespace ppo
