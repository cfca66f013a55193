// Minibatch order of the learner: Threefry-2x32 key splitting and the
// sort-based shuffle behind jax.random.permutation, as used by
// boonta/algorithms/ppo.py:199-201,230-231 (T*N samples per epoch) and
// boonta/algorithms/recurrent_ppo.py:269-279 (N envs per epoch).
//
// Algorithm (jax 0.10.2 with threefry_partitionable, restated):
//   split(key, n)[i] = threefry2x32(key, (i >> 32, i & 0xffffffff))
//   bits32(key)[i]   = out0 ^ out1 of the same call
//   permutation(key, n): x = arange(n); repeat ceil(3 ln n / ln(2^32-1)) times:
//       key, sub = split(key); x = stable_sort_by_key(bits32(sub)[0:n], x)
//
// The stable sort is an LSD radix sort over four 8-bit digits.  Each pass has
// three kernels: per-tile digit counts, one exclusive scan over the
// (digit, tile) table, and a scatter that ranks equal digits in input order
// with wavefront ballots (8 ballots give each lane the mask of lanes holding
// its digit), so the result is bit-identical to any stable sort.
#include "common.h"

#include <algorithm>
#include <math.h>
#include <utility>

namespace {

constexpr int RADIX_BITS = 8;
constexpr int RADIX = 1 << RADIX_BITS;
constexpr int SORT_THREADS = 256;
constexpr int SORT_ITEMS = 16;  // items per thread
constexpr int SORT_TILE = SORT_THREADS * SORT_ITEMS;
constexpr int SORT_WAVES = SORT_THREADS / 64;

__device__ __forceinline__ uint32_t rotl(uint32_t v, uint32_t r) {
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
    x0 += x1; x1 = rotl(x1, r0); x1 ^= x0;
    x0 += x1; x1 = rotl(x1, r1); x1 ^= x0;
    x0 += x1; x1 = rotl(x1, r2); x1 ^= x0;
    x0 += x1; x1 = rotl(x1, r3); x1 ^= x0;
    x0 += ks[s % 3];
    x1 += ks[(s + 1) % 3] + s;
  }
}

// keys[2*i..2*i+1] = split(key, num)[i]
__global__ void split_kernel(const uint32_t* __restrict__ key, uint32_t* __restrict__ out, int64_t num) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= num) return;
  uint32_t x0 = (uint32_t)((uint64_t)i >> 32), x1 = (uint32_t)((uint64_t)i & 0xffffffffu);
  threefry2x32(key[0], key[1], x0, x1);
  out[2 * i] = x0;
  out[2 * i + 1] = x1;
}

// One shuffle round's sort keys: bits32(subkey) with subkey = split(key, 2)[1],
// plus the iota values on the first round.
__global__ void round_bits_kernel(const uint32_t* __restrict__ key_in,
                                  uint32_t* __restrict__ sort_keys, int32_t* __restrict__ vals,
                                  int64_t n, int first_round) {
  const uint32_t k0 = key_in[0], k1 = key_in[1];
  uint32_t s0 = 0, s1 = 1;  // split(key, 2)[1] = threefry(key, (0, 1))
  threefry2x32(k0, k1, s0, s1);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t x0 = (uint32_t)((uint64_t)i >> 32), x1 = (uint32_t)((uint64_t)i & 0xffffffffu);
    threefry2x32(s0, s1, x0, x1);
    sort_keys[i] = x0 ^ x1;
    if (first_round) vals[i] = (int32_t)i;
  }
}

// Writes split(key, 2)[0] into key_out; launched after round_bits_kernel so an
// in-place update cannot race with its readers.
__global__ void advance_key_kernel(const uint32_t* key_in, uint32_t* key_out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    uint32_t x0 = 0, x1 = 0;
    threefry2x32(key_in[0], key_in[1], x0, x1);
    key_out[0] = x0;
    key_out[1] = x1;
  }
}

__global__ void __launch_bounds__(SORT_THREADS)
radix_hist_kernel(const uint32_t* __restrict__ keys, int64_t n, int shift, uint32_t* __restrict__ hist,
                  int tiles) {
  __shared__ uint32_t cnt[RADIX];
  for (int d = threadIdx.x; d < RADIX; d += SORT_THREADS) cnt[d] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * SORT_TILE;
#pragma unroll
  for (int it = 0; it < SORT_ITEMS; ++it) {
    const int64_t i = base + (int64_t)it * SORT_THREADS + threadIdx.x;
    if (i < n) atomicAdd(&cnt[(keys[i] >> shift) & (RADIX - 1)], 1u);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < RADIX; d += SORT_THREADS) hist[(int64_t)d * tiles + blockIdx.x] = cnt[d];
}

// Exclusive scan of hist[RADIX * tiles] (digit-major) in one workgroup:
// thread d totals digit d over the tiles, one LDS scan turns the 256 totals
// into digit bases, and each thread then rewrites its row as running offsets.
__global__ void __launch_bounds__(RADIX) radix_scan_kernel(uint32_t* __restrict__ hist, int tiles) {
  __shared__ uint32_t base[RADIX];
  const int d = threadIdx.x;
  uint32_t* row = hist + (int64_t)d * tiles;
  uint32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  int t = 0;
  for (; t + 3 < tiles; t += 4) {
    s0 += row[t];
    s1 += row[t + 1];
    s2 += row[t + 2];
    s3 += row[t + 3];
  }
  for (; t < tiles; ++t) s0 += row[t];
  base[d] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  for (int off = 1; off < RADIX; off <<= 1) {
    const uint32_t v = d >= off ? base[d - off] : 0u;
    __syncthreads();
    base[d] += v;
    __syncthreads();
  }
  uint32_t run = d ? base[d - 1] : 0u;
  for (t = 0; t < tiles; ++t) {
    const uint32_t v = row[t];
    row[t] = run;
    run += v;
  }
}

// Stable scatter of one 8-bit digit.  Wave w of a tile owns the contiguous
// items [w * 64 * SORT_ITEMS, (w+1) * 64 * SORT_ITEMS) and walks them in order
// 64 at a time, so counting equal digits in lane order inside each step and
// accumulating across steps and waves gives the stable rank.
__global__ void __launch_bounds__(SORT_THREADS)
radix_scatter_kernel(const uint32_t* __restrict__ keys_in, const int32_t* __restrict__ vals_in,
                     uint32_t* __restrict__ keys_out, int32_t* __restrict__ vals_out, int64_t n,
                     int shift, const uint32_t* __restrict__ offsets, int tiles) {
  __shared__ uint32_t wcount[SORT_WAVES][RADIX];
  __shared__ uint32_t base_off[RADIX];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int d = threadIdx.x; d < RADIX; d += SORT_THREADS) {
    base_off[d] = offsets[(int64_t)d * tiles + blockIdx.x];
#pragma unroll
    for (int w = 0; w < SORT_WAVES; ++w) wcount[w][d] = 0;
  }
  __syncthreads();
  const uint64_t lt_mask = lane ? (~0ull >> (64 - lane)) : 0ull;
  const int64_t wbase = (int64_t)blockIdx.x * SORT_TILE + (int64_t)wave * 64 * SORT_ITEMS;
  uint32_t key[SORT_ITEMS];
  int32_t val[SORT_ITEMS];
  uint32_t rank[SORT_ITEMS];
#pragma unroll
  for (int it = 0; it < SORT_ITEMS; ++it) {
    const int64_t i = wbase + (int64_t)it * 64 + lane;
    const bool ok = i < n;
    key[it] = ok ? keys_in[i] : 0u;
    val[it] = ok ? vals_in[i] : 0;
    const uint32_t d = (key[it] >> shift) & (RADIX - 1);
    uint64_t match = __ballot(ok);
#pragma unroll
    for (int b = 0; b < RADIX_BITS; ++b) {
      const uint64_t bal = __ballot((d >> b) & 1u);
      match &= ((d >> b) & 1u) ? bal : ~bal;
    }
    const uint32_t before = ok ? wcount[wave][d] : 0u;
    const uint32_t within = (uint32_t)__popcll(match & lt_mask);
    // every lane has read the running count before the group leader bumps it
    __builtin_amdgcn_wave_barrier();
    if (ok && within == 0) wcount[wave][d] = before + (uint32_t)__popcll(match);
    __builtin_amdgcn_wave_barrier();
    rank[it] = before + within;
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < SORT_ITEMS; ++it) {
    const int64_t i = wbase + (int64_t)it * 64 + lane;
    if (i >= n) continue;
    const uint32_t d = (key[it] >> shift) & (RADIX - 1);
    uint32_t off = base_off[d];
    for (int w = 0; w < wave; ++w) off += wcount[w][d];
    off += rank[it];
    keys_out[off] = key[it];
    vals_out[off] = val[it];
  }
}

int shuffle_rounds(int64_t n) {
  const double m = n > 1 ? (double)n : 1.0;
  return (int)ceil(3.0 * log(m) / log(4294967295.0));
}

struct SortSpace {
  uint32_t* keys_a;
  uint32_t* keys_b;
  int32_t* vals_b;
  uint32_t* hist;
  uint32_t* key;  // running round key [2]
};

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

size_t sort_space_bytes(int64_t n) {
  const int64_t tiles = ppo::ceil_div64(n > 0 ? n : 1, SORT_TILE);
  return 2 * align256(sizeof(uint32_t) * n) + align256(sizeof(int32_t) * n) +
         align256(sizeof(uint32_t) * RADIX * tiles) + 256;
}

SortSpace carve(void* ws, int64_t n) {
  const int64_t tiles = ppo::ceil_div64(n > 0 ? n : 1, SORT_TILE);
  char* p = (char*)ws;
  SortSpace s;
  s.keys_a = (uint32_t*)p; p += align256(sizeof(uint32_t) * n);
  s.keys_b = (uint32_t*)p; p += align256(sizeof(uint32_t) * n);
  s.vals_b = (int32_t*)p; p += align256(sizeof(int32_t) * n);
  s.hist = (uint32_t*)p; p += align256(sizeof(uint32_t) * RADIX * tiles);
  s.key = (uint32_t*)p;
  return s;
}

// permutation(key, n) into out (device); key is a device pointer to 2 words.
int permutation_impl(hipStream_t st, const uint32_t* key, int32_t* out, int64_t n, void* ws) {
  if (n <= 0) return PPO_OK;
  SortSpace s = carve(ws, n);
  const int tiles = (int)ppo::ceil_div64(n, SORT_TILE);
  const int rounds = shuffle_rounds(n);
  if (rounds == 0) {
    // n <= 1: the identity
    hipLaunchKernelGGL(round_bits_kernel, dim3(1), dim3(64), 0, st, key, s.keys_a, out, n, 1);
    return ppo::check_launch("ppo_permutation");
  }
  const int bits_blocks = (int)std::min<int64_t>(ppo::ceil_div64(n, 256), 4096);
  for (int r = 0; r < rounds; ++r) {
    const uint32_t* kr = r == 0 ? key : s.key;
    hipLaunchKernelGGL(round_bits_kernel, dim3(bits_blocks), dim3(256), 0, st, kr, s.keys_a, out, n,
                       r == 0 ? 1 : 0);
    if (r + 1 < rounds) hipLaunchKernelGGL(advance_key_kernel, dim3(1), dim3(64), 0, st, kr, s.key);
    uint32_t* kin = s.keys_a;
    int32_t* vin = out;
    uint32_t* kout = s.keys_b;
    int32_t* vout = s.vals_b;
    for (int pass = 0; pass < 32 / RADIX_BITS; ++pass) {
      const int shift = pass * RADIX_BITS;
      hipLaunchKernelGGL(radix_hist_kernel, dim3(tiles), dim3(SORT_THREADS), 0, st, kin, n, shift,
                         s.hist, tiles);
      hipLaunchKernelGGL(radix_scan_kernel, dim3(1), dim3(RADIX), 0, st, s.hist, tiles);
      hipLaunchKernelGGL(radix_scatter_kernel, dim3(tiles), dim3(SORT_THREADS), 0, st, kin, vin, kout,
                         vout, n, shift, s.hist, tiles);
      std::swap(kin, kout);
      std::swap(vin, vout);
    }
    // an even number of passes leaves the values back in `out`
  }
  return ppo::check_launch("ppo_permutation");
}

}  // namespace

PPO_EXPORT size_t ppo_permutation_workspace(int64_t n) { return sort_space_bytes(n); }

PPO_EXPORT int ppo_threefry_split(void* stream, const uint32_t* key, uint32_t* out, int64_t num) {
  if (num < 0 || !key || !out) return ppo::set_error(PPO_ERR_ARG, "ppo_threefry_split: bad argument");
  if (num == 0) return PPO_OK;
  hipLaunchKernelGGL(split_kernel, dim3((unsigned)ppo::ceil_div64(num, 256)), dim3(256), 0,
                     ppo::as_stream(stream), key, out, num);
  return ppo::check_launch("ppo_threefry_split");
}

PPO_EXPORT int ppo_permutation(void* stream, const uint32_t* key, int32_t* out, int64_t n, void* workspace,
                               size_t workspace_bytes) {
  if (n < 0 || n > INT32_MAX || !key || (n > 0 && !out))
    return ppo::set_error(PPO_ERR_ARG, "ppo_permutation: bad argument (n=%lld)", (long long)n);
  if (workspace_bytes < sort_space_bytes(n) || (n > 0 && !workspace))
    return ppo::set_error(PPO_ERR_SPACE, "ppo_permutation: workspace %zu < %zu bytes", workspace_bytes,
                          sort_space_bytes(n));
  return permutation_impl(ppo::as_stream(stream), key, out, n, workspace);
}

// out[e * n + i] = permutation(split(key, epochs)[e], n)[i]; epoch keys are
// written to the first 2 * epochs words after the sort space in `workspace`.
PPO_EXPORT size_t ppo_epoch_permutations_workspace(int epochs, int64_t n) {
  return sort_space_bytes(n) + align256(sizeof(uint32_t) * 2 * (epochs > 0 ? epochs : 1));
}

PPO_EXPORT int ppo_epoch_permutations(void* stream, const uint32_t* key, int epochs, int64_t n, int32_t* out,
                                      void* workspace, size_t workspace_bytes) {
  if (epochs < 0 || n < 0 || n > INT32_MAX || !key || (epochs > 0 && n > 0 && !out))
    return ppo::set_error(PPO_ERR_ARG, "ppo_epoch_permutations: bad argument");
  if (workspace_bytes < ppo_epoch_permutations_workspace(epochs, n) || !workspace)
    return ppo::set_error(PPO_ERR_SPACE, "ppo_epoch_permutations: workspace too small");
  if (epochs == 0) return PPO_OK;
  hipStream_t st = ppo::as_stream(stream);
  uint32_t* keys = (uint32_t*)((char*)workspace + sort_space_bytes(n));
  hipLaunchKernelGGL(split_kernel, dim3((unsigned)ppo::ceil_div64(epochs, 64)), dim3(64), 0, st, key, keys,
                     (int64_t)epochs);
  for (int e = 0; e < epochs; ++e) {
    int rc = permutation_impl(st, keys + 2 * e, out + (int64_t)e * n, n, workspace);
    if (rc) return rc;
  }
  return ppo::check_launch("ppo_epoch_permutations");
}
