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
// A stable sort by 32-bit keys is the same as a sort by the unique 64-bit
// pair (key, position).  Each shuffle round therefore runs as an MSD bucket
// sort, for all epochs at once (grid.y = epoch):
//   1. bits: the round's sort keys, and per 4096-element tile a histogram of
//      the top b key bits (b sized for ~512 elements per bucket);
//   2. scan: bucket bases and per-(bucket, tile) offsets;
//   3. scatter: every element, with its position, into its bucket (order
//      inside a bucket does not matter);
//   4. sort: one workgroup per bucket sorts (key, position) pairs in LDS with a
//      bitonic network and writes the values in order.
// A bucket larger than the LDS capacity (not reachable for Threefry keys at
// these sizes, but handled) is ranked by counting instead, which is exact.
#include "common.h"
#include "threefry.h"

#include <algorithm>
#include <math.h>
#include <mutex>
#include <utility>

namespace {

using ppo::threefry2x32;

constexpr int TILE = 4096;          // elements per histogram / scatter block
constexpr int TILE_THREADS = 256;
constexpr int BUCKET_CAP = 4096;    // elements a bucket sorts in LDS
constexpr int SORT_THREADS = 512;
constexpr int MAX_BUCKET_BITS = 12;

// keys[2*i..2*i+1] = split(key, num)[i]
__global__ void split_kernel(const uint32_t* __restrict__ key, uint32_t* __restrict__ out, int64_t num) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= num) return;
  uint32_t x0 = (uint32_t)((uint64_t)i >> 32), x1 = (uint32_t)((uint64_t)i & 0xffffffffu);
  threefry2x32(key[0], key[1], x0, x1);
  out[2 * i] = x0;
  out[2 * i + 1] = x1;
}

// The subkey of shuffle round `round` of epoch e: the epoch key is
// split(key, E)[e] (or key itself when `split_epochs` is 0); each round takes
// (key, sub) = split(key).
__device__ __forceinline__ void round_subkey(const uint32_t* key, int split_epochs, int e, int round, uint32_t& s0,
                                             uint32_t& s1) {
  uint32_t k0 = key[0], k1 = key[1];
  if (split_epochs) {
    uint32_t x0 = 0, x1 = (uint32_t)e;
    threefry2x32(k0, k1, x0, x1);
    k0 = x0;
    k1 = x1;
  }
  for (int r = 0; r < round; ++r) {
    uint32_t x0 = 0, x1 = 0;
    threefry2x32(k0, k1, x0, x1);
    k0 = x0;
    k1 = x1;
  }
  s0 = 0;
  s1 = 1;
  threefry2x32(k0, k1, s0, s1);
}

struct ShuffleArgs {
  const uint32_t* key;  // device key data [2]
  int split_epochs;
  int64_t n;
  int tiles;
  int bbits;            // bucket bits (0: one bucket)
  int nb;               // 1 << bbits
  int round;
  int32_t* out;         // [E][n]: values in, values out
  uint32_t* keys;       // [E][n]
  uint32_t* hist;       // [E][nb][tiles]
  uint32_t* bstart;     // [E][nb + 1]
  uint32_t* tkey;       // [E][n] bucketed keys
  uint32_t* tpos;       // [E][n] bucketed positions
  int32_t* tval;        // [E][n] bucketed values
};

__device__ __forceinline__ uint32_t bucket_of(uint32_t k, int bbits) {
  return bbits ? (k >> (32 - bbits)) : 0u;
}

__global__ void __launch_bounds__(TILE_THREADS) shuffle_bits_kernel(ShuffleArgs a) {
  extern __shared__ uint32_t cnt[];  // [nb]
  const int e = blockIdx.y;
  for (int d = threadIdx.x; d < a.nb; d += TILE_THREADS) cnt[d] = 0;
  __syncthreads();
  uint32_t s0, s1;
  round_subkey(a.key, a.split_epochs, e, a.round, s0, s1);
  const int64_t base = (int64_t)blockIdx.x * TILE;
  uint32_t* keys = a.keys + (int64_t)e * a.n;
  int32_t* vals = a.out + (int64_t)e * a.n;
  for (int it = 0; it < TILE / TILE_THREADS; ++it) {
    const int64_t i = base + (int64_t)it * TILE_THREADS + threadIdx.x;
    if (i >= a.n) break;
    uint32_t x0 = (uint32_t)((uint64_t)i >> 32), x1 = (uint32_t)((uint64_t)i & 0xffffffffu);
    threefry2x32(s0, s1, x0, x1);
    const uint32_t k = x0 ^ x1;
    keys[i] = k;
    if (a.round == 0) vals[i] = (int32_t)i;
    atomicAdd(&cnt[bucket_of(k, a.bbits)], 1u);
  }
  __syncthreads();
  uint32_t* hist = a.hist + (int64_t)e * a.nb * a.tiles;
  for (int d = threadIdx.x; d < a.nb; d += TILE_THREADS) hist[(int64_t)d * a.tiles + blockIdx.x] = cnt[d];
}

// One workgroup per epoch: bucket totals, their exclusive scan (bucket
// starts), and each (bucket, tile) count rewritten as its write offset.  The
// scan over the nb <= 4096 totals is a block scan: thread t owns buckets
// 4t .. 4t + 3, wave-level inclusive scans of the per-thread sums, then the
// 16 wave totals.
constexpr int SCAN_THREADS = 1024;

__global__ void __launch_bounds__(SCAN_THREADS) shuffle_scan_kernel(ShuffleArgs a) {
  extern __shared__ uint32_t tot[];  // [nb]
  __shared__ uint32_t wsum[SCAN_THREADS / 64];
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t* hist = a.hist + (int64_t)e * a.nb * a.tiles;
  for (int d = threadIdx.x; d < a.nb; d += SCAN_THREADS) {
    uint32_t s = 0;
    for (int t = 0; t < a.tiles; ++t) s += hist[(int64_t)d * a.tiles + t];
    tot[d] = s;
  }
  __syncthreads();
  // exclusive scan of tot[0 .. nb)
  const int d0 = 4 * threadIdx.x;
  uint32_t v[4], local = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = d0 + i < a.nb ? tot[d0 + i] : 0u;
    local += v[i];
  }
  uint32_t inc = local;  // inclusive scan of the per-thread sums across the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(inc, o, 64);
    if (lane >= o) inc += y;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  uint32_t before = 0;
  for (int w = 0; w < wave; ++w) before += wsum[w];
  uint32_t run = before + inc - local;  // exclusive prefix of this thread's first bucket
  __syncthreads();  // every tot[] read above happens before the writes below
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (d0 + i < a.nb) tot[d0 + i] = run;
    run += v[i];
  }
  __syncthreads();
  uint32_t* bstart = a.bstart + (int64_t)e * (a.nb + 1);
  for (int d = threadIdx.x; d < a.nb; d += SCAN_THREADS) {
    bstart[d] = tot[d];
    uint32_t r = tot[d];
    for (int t = 0; t < a.tiles; ++t) {
      const uint32_t c = hist[(int64_t)d * a.tiles + t];
      hist[(int64_t)d * a.tiles + t] = r;
      r += c;
    }
  }
  if (threadIdx.x == 0) bstart[a.nb] = (uint32_t)a.n;
}

__global__ void __launch_bounds__(TILE_THREADS) shuffle_scatter_kernel(ShuffleArgs a) {
  extern __shared__ uint32_t slot[];  // [nb]
  const int e = blockIdx.y;
  const uint32_t* hist = a.hist + (int64_t)e * a.nb * a.tiles;
  for (int d = threadIdx.x; d < a.nb; d += TILE_THREADS) slot[d] = hist[(int64_t)d * a.tiles + blockIdx.x];
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * TILE;
  const uint32_t* keys = a.keys + (int64_t)e * a.n;
  const int32_t* vals = a.out + (int64_t)e * a.n;
  const int64_t eo = (int64_t)e * a.n;
  for (int it = 0; it < TILE / TILE_THREADS; ++it) {
    const int64_t i = base + (int64_t)it * TILE_THREADS + threadIdx.x;
    if (i >= a.n) break;
    const uint32_t k = keys[i];
    const uint32_t pos = atomicAdd(&slot[bucket_of(k, a.bbits)], 1u);
    a.tkey[eo + pos] = k;
    a.tpos[eo + pos] = (uint32_t)i;
    a.tval[eo + pos] = vals[i];
  }
}

__global__ void __launch_bounds__(SORT_THREADS) shuffle_sort_kernel(ShuffleArgs a) {
  __shared__ uint64_t sk[BUCKET_CAP];
  __shared__ int32_t sv[BUCKET_CAP];
  const int e = blockIdx.y;
  const int b = blockIdx.x;
  const uint32_t* bstart = a.bstart + (int64_t)e * (a.nb + 1);
  const int64_t s = bstart[b], t = bstart[b + 1];
  const int m = (int)(t - s);
  const int64_t eo = (int64_t)e * a.n;
  int32_t* out = a.out + eo;
  if (m <= 0) return;
  if (m <= BUCKET_CAP) {
    int p2 = 1;
    while (p2 < m) p2 <<= 1;
    for (int i = threadIdx.x; i < p2; i += SORT_THREADS) {
      if (i < m) {
        sk[i] = ((uint64_t)a.tkey[eo + s + i] << 32) | (uint64_t)a.tpos[eo + s + i];
        sv[i] = a.tval[eo + s + i];
      } else {
        sk[i] = ~0ull;
        sv[i] = 0;
      }
    }
    __syncthreads();
    // bitonic sort of p2 unique-or-sentinel keys, ascending
    for (int k = 2; k <= p2; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = threadIdx.x; i < p2; i += SORT_THREADS) {
          const int l = i ^ j;
          if (l > i) {
            const bool up = (i & k) == 0;
            const uint64_t x = sk[i], y = sk[l];
            if ((x > y) == up) {
              sk[i] = y;
              sk[l] = x;
              const int32_t tv = sv[i];
              sv[i] = sv[l];
              sv[l] = tv;
            }
          }
        }
        __syncthreads();
      }
    }
    for (int i = threadIdx.x; i < m; i += SORT_THREADS) out[s + i] = sv[i];
  } else {
    // rank by counting: exact for any size, quadratic
    for (int i = threadIdx.x; i < m; i += SORT_THREADS) {
      const uint64_t ki = ((uint64_t)a.tkey[eo + s + i] << 32) | (uint64_t)a.tpos[eo + s + i];
      int rank = 0;
      for (int j = 0; j < m; ++j) {
        const uint64_t kj = ((uint64_t)a.tkey[eo + s + j] << 32) | (uint64_t)a.tpos[eo + s + j];
        rank += kj < ki ? 1 : 0;
      }
      out[s + rank] = a.tval[eo + s + i];
    }
  }
}

int shuffle_rounds(int64_t n) {
  const double m = n > 1 ? (double)n : 1.0;
  return (int)ceil(3.0 * log(m) / log(4294967295.0));
}

int bucket_bits(int64_t n) {
  if (n <= BUCKET_CAP) return 0;
  int b = 0;
  while (b < MAX_BUCKET_BITS && (n >> b) > 512) ++b;
  return b;
}

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

struct Space {
  uint32_t *keys, *hist, *bstart, *tkey, *tpos;
  int32_t* tval;
};

size_t space_bytes(int epochs, int64_t n) {
  const int64_t E = epochs > 0 ? epochs : 1;
  const int64_t nn = n > 0 ? n : 1;
  const int64_t tiles = ppo::ceil_div64(nn, TILE);
  const int64_t nb = int64_t(1) << bucket_bits(nn);
  return 4 * align256(sizeof(uint32_t) * E * nn) + align256(sizeof(uint32_t) * E * nb * tiles) +
         align256(sizeof(uint32_t) * E * (nb + 1));
}

Space carve(void* ws, int epochs, int64_t n) {
  const int64_t E = epochs > 0 ? epochs : 1;
  const int64_t tiles = ppo::ceil_div64(n, TILE);
  const int64_t nb = int64_t(1) << bucket_bits(n);
  char* p = (char*)ws;
  Space s;
  s.keys = (uint32_t*)p; p += align256(sizeof(uint32_t) * E * n);
  s.tkey = (uint32_t*)p; p += align256(sizeof(uint32_t) * E * n);
  s.tpos = (uint32_t*)p; p += align256(sizeof(uint32_t) * E * n);
  s.tval = (int32_t*)p; p += align256(sizeof(uint32_t) * E * n);
  s.hist = (uint32_t*)p; p += align256(sizeof(uint32_t) * E * nb * tiles);
  s.bstart = (uint32_t*)p;
  return s;
}

// out[e * n + i] = i for every epoch row
__global__ void iota_kernel(int32_t* out, int64_t n, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < total) out[i] = (int32_t)(i % n);
}

// permutation(split(key, epochs)[e], n) for every e (split_epochs = 1), or of
// key itself (split_epochs = 0, epochs = 1), into out[e * n + i].
int shuffle_impl(hipStream_t st, const uint32_t* key, int split_epochs, int epochs, int64_t n, int32_t* out,
                 void* ws) {
  if (n <= 0 || epochs <= 0) return PPO_OK;
  const int rounds = shuffle_rounds(n);
  if (rounds == 0) {
    // n == 1: the identity
    hipLaunchKernelGGL(iota_kernel, dim3((unsigned)ppo::ceil_div64(n * epochs, 256)), dim3(256), 0, st, out, n,
                       n * epochs);
    return ppo::check_launch("ppo_permutation");
  }
  Space sp = carve(ws, epochs, n);
  ShuffleArgs a;
  a.key = key; a.split_epochs = split_epochs; a.n = n;
  a.tiles = (int)ppo::ceil_div64(n, TILE);
  a.bbits = bucket_bits(n);
  a.nb = 1 << a.bbits;
  a.out = out; a.keys = sp.keys; a.hist = sp.hist; a.bstart = sp.bstart;
  a.tkey = sp.tkey; a.tpos = sp.tpos; a.tval = sp.tval;
  const size_t shm = sizeof(uint32_t) * a.nb;
  for (int r = 0; r < rounds; ++r) {
    a.round = r;
    hipLaunchKernelGGL(shuffle_bits_kernel, dim3(a.tiles, epochs), dim3(TILE_THREADS), shm, st, a);
    hipLaunchKernelGGL(shuffle_scan_kernel, dim3(epochs), dim3(SCAN_THREADS), shm, st, a);
    hipLaunchKernelGGL(shuffle_scatter_kernel, dim3(a.tiles, epochs), dim3(TILE_THREADS), shm, st, a);
    hipLaunchKernelGGL(shuffle_sort_kernel, dim3(a.nb, epochs), dim3(SORT_THREADS), 0, st, a);
  }
  return ppo::check_launch("ppo_permutation");
}

}  // namespace

// Scratch of ppo_epoch_permutations_noalloc: the bucket sort's keys,
// positions, values, histograms and bucket starts (every byte is rewritten by
// each call before it is read, so nothing is cleared).  Each GPU the library
// runs on holds its own copy until the process ends.  Host code never passes
// the symbol itself to a kernel: the device address is resolved per device
// with hipGetSymbolAddress and kept in `g_scratch`.
static constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(24) << 20;  // 4 epochs x 262144 items need 16.5 MB
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

static constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch[MAX_DEVICES] = {};

// Device address of `scratch` on the current device (resolved on the first
// call per device, with that device current).
static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return ppo::set_error(PPO_ERR_LAUNCH, "ppo_epoch_permutations_noalloc: no current device (%s)",
                          hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return ppo::set_error(PPO_ERR_LAUNCH, "ppo_epoch_permutations_noalloc: scratch address on device %d: %s", dev,
                            hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return PPO_OK;
}

PPO_EXPORT size_t ppo_permutation_workspace(int64_t n) { return space_bytes(1, n); }

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
  if (workspace_bytes < space_bytes(1, n) || (n > 0 && !workspace))
    return ppo::set_error(PPO_ERR_SPACE, "ppo_permutation: workspace %zu < %zu bytes", workspace_bytes,
                          space_bytes(1, n));
  return shuffle_impl(ppo::as_stream(stream), key, 0, 1, n, out, workspace);
}

PPO_EXPORT size_t ppo_epoch_permutations_workspace(int epochs, int64_t n) { return space_bytes(epochs, n); }

// out[e * n + i] = permutation(split(key, epochs)[e], n)[i], all epochs in the same launches.
PPO_EXPORT int ppo_epoch_permutations(void* stream, const uint32_t* key, int epochs, int64_t n, int32_t* out,
                                      void* workspace, size_t workspace_bytes) {
  if (epochs < 0 || epochs > 65535 || n < 0 || n > INT32_MAX || !key || (epochs > 0 && n > 0 && !out))
    return ppo::set_error(PPO_ERR_ARG, "ppo_epoch_permutations: bad argument");
  if (workspace_bytes < space_bytes(epochs, n) || !workspace)
    return ppo::set_error(PPO_ERR_SPACE, "ppo_epoch_permutations: workspace too small");
  return shuffle_impl(ppo::as_stream(stream), key, 1, epochs, n, out, workspace);
}

// ppo_epoch_permutations with its workspace in the library's own device
// scratch: no allocation, for callers that cannot allocate.  Rejects sizes
// whose workspace exceeds the scratch.  Calls that overlap on one GPU share
// the scratch and race.
PPO_EXPORT int ppo_epoch_permutations_noalloc(void* stream, const uint32_t* key, int epochs, int64_t n,
                                              int32_t* out) {
  if (epochs < 0 || epochs > 65535 || n < 0 || n > INT32_MAX || !key || (epochs > 0 && n > 0 && !out))
    return ppo::set_error(PPO_ERR_ARG, "ppo_epoch_permutations_noalloc: bad argument");
  if (space_bytes(epochs, n) > NOALLOC_SCRATCH_BYTES)
    return ppo::set_error(PPO_ERR_SPACE, "ppo_epoch_permutations_noalloc: %d epochs of %lld items need %zu bytes "
                          "of scratch, more than its %zu", epochs, (long long)n, space_bytes(epochs, n),
                          NOALLOC_SCRATCH_BYTES);
  hipStream_t st = ppo::as_stream(stream);
  int cur = -1, sdev = -1;
  if (hipGetDevice(&cur) != hipSuccess || hipStreamGetDevice(st, &sdev) != hipSuccess || cur != sdev)
    return ppo::set_error(PPO_ERR_ARG, "ppo_epoch_permutations_noalloc: the stream's device (%d) is not the "
                          "current device (%d)", sdev, cur);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != PPO_OK) return rc;
  return shuffle_impl(st, key, 1, epochs, n, out, ws);
}
