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
//   4. sort: one workgroup per bucket splits its unique (key, position) pairs
//      in LDS by the next 8 key bits, ranks each pair within its sub-bucket by
//      counting the smaller ones, and writes each value at its rank.
// A bucket larger than the LDS capacity (not reachable for Threefry keys at
// these sizes, but handled) is ranked from global memory instead.
#include "common.h"
#include "threefry.h"

#include <algorithm>
#include <math.h>
#include <mutex>
#include <utility>

namespace {

using ppo::threefry2x32;

constexpr int TILE = 4096;          // elements per histogram / scatter block
constexpr int TILE_THREADS = 1024;
constexpr int SORT_CAP = 2048;      // elements a bucket sorts in LDS
constexpr int SORT_THREADS = 512;
constexpr int MAX_BUCKET_BITS = 12;
// Buckets larger than SORT_CAP go to a second sort launch with room for
// SORT_CAP2 elements (run only when the expected bucket passes 512 elements,
// i.e. from 2^21 items per epoch, where the bucket count stops growing);
// larger ones still are ranked from global memory, exactly but slowly.
constexpr int SORT_CAP2 = 8192;
constexpr int SORT_THREADS2 = 1024;

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
  int big_pass;         // buckets over SORT_CAP go to a second sort launch
  int32_t* out;         // [E][n]: values in, values out
  uint32_t* keys;       // [E][n]
  uint32_t* hist;       // [E][tiles][nb]
  uint32_t* bstart;     // [E][nb + 1]
  uint4* trec;          // [E][n] bucketed records: key, position, value (one 16-byte store each)
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
  for (int d = threadIdx.x; d < a.nb; d += TILE_THREADS) hist[(int64_t)blockIdx.x * a.nb + d] = cnt[d];
}

// One workgroup per epoch: bucket totals, their exclusive scan (bucket
// starts), and each (tile, bucket) count rewritten as its write offset.  The
// counts are stored tile-major ([tiles][nb]), so the threads of a wave, one
// bucket each, read consecutive words at every tile, eight tiles' loads in
// flight at a time.  The scan over the nb <= 4096 totals is a block scan:
// thread t owns buckets 4t .. 4t + 3, wave-level inclusive scans of the
// per-thread sums, then the 16 wave totals.
constexpr int SCAN_THREADS = 1024;
constexpr int SCAN_BATCH = 8;

__global__ void __launch_bounds__(SCAN_THREADS) shuffle_scan_kernel(ShuffleArgs a) {
  extern __shared__ uint32_t tot[];  // [nb]
  __shared__ uint32_t wsum[SCAN_THREADS / 64];
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t* hist = a.hist + (int64_t)e * a.nb * a.tiles;
  const int64_t nb = a.nb;
  for (int d = threadIdx.x; d < a.nb; d += SCAN_THREADS) {
    uint32_t s = 0;
    int t = 0;
    for (; t + SCAN_BATCH <= a.tiles; t += SCAN_BATCH) {
      uint32_t c[SCAN_BATCH];
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i) c[i] = hist[(t + i) * nb + d];
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i) s += c[i];
    }
    for (; t < a.tiles; ++t) s += hist[t * nb + d];
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
    int t = 0;
    for (; t + SCAN_BATCH <= a.tiles; t += SCAN_BATCH) {
      uint32_t c[SCAN_BATCH];
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i) c[i] = hist[(t + i) * nb + d];
#pragma unroll
      for (int i = 0; i < SCAN_BATCH; ++i) {
        hist[(t + i) * nb + d] = r;
        r += c[i];
      }
    }
    for (; t < a.tiles; ++t) {
      const uint32_t c = hist[t * nb + d];
      hist[t * nb + d] = r;
      r += c;
    }
  }
  if (threadIdx.x == 0) bstart[a.nb] = (uint32_t)a.n;
}

__global__ void __launch_bounds__(TILE_THREADS) shuffle_scatter_kernel(ShuffleArgs a) {
  extern __shared__ uint32_t slot[];  // [nb]
  const int e = blockIdx.y;
  const uint32_t* hist = a.hist + (int64_t)e * a.nb * a.tiles;
  for (int d = threadIdx.x; d < a.nb; d += TILE_THREADS) slot[d] = hist[(int64_t)blockIdx.x * a.nb + d];
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * TILE;
  const uint32_t* keys = a.keys + (int64_t)e * a.n;
  const int32_t* vals = a.out + (int64_t)e * a.n;
  const int64_t eo = (int64_t)e * a.n;
  // every load of the thread's elements first, then the slots and stores
  constexpr int PER = TILE / TILE_THREADS;
  uint32_t k[PER];
  int32_t v[PER];
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int64_t i = base + (int64_t)it * TILE_THREADS + threadIdx.x;
    k[it] = i < a.n ? keys[i] : 0u;
    v[it] = i < a.n ? vals[i] : 0;
  }
#pragma unroll
  for (int it = 0; it < PER; ++it) {
    const int64_t i = base + (int64_t)it * TILE_THREADS + threadIdx.x;
    if (i >= a.n) break;
    const uint32_t pos = atomicAdd(&slot[bucket_of(k[it], a.bbits)], 1u);
    a.trec[eo + pos] = make_uint4(k[it], (uint32_t)i, (uint32_t)v[it], 0u);
  }
}

// One workgroup per bucket.  Its (key, position) pairs are split in LDS by
// the 8 key bits below the bucket's (an LDS histogram, its scan, and a
// scatter into per-sub-bucket ranges whose order inside a range is
// arbitrary); the pairs are unique, so each one's slot is its sub-bucket's
// start plus the number of smaller pairs in that sub-bucket (about
// m / 256 compares, not m).  The first launch (CAP = SORT_CAP) takes the
// buckets that fit it; the second (CAP = SORT_CAP2, only when a.big_pass)
// the ones from SORT_CAP + 1 to SORT_CAP2 elements; whichever launch is last
// ranks larger buckets from global memory.
constexpr int SUB_BITS = 8;
constexpr int SUB = 1 << SUB_BITS;

template <int CAP, int THREADS, int MIN_M>
__global__ void __launch_bounds__(THREADS) shuffle_sort_kernel(ShuffleArgs a) {
  constexpr int PER = CAP / THREADS;
  __shared__ uint64_t sk[CAP];
  __shared__ int32_t sv[CAP];
  __shared__ uint32_t cnt[SUB];
  __shared__ uint32_t start[SUB + 1];
  const int tid = threadIdx.x;
  const int e = blockIdx.y;
  const int b = blockIdx.x;
  const uint32_t* bstart = a.bstart + (int64_t)e * (a.nb + 1);
  const int64_t s = bstart[b], t = bstart[b + 1];
  const int m = (int)(t - s);
  const int64_t eo = (int64_t)e * a.n;
  int32_t* out = a.out + eo;
  if (m <= MIN_M) return;  // empty, or sorted by the first launch
  if (m <= CAP) {
    const int shift = 32 - a.bbits - SUB_BITS;
    for (int d = tid; d < SUB; d += THREADS) cnt[d] = 0;
    __syncthreads();
    uint64_t kk[PER];
    int32_t vv[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = tid + q * THREADS;
      const int ic = i < m ? i : m - 1;
      const uint4 rec = a.trec[eo + s + ic];
      kk[q] = ((uint64_t)rec.x << 32) | (uint64_t)rec.y;
      vv[q] = (int32_t)rec.z;
    }
#pragma unroll
    for (int q = 0; q < PER; ++q)
      if (tid + q * THREADS < m) atomicAdd(&cnt[(uint32_t)(kk[q] >> (32 + shift)) & (SUB - 1)], 1u);
    __syncthreads();
    // exclusive scan of the SUB counts by the first wave (SUB / 64 per lane)
    if (tid < 64) {
      constexpr int PL = SUB / 64;
      uint32_t c[PL], local = 0;
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        c[i] = cnt[PL * tid + i];
        local += c[i];
      }
      uint32_t inc = local;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(inc, o, 64);
        if (tid >= o) inc += y;
      }
      uint32_t run = inc - local;
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        start[PL * tid + i] = run;
        run += c[i];
      }
      if (tid == 63) start[SUB] = inc;
    }
    __syncthreads();
    for (int d = tid; d < SUB; d += THREADS) cnt[d] = start[d];  // cursors
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      if (tid + q * THREADS < m) {
        const uint32_t p = atomicAdd(&cnt[(uint32_t)(kk[q] >> (32 + shift)) & (SUB - 1)], 1u);
        sk[p] = kk[q];
        sv[p] = vv[q];
      }
    }
    __syncthreads();
    for (int i = tid; i < m; i += THREADS) {
      const uint64_t ki = sk[i];
      const uint32_t d = (uint32_t)(ki >> (32 + shift)) & (SUB - 1);
      const int j1 = (int)start[d + 1];
      int rank = (int)start[d];
      for (int j = (int)start[d]; j < j1; ++j) rank += sk[j] < ki;
      out[s + rank] = sv[i];
    }
  } else if (MIN_M > 0 || !a.big_pass) {
    // rank by counting from global memory: exact for any size
    for (int i = tid; i < m; i += THREADS) {
      const uint4 ri = a.trec[eo + s + i];
      const uint64_t ki = ((uint64_t)ri.x << 32) | (uint64_t)ri.y;
      int rank = 0;
      for (int j = 0; j < m; ++j) {
        const uint4 rj = a.trec[eo + s + j];
        const uint64_t kj = ((uint64_t)rj.x << 32) | (uint64_t)rj.y;
        rank += kj < ki ? 1 : 0;
      }
      out[s + rank] = (int32_t)ri.z;
    }
  }
}

int shuffle_rounds(int64_t n) {
  const double m = n > 1 ? (double)n : 1.0;
  return (int)ceil(3.0 * log(m) / log(4294967295.0));
}

int bucket_bits(int64_t n) {
  if (n <= SORT_CAP) return 0;
  int b = 0;
  while (b < MAX_BUCKET_BITS && (n >> b) > 512) ++b;
  return b;
}

// Whether the second sort launch runs: the expected bucket holds more than
// 512 elements (the bucket count has stopped growing).
bool big_pass(int64_t n) { return (n >> bucket_bits(n)) > 512; }

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

struct Space {
  uint32_t *keys, *hist, *bstart;
  uint4* trec;
};

size_t space_bytes(int epochs, int64_t n) {
  const int64_t E = epochs > 0 ? epochs : 1;
  const int64_t nn = n > 0 ? n : 1;
  const int64_t tiles = ppo::ceil_div64(nn, TILE);
  const int64_t nb = int64_t(1) << bucket_bits(nn);
  return align256(sizeof(uint32_t) * E * nn) + align256(sizeof(uint4) * E * nn) +
         align256(sizeof(uint32_t) * E * nb * tiles) + align256(sizeof(uint32_t) * E * (nb + 1));
}

Space carve(void* ws, int epochs, int64_t n) {
  const int64_t E = epochs > 0 ? epochs : 1;
  const int64_t tiles = ppo::ceil_div64(n, TILE);
  const int64_t nb = int64_t(1) << bucket_bits(n);
  char* p = (char*)ws;
  Space s;
  s.keys = (uint32_t*)p; p += align256(sizeof(uint32_t) * E * n);
  s.trec = (uint4*)p; p += align256(sizeof(uint4) * E * n);
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
  a.big_pass = big_pass(n) ? 1 : 0;
  a.out = out; a.keys = sp.keys; a.hist = sp.hist; a.bstart = sp.bstart;
  a.trec = sp.trec;
  const size_t shm = sizeof(uint32_t) * a.nb;
  for (int r = 0; r < rounds; ++r) {
    a.round = r;
    hipLaunchKernelGGL(shuffle_bits_kernel, dim3(a.tiles, epochs), dim3(TILE_THREADS), shm, st, a);
    hipLaunchKernelGGL(shuffle_scan_kernel, dim3(epochs), dim3(SCAN_THREADS), shm, st, a);
    hipLaunchKernelGGL(shuffle_scatter_kernel, dim3(a.tiles, epochs), dim3(TILE_THREADS), shm, st, a);
    hipLaunchKernelGGL((shuffle_sort_kernel<SORT_CAP, SORT_THREADS, 0>), dim3(a.nb, epochs), dim3(SORT_THREADS), 0,
                       st, a);
    if (a.big_pass)
      hipLaunchKernelGGL((shuffle_sort_kernel<SORT_CAP2, SORT_THREADS2, SORT_CAP>), dim3(a.nb, epochs),
                         dim3(SORT_THREADS2), 0, st, a);
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
static constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(24) << 20;  // 4 epochs x 262144 items need 20.5 MiB
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

// The bucket sort's plan for n items (host only): bucket count bits, and the
// largest bucket sorted in LDS (larger ones are ranked from global memory).
PPO_EXPORT int ppo_permutation_bucket_bits(int64_t n) { return n > 0 ? bucket_bits(n) : 0; }
PPO_EXPORT int ppo_permutation_bucket_cap(int64_t n) { return n > 0 && big_pass(n) ? SORT_CAP2 : SORT_CAP; }

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
