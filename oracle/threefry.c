/*
 * CPU oracle (test infrastructure only, never shipped or measured): a plain-C
 * restatement of the integer work behind boonta's minibatch order.
 *
 *   PPO.update        boonta/algorithms/ppo.py:199-201, :230-231
 *   RecurrentPPO      boonta/algorithms/recurrent_ppo.py:269-279
 *
 * Both call jax.random.split(key, E) and jax.random.permutation(key, n) of
 * jax 0.10.2 (uv.lock:6802-6803), a third-party dependency that is not under
 * the reference tree.  Its published algorithm, restated here:
 *
 *   - key(seed) holds the words (seed >> 32, seed & 0xffffffff).
 *   - Threefry-2x32 with 20 rounds (Salmon et al., SC'11, Random123):
 *     rotations {13,15,26,6} / {17,29,16,24}, key schedule with parity
 *     constant 0x1BD11BDA, injection every 4 rounds with counter s.
 *   - With jax_threefry_partitionable (default on since jax 0.5), split(key, n)
 *     returns threefry(key, (hi(i), lo(i))) for i = 0..n-1 (a 64-bit iota split
 *     into two 32-bit words), and 32-bit random bits at flat index i are
 *     out0 ^ out1 of the same call.
 *   - permutation(key, n) shuffles arange(n) with ceil(3 ln n / ln(2^32 - 1))
 *     rounds; each round does `key, subkey = split(key)` and a stable ascending
 *     sort of the values keyed by random_bits(subkey, 32, (n,)).
 *
 * Pinned by the Random123 known-answer vectors (tests), by the is-a-permutation
 * invariant, and by brute-force stable-sort checks.  The composition above
 * (split layout, xor of the two output words, round count, stability) is
 * restated from jax's source as published; no jax is importable in this image,
 * so bit-parity with a live jax run is "parity unpinned" beyond those checks.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

static inline uint32_t rotl32(uint32_t v, uint32_t r) {
  return (v << r) | (v >> (32u - r));
}

void oracle_threefry2x32(uint32_t k0, uint32_t k1, uint32_t x0, uint32_t x1,
                         uint32_t out[2]) {
  static const uint32_t rot[2][4] = {{13, 15, 26, 6}, {17, 29, 16, 24}};
  uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  uint32_t x[2] = {x0 + ks[0], x1 + ks[1]};
  for (uint32_t s = 1; s <= 5; ++s) {
    const uint32_t* r = rot[(s - 1) & 1];
    for (int i = 0; i < 4; ++i) {
      x[0] += x[1];
      x[1] = rotl32(x[1], r[i]);
      x[1] ^= x[0];
    }
    x[0] += ks[s % 3];
    x[1] += ks[(s + 1) % 3] + s;
  }
  out[0] = x[0];
  out[1] = x[1];
}

void oracle_key(uint64_t seed, uint32_t key[2]) {
  key[0] = (uint32_t)(seed >> 32);
  key[1] = (uint32_t)(seed & 0xffffffffu);
}

/* split(key, num): new key i = threefry(key, (i >> 32, i & 0xffffffff)). */
void oracle_split(const uint32_t key[2], int64_t num, uint32_t* out) {
  for (int64_t i = 0; i < num; ++i) {
    oracle_threefry2x32(key[0], key[1], (uint32_t)((uint64_t)i >> 32),
                        (uint32_t)((uint64_t)i & 0xffffffffu), out + 2 * i);
  }
}

void oracle_random_bits32(const uint32_t key[2], int64_t n, uint32_t* out) {
  uint32_t o[2];
  for (int64_t i = 0; i < n; ++i) {
    oracle_threefry2x32(key[0], key[1], (uint32_t)((uint64_t)i >> 32),
                        (uint32_t)((uint64_t)i & 0xffffffffu), o);
    out[i] = o[0] ^ o[1];
  }
}

int oracle_shuffle_rounds(int64_t n) {
  double m = n > 1 ? (double)n : 1.0;
  return (int)ceil(3.0 * log(m) / log(4294967295.0));
}

typedef struct {
  uint32_t key;
  uint32_t pos;
  int32_t val;
} sort_item;

static int cmp_item(const void* a, const void* b) {
  const sort_item* x = (const sort_item*)a;
  const sort_item* y = (const sort_item*)b;
  if (x->key != y->key) return x->key < y->key ? -1 : 1;
  /* ties keep their input order: a stable sort */
  return x->pos < y->pos ? -1 : (x->pos > y->pos ? 1 : 0);
}

/* Stable sort of vals by keys (ascending, unsigned). */
void oracle_stable_sort_by_key(const uint32_t* keys, int32_t* vals, int64_t n) {
  sort_item* items = (sort_item*)malloc(sizeof(sort_item) * (size_t)(n ? n : 1));
  for (int64_t i = 0; i < n; ++i) {
    items[i].key = keys[i];
    items[i].pos = (uint32_t)i;
    items[i].val = vals[i];
  }
  qsort(items, (size_t)n, sizeof(sort_item), cmp_item);
  for (int64_t i = 0; i < n; ++i) vals[i] = items[i].val;
  free(items);
}

void oracle_permutation(const uint32_t key_in[2], int64_t n, int32_t* out) {
  uint32_t key[2] = {key_in[0], key_in[1]};
  uint32_t pair[4];
  uint32_t* bits = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(n ? n : 1));
  for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)i;
  int rounds = oracle_shuffle_rounds(n);
  for (int r = 0; r < rounds; ++r) {
    oracle_split(key, 2, pair);
    key[0] = pair[0];
    key[1] = pair[1];
    oracle_random_bits32(pair + 2, n, bits);
    oracle_stable_sort_by_key(bits, out, n);
  }
  free(bits);
}

/* The E epoch permutations of one update: split(key, E), then one
 * permutation of n per epoch key, written row by row into out[E * n]. */
void oracle_epoch_permutations(const uint32_t key[2], int epochs, int64_t n,
                               int32_t* out) {
  uint32_t* keys = (uint32_t*)malloc(sizeof(uint32_t) * 2 * (size_t)epochs);
  oracle_split(key, epochs, keys);
  for (int e = 0; e < epochs; ++e) oracle_permutation(keys + 2 * e, n, out + (int64_t)e * n);
  free(keys);
}
