// l2sim.c — set-associative LRU cache over a stream of 128-byte line addresses (CPU,
// used by measure/line_model.py; not part of the operator).
#include <stdint.h>
#include <stdlib.h>

static inline uint64_t mix64(uint64_t x) {  // splitmix64 finaliser: set index of a line
  x ^= x >> 30; x *= 0xbf58476d1ce4e5b9ULL; x ^= x >> 27; x *= 0x94d049bb133111ebULL; x ^= x >> 31;
  return x;
}

// Misses of `lines[0..n)` through a cache of `sets` x `ways` lines with LRU replacement;
// hashed != 0 spreads lines over sets by a hash, as the L2's channel and set
// interleaving does.  Returns -1 if memory runs out.
int64_t lru_misses(const uint64_t* lines, int64_t n, int sets, int ways, int hashed) {
  uint64_t* tag = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)sets * ways);
  uint64_t* age = (uint64_t*)calloc((size_t)sets * ways, sizeof(uint64_t));
  if (!tag || !age) { free(tag); free(age); return -1; }
  for (int64_t i = 0; i < (int64_t)sets * ways; ++i) tag[i] = ~0ULL;
  int64_t misses = 0;
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t l = lines[i];
    const uint64_t s = (hashed ? mix64(l) : l) % (uint64_t)sets;
    uint64_t* tg = tag + s * ways;
    uint64_t* ag = age + s * ways;
    int hit = -1, lru = 0;
    for (int w = 0; w < ways; ++w) {
      if (tg[w] == l) { hit = w; break; }
      if (ag[w] < ag[lru]) lru = w;
    }
    if (hit >= 0) { ag[hit] = (uint64_t)i + 1; continue; }
    ++misses;
    tg[lru] = l;
    ag[lru] = (uint64_t)i + 1;
  }
  free(tag);
  free(age);
  return misses;
}
