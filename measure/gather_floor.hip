// gather_floor.hip — measurement kernel of bench.py (libtbe_floor.so, built by
// measure/build.py; not part of the operator or of its C ABI).
//
// It moves the memory traffic of one TBE forward with no pooling: every lookup's
// row (the header word and the payload words the operator reads, so the same
// 128-byte lines) is gathered, and the output is written, with a gather structure
// chosen only for throughput.  Persistent waves walk the lookups in chunks of 64
// (each XCD one contiguous eighth of the chunks, its waves interleaved over it, as
// the operator's items); a row is read by 2^LG lanes of 4 B (as the operator reads
// it), 64 / 2^LG rows per load instruction and 16 instructions per chunk, the header
// in a second load of the same rows, and the rows of the next chunk are in flight
// while the current one is folded into one word per lane.  Rows
// are addressed by 64-bit addresses precomputed outside the timed region (8 B read
// per lookup instead of the operator's 4-byte index).  Each lookup writes
// `out_words` 4-byte words (chunk-contiguous, coalesced), so a pooled output's bytes
// per lookup or a nobag row can be matched.  Its time is a floor for the operator's
// memory work on that workload: what the memory system takes for the same lines
// from a gather that does nothing else.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

namespace {

constexpr int kWave = 64;

__device__ __forceinline__ uint32_t load_word(const uint8_t* p) {
  using GlobalWord = const __attribute__((address_space(1))) uint32_t;
  return *(GlobalWord*)(p);
}

template <int LG, int kChunkInstr>
__global__ __launch_bounds__(256) void gather_floor_kernel(const uint64_t* __restrict__ addr, int64_t n,
                                                           uint64_t fallback, int payload_words,
                                                           uint32_t* __restrict__ out, int out_words) {
  constexpr int R = kWave >> LG;        // rows per load instruction
  constexpr int CH = kChunkInstr * R;   // lookups per chunk
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x >> 6;
  const uint32_t part = blockIdx.x % 8, lblk = blockIdx.x / 8, nblk = gridDim.x / 8;
  const int64_t nch = (n + CH - 1) / CH;
  const int64_t e = nch * (part + 1) / 8;
  const int64_t step = static_cast<int64_t>(nblk) * 4;
  int64_t c = nch * part / 8 + static_cast<int64_t>(lblk) * 4 + wv;
  if (c >= e) return;
  const int slot = lane >> LG;
  // payload word of this lane (lanes past a row's words re-read its last word)
  const uint32_t col = 4u + 4u * static_cast<uint32_t>(min(lane & ((1 << LG) - 1), payload_words - 1));
  // lanes past the lookups read row `fallback` (a valid row), and fold nothing
  auto lookup_addr = [&](int64_t ch) {
    const int64_t i = ch * CH + lane;
    return ch < e && lane < CH && i < n ? addr[i] : fallback;
  };
  auto issue = [&](uint64_t a, uint32_t (&d)[kChunkInstr], uint32_t (&h)[kChunkInstr]) {
#pragma unroll
    for (int u = 0; u < kChunkInstr; ++u) {
      const int src = (u * R + slot) * 4;
      const uint32_t lo = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(static_cast<uint32_t>(a)));
      const uint32_t hi = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(static_cast<uint32_t>(a >> 32)));
      const uint8_t* p = reinterpret_cast<const uint8_t*>((static_cast<uint64_t>(hi) << 32) | lo);
      d[u] = load_word(p + col);
      h[u] = load_word(p);
    }
  };
  uint32_t d0[kChunkInstr], h0[kChunkInstr];
  issue(lookup_addr(c), d0, h0);
  int64_t cn = c + step;
  uint64_t an = lookup_addr(cn);
  uint32_t acc = 0;
  while (true) {
    uint32_t d1[kChunkInstr], h1[kChunkInstr];
    const bool more = cn < e;
    if (more) issue(an, d1, h1);
    const int64_t c2 = cn + step;
    const uint64_t a2 = lookup_addr(c2);
#pragma unroll
    for (int u = 0; u < kChunkInstr; ++u) acc ^= d0[u] + h0[u];
    // the chunk's output: out_words words per lookup, written by the 64 lanes together
    const int64_t base = c * CH * out_words;
    const int64_t lim = min(n, (c + 1) * CH) * out_words;
    for (int k = 0; k * kWave < CH * out_words; ++k) {
      const int64_t o = base + static_cast<int64_t>(k) * kWave + lane;
      if (o < lim) out[o] = acc + k;
    }
    if (!more) break;
#pragma unroll
    for (int u = 0; u < kChunkInstr; ++u) {
      d0[u] = d1[u];
      h0[u] = h1[u];
    }
    c = cn;
    cn = c2;
    an = a2;
  }
}

}  // namespace

// addr[n]: the byte address of every lookup's row (header first); fallback: the
// address of any valid row; payload_words: 4-byte payload words of a row (1..16
// read per row); out: n * out_words 4-byte words.  Returns 0 or a HIP error code.
template <int LG, int CI>
int launch_floor(const uint64_t* a, int64_t n, uint64_t fallback, int32_t payload_words, uint32_t* o,
                 int32_t out_words, hipStream_t s, int rounds) {
  int dev = 0, cus = 0, per_cu = 0;
  const void* fn = reinterpret_cast<const void*>(gather_floor_kernel<LG, CI>);
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0) != hipSuccess)
    return -1;
  // `rounds` rounds of the resident blocks, a multiple of 8 (one part per XCD)
  const int blocks = 8 * ((rounds * cus * per_cu + 7) / 8);
  hipLaunchKernelGGL((gather_floor_kernel<LG, CI>), dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, s, a, n,
                     fallback, payload_words, o, out_words);
  return static_cast<int>(hipGetLastError());
}

extern "C" int tbe_gather_floor(const void* addr, int64_t n, uint64_t fallback, int32_t payload_words,
                                void* out, int32_t out_words, void* stream) {
  if (n <= 0) return 0;
  if (payload_words < 1 || payload_words > 64 || out_words < 1) return -1;
  int lg = 0;
  while ((1 << lg) < payload_words) ++lg;
  lg = lg < 2 ? 2 : lg;
  if (lg > 5) return -1;  // rows of more than 32 payload words: not measured here
  // measured on configuration 2 (rows of 16 words): 16 instructions per chunk and two
  // rounds of resident blocks are the fastest of 8/12/16 and 1/2/3/4 (TBE_FLOOR_SHAPE=
  // <instructions>x<rounds> selects another shape)
  static const int shape = [] {
    const char* e = getenv("TBE_FLOOR_SHAPE");
    int ci = 16, r = 2;
    if (e) sscanf(e, "%dx%d", &ci, &r);
    return ci * 16 + (r >= 1 && r <= 8 ? r : 2);
  }();
  const int ci = shape / 16, rounds = shape % 16;
  const uint64_t* a = static_cast<const uint64_t*>(addr);
  uint32_t* o = static_cast<uint32_t*>(out);
  const hipStream_t s = static_cast<hipStream_t>(stream);
#define TBE_FLOOR_LG(L)                                                                           \
  case L:                                                                                         \
    if (ci == 8) return launch_floor<L, 8>(a, n, fallback, payload_words, o, out_words, s, rounds);  \
    if (ci == 12) return launch_floor<L, 12>(a, n, fallback, payload_words, o, out_words, s, rounds); \
    return launch_floor<L, 16>(a, n, fallback, payload_words, o, out_words, s, rounds);
  switch (lg) {
    TBE_FLOOR_LG(2) TBE_FLOOR_LG(3) TBE_FLOOR_LG(4) TBE_FLOOR_LG(5)
    default: return -1;
  }
#undef TBE_FLOOR_LG
}
