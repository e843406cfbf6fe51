// sparse_ops.hip — gfx950 kernels and C ABI of block_bucketize_sparse_features
// (include/tbe_sparse_ops.h).
//
// Reference (paths relative to the reference repository root):
//   BA = src/sparse_ops/block_bucketize_sparse_features/block_bucketize_sparse_features.cpp
//   BK = src/sparse_ops/block_bucketize_sparse_features/c310/op_kernel/block_bucketize_sparse_features_kernel_full.h
//
// Three phases, as in BA:142-231: count the indices of every (bucket, row)
// segment, turn the counts into segment offsets with a device scan, scatter.  One
// 64-wide wavefront owns one row at a time and walks its indices in chunks of
// kChunk x 64 (all loads of a chunk in flight at once); the row metadata of 64
// rows is loaded together, one row per lane.  Buckets divide by a per-row
// multiply-shift reciprocal.  For my_size <= 64 the count phase adds into a
// per-wave LDS histogram, and the scatter phase counting-sorts each chunk by
// bucket in LDS so that its stores run along segments; larger my_size groups the
// lanes of a bucket with a ballot loop (one pass per distinct bucket in a step)
// and advances in-memory counters with one atomic per group.  Only the owning
// wave touches a row's counters and ranks follow index order, so segments are
// filled in row order and the result is deterministic, including for
// sequence = 0 where the reference's per-lane atomics (BK:582-584) leave the
// order inside a segment unspecified.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "tbe_internal.h"
#include "tbe_nbit.h"
#include "tbe_sparse_ops.h"

namespace tbe {
namespace {

constexpr int kWaveBB = 64;
constexpr int kChunk = 8;                            // index loads in flight per wave
constexpr int kRsrcWord3 = 0x00020000;               // raw buffer resource word 3 (gfx9: 32-bit data, no swizzle)
constexpr int kBBBlock = 256;
constexpr int kScanItems = 4;                        // elements per thread in the scan
constexpr int kScanTile = kBBBlock * kScanItems;     // elements per scan work-group

template <typename IT, typename OT>
struct BBParams {
  const IT* __restrict__ indices;
  const OT* __restrict__ offsets;
  const IT* __restrict__ block_sizes;
  const float* __restrict__ weights;
  const OT* __restrict__ bso;
  const IT* __restrict__ tnb;
  const IT* const* __restrict__ pos;
  const int64_t* __restrict__ pos_len;
  OT* __restrict__ new_lengths;
  const OT* __restrict__ new_offsets;
  IT* __restrict__ new_indices;
  float* __restrict__ new_weights;
  IT* __restrict__ new_pos;
  IT* __restrict__ unb;
  uint32_t* __restrict__ done;  // [my_size * L] write cursors of the scatter (my_size > 64)
  uint8_t* __restrict__ slow;   // [L] my_size <= 64: rows the scatter maps with the general code
  int64_t L;
  int64_t N;
  int64_t my_size;
  int64_t B;                    // rows per feature without batch_size_offsets
  int32_t F;
  int32_t keep;
};

// An element of device memory read through a global (not flat) load.  The position
// lists are reached through pointers read from memory, which the compiler would
// otherwise load with flat instructions; a flat load also counts as an LDS
// operation, so the LDS waits of the histogram and sort code would wait for it.
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
  using G = const __attribute__((address_space(1))) T;
  return *(G*)(p);
}

__device__ __forceinline__ int64_t uni(int64_t v) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v & 0xFFFFFFFF)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// n / d for a wave-uniform 32-bit divisor d >= 1 by multiply and shift
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, figure 4.1): l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0)
// with t = mulhi(m, n); exact for every 32-bit n.
struct FastDiv32 {
  uint32_t d, m, s1, s2;
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint32_t t = __umulhi(m, n);
    return (t + ((n - t) >> s1)) >> s2;
  }
};

__device__ __forceinline__ FastDiv32 make_fastdiv(uint32_t d) {
  FastDiv32 f;
  const uint32_t l = d > 1 ? 32u - static_cast<uint32_t>(__clz(static_cast<int>(d - 1))) : 0u;
  f.d = d;
  f.m = static_cast<uint32_t>(((static_cast<uint64_t>((uint64_t(1) << l) - d)) << 32) / d + 1);
  f.s1 = l < 1 ? l : 1u;
  f.s2 = l > 0 ? l - 1 : 0u;
  return f;
}

// What a wave needs to map the indices of one row.  A wave computes these for
// up to 64 of its rows at once, one row per lane (row_ctx_lane), and hands the
// row it is about to walk to every lane with readlane (row_ctx_of), so the
// offsets and per-feature loads of 64 rows share one memory round trip.
// `fast` marks the rows whose indices below gsize take the 32-bit
// multiply-shift division by lsize: no bucketize_pos, blk > 0, gsize < 2^32.
template <typename IT>
struct RowCtx {
  using UIT = std::make_unsigned_t<IT>;
  bool ok;
  bool fast;
  int64_t s, e;
  IT blk;
  UIT gb, lbk, gsize, lsize, scalar;
  const IT* pos;
  int64_t pos_len;
  FastDiv32 dl;
};

// BK:322-347 (row -> feature) and BK:388-421 (per-feature parameters) for row r
// of this lane; r < 0 gives ok = false.
template <typename IT, typename OT>
__device__ __forceinline__ RowCtx<IT> row_ctx_lane(const BBParams<IT, OT>& p, int64_t r) {
  using UIT = std::make_unsigned_t<IT>;
  RowCtx<IT> c{};
  c.ok = false;
  if (r < 0) return c;
  int f;
  if (p.bso) {
    int lo = 0, hi = p.F;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (static_cast<int64_t>(p.bso[mid]) <= r) lo = mid; else hi = mid - 1;
    }
    f = lo;
  } else {
    const uint64_t bdiv = static_cast<uint64_t>(p.B > 0 ? p.B : 1);
    f = ((static_cast<uint64_t>(r) | bdiv) >> 32) == 0
            ? static_cast<int>(static_cast<uint32_t>(r) / static_cast<uint32_t>(bdiv))
            : static_cast<int>(static_cast<uint64_t>(r) / bdiv);
  }
  if (f < 0 || f >= p.F) return c;
  const IT blk = p.block_sizes[f];
  if (blk < 0) return c;
  c.ok = true;
  const IT my = static_cast<IT>(p.my_size);
  IT gb = p.tnb ? p.tnb[f] : my;
  if (gb <= 0) gb = my;
  IT lbk = p.tnb ? static_cast<IT>(gb / my) : IT(1);
  if (lbk <= 0) lbk = 1;
  c.blk = blk;
  c.gb = static_cast<UIT>(gb);
  c.lbk = static_cast<UIT>(lbk);
  c.gsize = static_cast<UIT>(static_cast<UIT>(blk) * static_cast<UIT>(gb));
  c.lsize = static_cast<UIT>(static_cast<UIT>(blk) * static_cast<UIT>(lbk));
  c.pos = nullptr;
  c.pos_len = 0;
  if (p.pos) {
    c.pos = p.pos[f];
    c.pos_len = p.pos_len[f];
    if (!c.pos || c.pos_len <= 0) {
      c.pos = nullptr;
      c.pos_len = 0;
    }
  }
  c.scalar = 1;
  if (c.pos && blk == 0) c.scalar = static_cast<UIT>(static_cast<UIT>(ldg(c.pos + (c.pos_len - 1))) / c.gb);
  c.fast = !c.pos && blk > 0 && c.lsize > 0 && (static_cast<uint64_t>(c.gsize) >> 32) == 0 &&
           (static_cast<uint64_t>(c.lsize) >> 32) == 0;
  c.dl = make_fastdiv(c.fast ? static_cast<uint32_t>(c.lsize) : 1u);
  int64_t s = r == 0 ? 0 : static_cast<int64_t>(p.offsets[r - 1]);
  int64_t e = static_cast<int64_t>(p.offsets[r]);
  s = std::min<int64_t>(std::max<int64_t>(s, 0), p.N);  // malformed offsets never read out of bounds
  e = std::min<int64_t>(std::max<int64_t>(e, s), p.N);
  c.s = s;
  c.e = e;
  return c;
}

__device__ __forceinline__ uint32_t rdl(uint32_t v, int j) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), j));
}
template <typename T>
__device__ __forceinline__ T rdl_of(T v, int j) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = static_cast<uint64_t>(v);
    return static_cast<T>((static_cast<uint64_t>(rdl(static_cast<uint32_t>(u >> 32), j)) << 32) |
                          rdl(static_cast<uint32_t>(u), j));
  } else {
    return static_cast<T>(rdl(static_cast<uint32_t>(v), j));
  }
}

// Lane j's row context, wave-uniform.
template <typename IT>
__device__ __forceinline__ RowCtx<IT> row_ctx_of(const RowCtx<IT>& m, int j) {
  RowCtx<IT> c;
  c.ok = rdl(m.ok ? 1u : 0u, j) != 0;
  c.fast = rdl(m.fast ? 1u : 0u, j) != 0;
  c.s = rdl_of(m.s, j);
  c.e = rdl_of(m.e, j);
  c.blk = rdl_of(m.blk, j);
  c.gb = rdl_of(m.gb, j);
  c.lbk = rdl_of(m.lbk, j);
  c.gsize = rdl_of(m.gsize, j);
  c.lsize = rdl_of(m.lsize, j);
  c.scalar = rdl_of(m.scalar, j);
  c.pos = reinterpret_cast<const IT*>(rdl_of(reinterpret_cast<uint64_t>(m.pos), j));
  c.pos_len = rdl_of(m.pos_len, j);
  c.dl.d = rdl(m.dl.d, j);
  c.dl.m = rdl(m.dl.m, j);
  c.dl.s1 = rdl(m.dl.s1, j);
  c.dl.s2 = rdl(m.dl.s2, j);
  return c;
}

// a / d and a % d; 64-bit operands that fit in 32 bits take the 32-bit divide.
template <typename UIT>
__device__ __forceinline__ void divmod(UIT a, UIT d, UIT& q, UIT& r) {
  if constexpr (sizeof(UIT) == 8) {
    if (((a | d) >> 32) == 0) {
      const uint32_t q32 = static_cast<uint32_t>(a) / static_cast<uint32_t>(d);
      q = q32;
      r = a - static_cast<UIT>(q32) * d;
      return;
    }
  }
  q = a / d;
  r = a - q * d;
}

// BK:423-453 (bucket) and BK:560-603 (new index).  Returns false for an index
// whose bucket falls outside [0, my_size).
template <typename IT>
__device__ __forceinline__ bool map_index(const RowCtx<IT>& c, std::make_unsigned_t<IT> u, uint64_t my, bool keep,
                                          int64_t& bucket, IT& nidx) {
  using UIT = std::make_unsigned_t<IT>;
  if (c.pos) {
    UIT adj = u;
    if (c.blk == 0) adj = static_cast<UIT>((u % c.gb) * c.scalar);
    int64_t first = 0, last = c.pos_len;
    while (first < last) {
      const int64_t mid = first + ((last - first) >> 1);
      if (static_cast<UIT>(ldg(c.pos + mid)) <= adj) first = mid + 1; else last = mid;
    }
    const int64_t lb = first - 1;
    const bool in = lb >= 0 && static_cast<uint64_t>(lb) < my;
    bucket = in ? lb : static_cast<int64_t>(static_cast<uint64_t>(u) % my);
    if (keep) nidx = static_cast<IT>(u);
    else if (c.blk == 0) nidx = static_cast<IT>(u / c.gb);
    else if (in) nidx = static_cast<IT>(static_cast<UIT>(u - static_cast<UIT>(ldg(c.pos + lb))));
    else nidx = static_cast<IT>(static_cast<uint64_t>(u) / my);
  } else if (c.blk != 0 && u < c.gsize) {
    UIT q, r;
    divmod<UIT>(u, c.lsize, q, r);
    bucket = static_cast<int64_t>(q);
    nidx = keep ? static_cast<IT>(u) : static_cast<IT>(r);
  } else {
    UIT q, r, qb, rb;
    divmod<UIT>(u, c.gb, q, r);
    divmod<UIT>(r, c.lbk, qb, rb);
    bucket = static_cast<int64_t>(qb);
    nidx = keep ? static_cast<IT>(u) : static_cast<IT>(q);
  }
  return static_cast<uint64_t>(bucket) < my;
}

// Maps one step's index u of this lane (in: the lane holds an index of the row).
// For rows marked fast, when no lane of the wave holds an index at or above
// gsize (the wave-uniform common case), bucket = u / lsize and new index
// u % lsize by the 32-bit multiply-shift division, without branches; otherwise
// the general map_index.  ONLY_FAST: the caller has checked that every index of
// the step is below gsize, so the general code is not compiled in (it costs the
// scatter ~17 VGPRs and ~8 % of its time).
template <bool FAST, typename IT, bool ONLY_FAST = false>
__device__ __forceinline__ bool map_step(const RowCtx<IT>& c, bool in, std::make_unsigned_t<IT> u, uint64_t my,
                                         bool keep, int64_t& bucket, IT& nidx) {
  if constexpr (ONLY_FAST) {
    const uint32_t n = static_cast<uint32_t>(u);
    const uint32_t q = c.dl.div(n);
    bucket = static_cast<int64_t>(q);
    nidx = keep ? static_cast<IT>(u) : static_cast<IT>(n - q * c.dl.d);
    return in && q < my;
  }
  if constexpr (FAST) {
    if (__builtin_amdgcn_ballot_w64(in && !(u < c.gsize)) == 0) {
      const uint32_t n = static_cast<uint32_t>(u);
      const uint32_t q = c.dl.div(n);
      bucket = static_cast<int64_t>(q);
      nidx = keep ? static_cast<IT>(u) : static_cast<IT>(n - q * c.dl.d);
      return in && q < my;
    }
  }
  return in && map_index<IT>(c, u, my, keep, bucket, nidx);
}

// The rows of one wave: each work-group takes a contiguous run of rows and its
// waves interleave over it, so the group's waves walk neighbouring rows at the
// same time (their segments of one bucket are neighbours in the output) and a
// wave's rows mostly share one feature.
//
// The scatter passes `reverse`: its work-groups take the row ranges last to first.
// The count phase reads the indices roughly first to last (work-groups start in
// order), so the indices it read last are still in the memory-side cache when the
// scatter starts on them (i64_stress: 327 -> 322 us with fresh inputs each call).
__device__ __forceinline__ void wave_rows(int64_t L, int64_t& r0, int64_t& r1, int64_t& rs, bool reverse = false) {
  const int64_t per = (L + gridDim.x - 1) / gridDim.x;
  const int64_t bid = reverse ? gridDim.x - 1 - blockIdx.x : blockIdx.x;
  const int64_t b0 = std::min<int64_t>(bid * per, L);
  r0 = b0 + (threadIdx.x >> 6);
  r1 = std::min<int64_t>(b0 + per, L);
  rs = kBBBlock / kWaveBB;
}

// Integer add on an int32 / int64 counter (two's complement: the unsigned add is the same).
__device__ __forceinline__ void add_count(int32_t* a, uint32_t v) { atomicAdd(reinterpret_cast<unsigned int*>(a), v); }
__device__ __forceinline__ void add_count(int64_t* a, uint32_t v) {
  atomicAdd(reinterpret_cast<unsigned long long*>(a), static_cast<unsigned long long>(v));
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & (kWaveBB - 1)); }

__device__ __forceinline__ uint64_t lanes_below() {
  return (uint64_t(1) << lane_id()) - 1;  // lane 0: 0
}

// Bucket ranks without a pass per bucket (my_size <= 2^NB <= 64): one ballot
// per bit of the bucket number; the lanes whose bucket equals `key` are the
// valid lanes that agree with `key` on every bit.
template <int NB>
struct BucketBits {
  uint64_t valid;
  uint64_t bit[NB];
};

template <int NB>
__device__ __forceinline__ BucketBits<NB> bucket_bits(bool valid, uint32_t bucket) {
  BucketBits<NB> r;
  r.valid = __builtin_amdgcn_ballot_w64(valid);
  const uint32_t bv = valid ? bucket : 0u;  // invalid lanes set no bit
#pragma unroll
  for (int j = 0; j < NB; ++j) r.bit[j] = __builtin_amdgcn_ballot_w64((bv >> j) & 1u);
  return r;
}

template <int NB>
__device__ __forceinline__ uint64_t lanes_with_bucket(const BucketBits<NB>& bb, uint32_t key) {
  uint32_t lo = static_cast<uint32_t>(bb.valid), hi = static_cast<uint32_t>(bb.valid >> 32);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const uint32_t k = static_cast<uint32_t>(static_cast<int32_t>(key << (31 - j)) >> 31);  // bit j of key, all ones or zeros
    lo &= ~(static_cast<uint32_t>(bb.bit[j]) ^ k);
    hi &= ~(static_cast<uint32_t>(bb.bit[j] >> 32) ^ k);
  }
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <typename T>
__global__ __launch_bounds__(kBBBlock) void bb_fill_zero(T* __restrict__ a, int64_t n, uint32_t* __restrict__ b,
                                                        int64_t nb) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * kBBBlock;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kBBBlock) + threadIdx.x; i < n; i += step) a[i] = T(0);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kBBBlock) + threadIdx.x; i < nb; i += step) b[i] = 0u;
}

// Phase 1 (BK:350-456): new_lengths[bucket * L + r] for every row r.  With
// REG (my_size <= 64) every index adds one to its bucket's slot of a per-wave
// 64-entry LDS histogram (an LDS atomic, no return value) and every row stores
// all its my_size counts; otherwise counts go to new_lengths (zero-filled first)
// with one atomic per (step, bucket).  A row's indices are read in chunks of
// kChunk x 64 with all loads of a chunk in flight; with REG the first chunk of
// the next row loads while the current row is counted.
template <bool FAST, bool REG, typename IT, typename OT>
__device__ __forceinline__ void count_row(const BBParams<IT, OT>& p, const RowCtx<IT>& c, int64_t r, uint32_t* hist,
                                          const std::make_unsigned_t<IT> (*first)[kChunk]) {
  using UIT = std::make_unsigned_t<IT>;
  const UIT* __restrict__ idx = reinterpret_cast<const UIT*>(p.indices);
  auto count_chunk = [&](int64_t chunk, const UIT (&uk)[kChunk]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      const int64_t base = chunk + k * kWaveBB;
      if (base >= c.e) break;
      const int64_t i = base + lane_id();
      int64_t b = 0;
      IT v;
      bool valid = map_step<FAST, IT>(c, i < c.e, uk[k], p.my_size, p.keep, b, v);
      if constexpr (REG) {
        if (valid) atomicAdd(hist + static_cast<uint32_t>(b), 1u);
      } else {
        uint64_t pending = __builtin_amdgcn_ballot_w64(valid);
        while (pending) {
          const int leader = __builtin_ctzll(pending);
          const int64_t bl = uni(__builtin_amdgcn_readlane(static_cast<int>(b), leader)) & 0xFFFFFFFFll;
          const bool mine = valid && b == bl;
          const uint64_t m = __builtin_amdgcn_ballot_w64(mine);
          const uint32_t n = static_cast<uint32_t>(__builtin_popcountll(m));
          if (lane_id() == leader) add_count(p.new_lengths + bl * p.L + r, n);
          pending &= ~m;
          valid = valid && !mine;
        }
      }
    }
  };
  int64_t chunk = c.s;
  if (first && chunk < c.e) {  // loaded while the previous row was counted: its own
    count_chunk(chunk, *first);  // code path, so no wait here covers later loads
    chunk += kChunk * kWaveBB;
  }
  for (; chunk < c.e; chunk += kChunk * kWaveBB) {
    UIT uk[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k)  // clamped, not branched: the row is not empty
      uk[k] = idx[std::min<int64_t>(chunk + k * kWaveBB + lane_id(), c.e - 1)];
    count_chunk(chunk, uk);
  }
}

// The first chunk of a row's indices (up to kChunk x 64) with range-checked
// buffer loads: lanes past the row, and rows that do not exist (j >= nrows) or
// are empty, read zero.  Every call issues the same kChunk loads, so the wait for
// them is exact whatever rows exist.
template <typename IT, typename OT>
__device__ __forceinline__ void load_first_chunk(const BBParams<IT, OT>& p, const RowCtx<IT>& c, bool exists,
                                                 std::make_unsigned_t<IT> (&uk)[kChunk]) {
  using UIT = std::make_unsigned_t<IT>;
  // wave-uniform by construction; readfirstlane keeps the descriptor in SGPRs
  const int n = __builtin_amdgcn_readfirstlane(
      exists && c.ok ? static_cast<int>(std::min<int64_t>(c.e - c.s, kChunk * kWaveBB)) : 0);
  const int64_t first = uni(n > 0 ? c.s : 0);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<IT*>(p.indices) + first, 0, n * static_cast<int>(sizeof(IT)), kRsrcWord3);
#pragma unroll
  for (int k = 0; k < kChunk; ++k) {
    const int off = (k * kWaveBB + lane_id()) * static_cast<int>(sizeof(IT));
    if constexpr (sizeof(IT) == 8) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
      uk[k] = static_cast<UIT>((static_cast<uint64_t>(v[1]) << 32) | v[0]);
    } else {
      uk[k] = static_cast<UIT>(__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
    }
  }
}

template <typename IT, typename OT, bool REG>
__global__ __launch_bounds__(kBBBlock) void bb_count(BBParams<IT, OT> p) {
  using UIT = std::make_unsigned_t<IT>;
  __shared__ uint32_t lds_hist[kBBBlock / kWaveBB][kWaveBB];
  uint32_t* hist = lds_hist[threadIdx.x >> 6];
  if constexpr (REG) hist[lane_id()] = 0;
  int64_t r0, r1, rs;
  wave_rows(p.L, r0, r1, rs);
  for (int64_t g0 = r0; g0 < r1; g0 += kWaveBB * rs) {
    const int64_t rl = g0 + lane_id() * rs;
    const RowCtx<IT> mine = row_ctx_lane(p, rl < r1 ? rl : -1);
    const int nrows = static_cast<int>(std::min<int64_t>(kWaveBB, (r1 - g0 + rs - 1) / rs));
    if constexpr (REG) {
      // row j is counted while the first indices of row j + 1 load (two buffers,
      // no register copies: a copy would wait for the load)
      auto count_one = [&](int j, const UIT (&buf)[kChunk]) __attribute__((always_inline)) {
        const int64_t r = g0 + j * rs;
        const RowCtx<IT> c = row_ctx_of(mine, j);
        if (c.ok) {
          if (c.fast) count_row<true, true>(p, c, r, hist, &buf);
          else count_row<false, true>(p, c, r, hist, &buf);
        }
        // the wave's LDS operations complete in order: the reads see every add
        const uint32_t cnt = hist[lane_id()];
        hist[lane_id()] = 0;
        if (lane_id() < p.my_size) p.new_lengths[lane_id() * p.L + r] = static_cast<OT>(cnt);
      };
      auto prefetch = [&](int j, UIT (&buf)[kChunk]) __attribute__((always_inline)) {
        load_first_chunk(p, row_ctx_of(mine, std::min(j, kWaveBB - 1)), j < nrows, buf);
      };
      UIT ba[kChunk], bb[kChunk];
      prefetch(0, ba);
      for (int j = 0; j < nrows; j += 2) {
        prefetch(j + 1, bb);
        count_one(j, ba);
        if (j + 1 >= nrows) break;
        prefetch(j + 2, ba);
        count_one(j + 1, bb);
      }
    } else {
      for (int j = 0; j < nrows; ++j) {
        const RowCtx<IT> c = row_ctx_of(mine, j);
        if (!c.ok) continue;
        if (c.fast) count_row<true, false>(p, c, g0 + j * rs, hist, nullptr);
        else count_row<false, false>(p, c, g0 + j * rs, hist, nullptr);
      }
    }
  }
}

// Phase 3 (BK:458-606 and 608-762): write every index to its segment, in row
// order.
//
// my_size <= 64 (NB = ceil(log2 my_size) rounded up to 4 or 6): a wave walks its
// row in chunks of up to kChunk * 64 indices and counting-sorts each chunk by
// bucket in LDS before writing it, so consecutive lanes store consecutive
// positions of one segment instead of 64 lanes hitting ~my_size segments:
//   1. map every index, count the chunk's indices per bucket (LDS atomics);
//   2. exclusive scan of the counts over the buckets (lane b = bucket b) gives
//      each bucket's first slot in the chunk; the row's write cursor of bucket
//      b (LDS, loaded from new_offsets at the row's first chunk) minus that
//      slot is the slot -> output offset of bucket b;
//   3. every index takes slot = first slot of its bucket + its rank among the
//      chunk's earlier indices of that bucket (one ballot per bit of the bucket
//      number; the highest lane of each bucket advances the bucket's slot);
//   4. the wave writes the slots out in order, 64 at a time.
// Ranks follow index order, so every segment keeps the row's order.
//
// my_size > 64: the cursors are per-segment counters in the workspace,
// advanced with one atomic per (step, bucket), and indices are written in place.
template <typename IT>
struct ScatterStage {
  IT v[kChunk * kWaveBB];         // new index of each slot
  uint32_t meta[kChunk * kWaveBB];  // bucket | (position in the chunk << 8)
  int64_t cur[kWaveBB];           // row's next output offset per bucket
  int64_t delta[kWaveBB];         // output offset - slot, per bucket, this chunk
  uint32_t cnt[kWaveBB];          // chunk count, then next slot, per bucket
};

__device__ __forceinline__ uint32_t wave_exclusive_scan(uint32_t x) {
  uint32_t s = x;
#pragma unroll
  for (int d = 1; d < kWaveBB; d <<= 1) {
    const uint32_t t = static_cast<uint32_t>(__shfl_up(static_cast<int>(s), d, kWaveBB));
    if (lane_id() >= d) s += t;
  }
  return s - x;
}

//
// ONLY_FAST (rows marked fast): gives up on the row, returning false, at the
// first chunk holding an index at or above gsize, before writing anything of that
// chunk; the general pass then rewrites the whole row (the same values at the same
// positions).  Returns true when the row is done.
template <bool FAST, int NB, typename IT, typename OT, bool ONLY_FAST = false>
__device__ __forceinline__ bool scatter_row_staged(const BBParams<IT, OT>& p, const RowCtx<IT>& c, int64_t r,
                                                   ScatterStage<IT>& st) {
  using UIT = std::make_unsigned_t<IT>;
  constexpr uint32_t kNone = 0xFFu;
  const UIT* __restrict__ idx = reinterpret_cast<const UIT*>(p.indices);
  const int lane = lane_id();
  for (int64_t chunk = c.s; chunk < c.e; chunk += kChunk * kWaveBB) {
    UIT uk[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k)  // clamped, not branched: the row is not empty
      uk[k] = idx[std::min<int64_t>(chunk + k * kWaveBB + lane, c.e - 1)];
    // the row's cursors, loaded with its first indices (one wait for both)
    if (chunk == c.s && lane < p.my_size) st.cur[lane] = static_cast<int64_t>(p.new_offsets[lane * p.L + r]);
    if constexpr (ONLY_FAST) {
      bool high = false;
#pragma unroll
      for (int k = 0; k < kChunk; ++k) high |= chunk + k * kWaveBB + lane < c.e && !(uk[k] < c.gsize);
      if (__builtin_amdgcn_ballot_w64(high) != 0) return false;
    }
    // 1. map and count
    uint32_t bk[kChunk];
    IT vk[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      bk[k] = kNone;
      vk[k] = 0;
      const int64_t base = chunk + k * kWaveBB;
      if (base < c.e) {
        int64_t b = 0;
        IT v = 0;
        if (map_step<FAST, IT, ONLY_FAST>(c, base + lane < c.e, uk[k], p.my_size, p.keep, b, v)) {
          bk[k] = static_cast<uint32_t>(b);
          vk[k] = v;
          atomicAdd(&st.cnt[b], 1u);
        }
      }
    }
    // 2. first slot per bucket and slot -> output offset
    const uint32_t n = st.cnt[lane];
    const uint32_t first = wave_exclusive_scan(n);
    const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(first + n), kWaveBB - 1));
    const int64_t cu = st.cur[lane];
    st.delta[lane] = cu - static_cast<int64_t>(first);
    st.cur[lane] = cu + n;
    st.cnt[lane] = first;
    // 3. slots
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      if (chunk + k * kWaveBB >= c.e) break;
      const bool valid = bk[k] != kNone;
      const BucketBits<NB> bb = bucket_bits<NB>(valid, bk[k]);
      const uint64_t mine = lanes_with_bucket<NB>(bb, bk[k]);
      if (valid) {
        // every lane reads before the highest lane of the bucket writes (in-order LDS)
        const uint32_t slot = st.cnt[bk[k]] + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mine >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mine), 0u));
        if ((mine >> lane) == 1) st.cnt[bk[k]] = slot + 1;
        st.v[slot] = vk[k];
        st.meta[slot] = bk[k] | (static_cast<uint32_t>(k * kWaveBB + lane) << 8);
      }
    }
    // 4. write out in slot order
    for (uint32_t t0 = 0; t0 < total; t0 += kWaveBB) {
      const uint32_t t = t0 + static_cast<uint32_t>(lane);
      if (t < total) {
        const uint32_t m = st.meta[t];
        const int64_t w = st.delta[m & 0xFFu] + t;
        const int64_t i = chunk + (m >> 8);
        if (w >= 0 && w < p.N) {
          p.new_indices[w] = st.v[t];
          if (p.new_weights) p.new_weights[w] = p.weights[i];
          if (p.new_pos) p.new_pos[w] = static_cast<IT>(i - c.s);
          if (p.unb) p.unb[i] = static_cast<IT>(w);
        }
      }
    }
    st.cnt[lane] = 0;
  }
  return true;
}

template <bool FAST, typename IT, typename OT>
__device__ __forceinline__ void scatter_row_atomic(const BBParams<IT, OT>& p, const RowCtx<IT>& c, int64_t r) {
  using UIT = std::make_unsigned_t<IT>;
  const UIT* __restrict__ idx = reinterpret_cast<const UIT*>(p.indices);
  for (int64_t chunk = c.s; chunk < c.e; chunk += kChunk * kWaveBB) {
    UIT uk[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k)  // clamped, not branched: the row is not empty
      uk[k] = idx[std::min<int64_t>(chunk + k * kWaveBB + lane_id(), c.e - 1)];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
      const int64_t base = chunk + k * kWaveBB;
      if (base >= c.e) break;
      const int64_t i = base + lane_id();
      int64_t b = 0;
      IT v = 0;
      const bool valid0 = map_step<FAST, IT>(c, i < c.e, uk[k], p.my_size, p.keep, b, v);
      int64_t w = 0;
      bool valid = valid0;
      uint64_t pending = __builtin_amdgcn_ballot_w64(valid);
      while (pending) {
        const int leader = __builtin_ctzll(pending);
        const int64_t bl = uni(__builtin_amdgcn_readlane(static_cast<int>(b), leader)) & 0xFFFFFFFFll;
        const bool mine = valid && b == bl;
        const uint64_t m = __builtin_amdgcn_ballot_w64(mine);
        const uint32_t cnt = static_cast<uint32_t>(__builtin_popcountll(m));
        uint32_t old = 0;
        if (lane_id() == leader) old = atomicAdd(p.done + bl * p.L + r, cnt);
        old = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(old), leader));
        const int64_t seg0 = static_cast<int64_t>(p.new_offsets[bl * p.L + r]) + old;
        if (mine) w = seg0 + __builtin_popcountll(m & lanes_below());
        pending &= ~m;
        valid = valid && !mine;
      }
      if (valid0 && w >= 0 && w < p.N) {
        p.new_indices[w] = v;
        if (p.new_weights) p.new_weights[w] = p.weights[i];
        if (p.new_pos) p.new_pos[w] = static_cast<IT>(i - c.s);
        if (p.unb) p.unb[i] = static_cast<IT>(w);
      }
    }
  }
}

// PASS (my_size <= 64): 1 takes every row marked fast with the fast map only and
// flags (`slow`, one byte per row) the rows it leaves: those not marked fast and
// those holding an index at or above gsize; 2 takes the flagged rows with the
// general map.  Two kernels, so the general map's registers do not limit the fast
// pass.  my_size > 64: PASS 0, every row.
template <typename IT, typename OT, int NB, int PASS>
__global__ __launch_bounds__(kBBBlock) void bb_scatter(BBParams<IT, OT> p) {
  __shared__ ScatterStage<IT> lds_stage[NB > 0 ? kBBBlock / kWaveBB : 1];
  ScatterStage<IT>& st = lds_stage[NB > 0 ? (threadIdx.x >> 6) : 0];
  if constexpr (NB > 0) st.cnt[lane_id()] = 0;
  int64_t r0, r1, rs;
  if constexpr (PASS == 2) {
    // few rows if any: each wave checks 64 consecutive rows' flags at a time
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (kBBBlock / kWaveBB);
    r0 = (static_cast<int64_t>(blockIdx.x) * (kBBBlock / kWaveBB) + (threadIdx.x >> 6)) * kWaveBB;
    r1 = p.L;
    rs = 1;
    for (int64_t g0 = r0; g0 < r1; g0 += waves * kWaveBB) {
      const int64_t rl = g0 + lane_id();
      uint64_t take = __builtin_amdgcn_ballot_w64(rl < r1 && p.slow[rl] != 0);
      if (take == 0) continue;  // wave-uniform
      const RowCtx<IT> mine = row_ctx_lane(p, rl < r1 ? rl : -1);
      while (take) {
        const int j = __builtin_ctzll(take);
        take &= take - 1;
        const RowCtx<IT> c = row_ctx_of(mine, j);
        if (!c.ok) continue;
        if (c.fast) scatter_row_staged<true, NB>(p, c, g0 + j, st);
        else scatter_row_staged<false, NB>(p, c, g0 + j, st);
      }
    }
    return;
  }
  wave_rows(p.L, r0, r1, rs, true);
  for (int64_t g0 = r0; g0 < r1; g0 += kWaveBB * rs) {
    const int64_t rl = g0 + lane_id() * rs;
    uint64_t take = __builtin_amdgcn_ballot_w64(rl < r1);
    const RowCtx<IT> mine = row_ctx_lane(p, rl < r1 ? rl : -1);
    while (take) {
      const int j = __builtin_ctzll(take);
      take &= take - 1;
      const int64_t r = g0 + j * rs;
      const RowCtx<IT> c = row_ctx_of(mine, j);
      if constexpr (PASS == 1) {
        const bool done = !c.ok || (c.fast && scatter_row_staged<true, NB, IT, OT, true>(p, c, r, st));
        if (lane_id() == 0) p.slow[r] = done ? 0 : 1;
        continue;
      }
      if (!c.ok) continue;
      if constexpr (NB > 0) {
        if (c.fast) scatter_row_staged<true, NB>(p, c, r, st);
        else scatter_row_staged<false, NB>(p, c, r, st);
      } else {
        if (c.fast) scatter_row_atomic<true>(p, c, r);
        else scatter_row_atomic<false>(p, c, r);
      }
    }
  }
}

// Phase 2: out[0] = 0, out[k + 1] = in[0] + ... + in[k] over n elements, in three
// passes: tile sums, an exclusive scan of the tile sums by one work-group, then
// each tile's scan plus its base.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* lds_wave, T& total) {
  // inclusive scan inside the wave with DPP-free shuffles, then across the 4 waves
  const int lane = lane_id();
  T x = v;
#pragma unroll
  for (int d = 1; d < kWaveBB; d <<= 1) {
    const T y = __shfl_up(x, d, kWaveBB);
    if (lane >= d) x += y;
  }
  const int w = threadIdx.x >> 6;
  if (lane == kWaveBB - 1) lds_wave[w] = x;
  __syncthreads();
  T wbase = 0;
  total = 0;
  for (int k = 0; k < kBBBlock / kWaveBB; ++k) {
    if (k < w) wbase += lds_wave[k];
    total += lds_wave[k];
  }
  __syncthreads();
  return wbase + x - v;
}

template <typename T>
__global__ __launch_bounds__(kBBBlock) void scan_tile_sums(const T* __restrict__ in, int64_t n, T* __restrict__ sums) {
  __shared__ T lds[kBBBlock / kWaveBB];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * static_cast<int64_t>(kScanItems);
  T s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k)
    if (base + k < n) s += in[base + k];
  T total;
  (void)block_exclusive_scan(s, lds, total);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

template <typename T>
__global__ __launch_bounds__(kBBBlock) void scan_sums_exclusive(T* __restrict__ sums, int64_t m) {
  // one work-group, kSumItems consecutive sums per thread per pass
  constexpr int kSumItems = 8;
  __shared__ T lds[kBBBlock / kWaveBB];
  T carry = 0;
  for (int64_t t0 = 0; t0 < m; t0 += static_cast<int64_t>(kBBBlock) * kSumItems) {
    const int64_t base = t0 + threadIdx.x * static_cast<int64_t>(kSumItems);
    T v[kSumItems];
    T s = 0;
#pragma unroll
    for (int k = 0; k < kSumItems; ++k) {
      v[k] = base + k < m ? sums[base + k] : T(0);
      s += v[k];
    }
    T total;
    T run = carry + block_exclusive_scan(s, lds, total);
#pragma unroll
    for (int k = 0; k < kSumItems; ++k) {
      if (base + k < m) sums[base + k] = run;
      run += v[k];
    }
    carry += total;
  }
}

template <typename T>
__global__ __launch_bounds__(kBBBlock) void scan_tiles(const T* __restrict__ in, int64_t n, const T* __restrict__ sums,
                                                       T* __restrict__ out) {
  __shared__ T lds[kBBBlock / kWaveBB];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * static_cast<int64_t>(kScanItems);
  T v[kScanItems];
  T s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    v[k] = base + k < n ? in[base + k] : T(0);
    s += v[k];
  }
  T total;
  T run = sums[blockIdx.x] + block_exclusive_scan(s, lds, total);
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    run += v[k];
    if (base + k < n) out[base + k + 1] = run;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = T(0);
}

// Up to this many tiles, each tile's work-group sums the tile sums before it itself
// (at most 2048 values, from L2) instead of a separate one-work-group pass over them:
// one launch fewer (the stress case's call: 0.333 -> 0.331 ms).  Above it the sums are
// scanned by scan_sums_exclusive (the per-tile reads would grow with tiles^2).
constexpr int64_t kScanBaseMaxTiles = 2048;

template <typename T>
__global__ __launch_bounds__(kBBBlock) void scan_tiles_based(const T* __restrict__ in, int64_t n,
                                                             const T* __restrict__ sums, T* __restrict__ out) {
  __shared__ T lds[kBBBlock / kWaveBB];
  T part = 0;
  for (int64_t t = threadIdx.x; t < static_cast<int64_t>(blockIdx.x); t += kBBBlock) part += sums[t];
  T base;
  (void)block_exclusive_scan(part, lds, base);  // base = sum of every earlier tile
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * static_cast<int64_t>(kScanItems);
  T v[kScanItems];
  T s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    v[k] = first + k < n ? in[first + k] : T(0);
    s += v[k];
  }
  T total;
  T run = base + block_exclusive_scan(s, lds, total);
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    run += v[k];
    if (first + k < n) out[first + k + 1] = run;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = T(0);
}

int64_t scan_tiles_of(int64_t n) { return (n + kScanTile - 1) / kScanTile; }

// Bytes of the row offsets the library forms when the caller passes lengths only:
// the complete cumsum, L + 1 elements.
int64_t offsets_bytes(int64_t L, int32_t os) { return ((L + 1) * os + 255) / 256 * 256; }

int64_t ws_layout(int64_t my, int64_t L, int32_t os, int64_t* sums_off) {
  // [done: my*L uint32 (my_size <= 64: the first L bytes hold the row flags)][pad to 256]
  // [row offsets: (L + 1) * os][pad to 256][tile sums: tiles * os]
  const int64_t done_bytes = my * L * 4;
  const int64_t so = (done_bytes + 255) / 256 * 256 + offsets_bytes(L, os);
  if (sums_off) *sums_off = so;
  return so + std::max<int64_t>(1, scan_tiles_of(my * L)) * os;
}

// Scratch of the entry point that allocates nothing
// (tbe_block_bucketize_sparse_features_noalloc): one copy per GPU, held until the
// process ends.  Host code never passes `scratch` itself (on the host it is only a
// stand-in symbol); it passes the device address hipGetSymbolAddress returns.
constexpr int64_t kNoAllocScratchBytes = TBE_BLOCK_BUCKETIZE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// Per-GPU state of the entry point that allocates nothing, set up on its first call
// on that GPU (with the GPU current): the scratch array's device address, and an
// event recorded after every eager call, which the next eager call on that GPU (any
// stream, any thread) waits for, so calls that would overlap run one after another
// on the shared scratch instead of racing on it.
struct NoAllocDevice {
  void* scratch = nullptr;
  hipEvent_t done = nullptr;
  bool recorded = false;
};
std::mutex g_noalloc_mu;  // held across a call's set-up, wait, launches and record
NoAllocDevice g_noalloc[kMaxDevices];

// This GPU's state (g_noalloc_mu held).  Returns nullptr and sets the error on failure.
NoAllocDevice* noalloc_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(TBE_ERR_LAUNCH, "no current HIP device");
    return nullptr;
  }
  NoAllocDevice& d = g_noalloc[dev];
  if (!d.scratch) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
      fail(TBE_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(err));
      return nullptr;
    }
    d.scratch = ptr;
  }
  if (!d.done) {
    const hipError_t err = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
    if (err != hipSuccess) {
      d.done = nullptr;
      fail(TBE_ERR_LAUNCH, "hipEventCreateWithFlags failed: %s", hipGetErrorString(err));
      return nullptr;
    }
  }
  return &d;
}

// Scratch bytes a call needs: the per-segment write cursors (my_size > 64; up to 64
// buckets the cursors live in registers and LDS, and the region holds the count
// phase's one-byte row flags instead), the row offsets formed from lengths, and the
// scan's tile sums.
int64_t noalloc_need(int64_t my, int64_t L, int32_t os, int64_t* sums_off) {
  const int64_t done_bytes = ((my > kWaveBB ? my * L * 4 : L) + 255) / 256 * 256 + offsets_bytes(L, os);
  if (sums_off) *sums_off = done_bytes;
  return done_bytes + std::max<int64_t>(1, scan_tiles_of(my * L)) * os;
}

template <typename IT, typename OT>
int run(const TbeBlockBucketizeArgs* a, hipStream_t s, void* ws, int64_t sums_off) {
  BBParams<IT, OT> p{};
  p.indices = static_cast<const IT*>(a->indices);
  p.offsets = static_cast<const OT*>(a->offsets);
  p.block_sizes = static_cast<const IT*>(a->block_sizes);
  p.weights = a->weights;
  p.bso = static_cast<const OT*>(a->batch_size_offsets);
  p.tnb = static_cast<const IT*>(a->total_num_blocks);
  p.pos = reinterpret_cast<const IT* const*>(a->bucketize_pos);
  p.pos_len = a->bucketize_pos_len;
  p.new_lengths = static_cast<OT*>(a->new_lengths);
  p.new_offsets = static_cast<const OT*>(a->new_offsets);
  p.new_indices = static_cast<IT*>(a->new_indices);
  p.new_weights = a->weights ? a->new_weights : nullptr;
  p.new_pos = static_cast<IT*>(a->new_pos);
  p.unb = static_cast<IT*>(a->unbucketize_permute);
  p.done = static_cast<uint32_t*>(ws);
  p.slow = static_cast<uint8_t*>(ws);  // my_size <= 64 only, where the cursors are not used
  OT* sums = reinterpret_cast<OT*>(static_cast<uint8_t*>(ws) + sums_off);
  // offsets given, or formed here from the lengths (BA:167): the complete cumsum sits
  // just below the tile sums, and the kernels read its inclusive part
  OT* formed = reinterpret_cast<OT*>(reinterpret_cast<uint8_t*>(sums) - offsets_bytes(a->lengths_size, a->offset_size));
  if (!a->offsets) p.offsets = formed + 1;
  p.L = a->lengths_size;
  p.N = a->num_indices;
  p.my_size = a->my_size;
  p.B = a->batch_size_offsets ? 0 : a->lengths_size / a->num_features;
  p.F = a->num_features;
  p.keep = a->keep_orig_idx;
  int nbits = 0;  // ceil(log2(my_size))
  while (nbits < 6 && (int64_t(1) << nbits) < a->my_size) ++nbits;
  const int64_t nseg = a->my_size * a->lengths_size;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const int64_t fill_blocks = std::min<int64_t>(std::max<int64_t>(1, (nseg + kBBBlock - 1) / kBBBlock), 8LL * cus);
  // count and scatter: at most 4 rows per wave (one row per wave while that keeps
  // the grid at or below 16 work-groups per CU).  Short row runs per wave even out
  // the waves' finishing times; on i64_stress (131 K rows of ~320 indices) 4 rows per
  // wave beat 8 by 4-5 %, and 3-5 rows per wave (uneven) by 2-3 %.
  const int64_t row_blocks = std::max(std::min<int64_t>(std::max<int64_t>(1, (p.L + 3) / 4), 16LL * cus),
                                      (p.L + 15) / 16);
  const int64_t tiles = std::max<int64_t>(1, scan_tiles_of(nseg));
  if (!a->offsets) {
    // the scans below run after the count, so the two scans share the tile sums
    const OT* len = static_cast<const OT*>(a->lengths);
    const int64_t ltiles = std::max<int64_t>(1, scan_tiles_of(p.L));
    hipLaunchKernelGGL(scan_tile_sums<OT>, dim3(static_cast<uint32_t>(ltiles)), dim3(kBBBlock), 0, s, len, p.L, sums);
    if (ltiles <= kScanBaseMaxTiles) {
      hipLaunchKernelGGL(scan_tiles_based<OT>, dim3(static_cast<uint32_t>(ltiles)), dim3(kBBBlock), 0, s, len, p.L,
                         const_cast<const OT*>(sums), formed);
    } else {
      hipLaunchKernelGGL(scan_sums_exclusive<OT>, dim3(1), dim3(kBBBlock), 0, s, sums, ltiles);
      hipLaunchKernelGGL(scan_tiles<OT>, dim3(static_cast<uint32_t>(ltiles)), dim3(kBBBlock), 0, s, len, p.L,
                         const_cast<const OT*>(sums), formed);
    }
  }
  // counters and cursors in registers when every bucket fits a lane
  const bool reg = a->my_size <= kWaveBB;
  if (!reg)
    hipLaunchKernelGGL(bb_fill_zero<OT>, dim3(static_cast<uint32_t>(fill_blocks)), dim3(kBBBlock), 0, s,
                       p.new_lengths, nseg, p.done, nseg);
  if (reg)
    hipLaunchKernelGGL((bb_count<IT, OT, true>), dim3(static_cast<uint32_t>(row_blocks)), dim3(kBBBlock), 0, s, p);
  else
    hipLaunchKernelGGL((bb_count<IT, OT, false>), dim3(static_cast<uint32_t>(row_blocks)), dim3(kBBBlock), 0, s, p);
  hipLaunchKernelGGL(scan_tile_sums<OT>, dim3(static_cast<uint32_t>(tiles)), dim3(kBBBlock), 0, s,
                     const_cast<const OT*>(p.new_lengths), nseg, sums);
  if (tiles <= kScanBaseMaxTiles) {
    hipLaunchKernelGGL(scan_tiles_based<OT>, dim3(static_cast<uint32_t>(tiles)), dim3(kBBBlock), 0, s,
                       const_cast<const OT*>(p.new_lengths), nseg, const_cast<const OT*>(sums),
                       static_cast<OT*>(a->new_offsets));
  } else {
    hipLaunchKernelGGL(scan_sums_exclusive<OT>, dim3(1), dim3(kBBBlock), 0, s, sums, tiles);
    hipLaunchKernelGGL(scan_tiles<OT>, dim3(static_cast<uint32_t>(tiles)), dim3(kBBBlock), 0, s,
                       const_cast<const OT*>(p.new_lengths), nseg, const_cast<const OT*>(sums),
                       static_cast<OT*>(a->new_offsets));
  }
  if (p.N > 0) {
    const dim3 g(static_cast<uint32_t>(row_blocks));
    // the general pass: one wave per 64 rows, at most one block per CU
    const dim3 g2(static_cast<uint32_t>(std::min<int64_t>(std::max<int64_t>(1, (p.L + 255) / 256), cus)));
    if (!reg) {
      hipLaunchKernelGGL((bb_scatter<IT, OT, 0, 0>), g, dim3(kBBBlock), 0, s, p);
    } else if (nbits <= 4) {
      hipLaunchKernelGGL((bb_scatter<IT, OT, 4, 1>), g, dim3(kBBBlock), 0, s, p);
      hipLaunchKernelGGL((bb_scatter<IT, OT, 4, 2>), g2, dim3(kBBBlock), 0, s, p);
    } else {
      hipLaunchKernelGGL((bb_scatter<IT, OT, 6, 1>), g, dim3(kBBBlock), 0, s, p);
      hipLaunchKernelGGL((bb_scatter<IT, OT, 6, 2>), g2, dim3(kBBBlock), 0, s, p);
    }
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(TBE_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return TBE_OK;
}

}  // namespace
}  // namespace tbe

using namespace tbe;

extern "C" int64_t tbe_block_bucketize_workspace_bytes(int64_t my_size, int64_t lengths_size, int32_t offset_size) {
  if (my_size < 1 || lengths_size < 0 || (offset_size != 4 && offset_size != 8)) return -1;
  return ws_layout(my_size, lengths_size, offset_size, nullptr);
}

namespace tbe {
namespace {

// Argument checks shared by both entry points (BA:37-91, BA:107-128).
int check_args(const TbeBlockBucketizeArgs* a) {
  if (!a) return fail(TBE_ERR_INVALID_ARG, "null args");
  if (a->my_size <= 0) return fail(TBE_ERR_INVALID_ARG, "my_size must be positive.");
  if ((a->index_size != 4 && a->index_size != 8) || (a->offset_size != 4 && a->offset_size != 8))
    return fail(TBE_ERR_INVALID_ARG, "indices and lengths must be int32 or int64");
  if (a->num_features <= 0) return fail(TBE_ERR_INVALID_ARG, "block_sizes must be non-empty.");
  if (a->lengths_size < 0 || a->num_indices < 0) return fail(TBE_ERR_INVALID_ARG, "negative size");
  if (!a->batch_size_offsets && a->lengths_size % a->num_features != 0)
    return fail(TBE_ERR_INVALID_ARG,
                "lengths.size(0) must be divisible by block_sizes.size(0) when batch_size_per_feature is absent.");
  if (a->index_size == 4 && a->my_size > 0xFFFFFFFFLL)
    return fail(TBE_ERR_INVALID_ARG, "my_size must fit into uint32 for int32 tensors.");
  if (a->my_size * a->lengths_size > 0xFFFFFFFFLL)
    return fail(TBE_ERR_UNSUPPORTED, "my_size * lengths_size must stay below 2^32");
  if (a->bucketize_pos && !a->bucketize_pos_len) return fail(TBE_ERR_INVALID_ARG, "missing bucketize_pos_len");
  if (a->weights && !a->new_weights) return fail(TBE_ERR_INVALID_ARG, "weights given without new_weights");
  return TBE_OK;
}

int check_pointers(const TbeBlockBucketizeArgs* a) {
  if (!a->new_lengths || !a->new_offsets ||
      (a->lengths_size > 0 && ((!a->offsets && !a->lengths) || !a->block_sizes)) ||
      (a->num_indices > 0 && (!a->indices || !a->new_indices)))
    return fail(TBE_ERR_INVALID_ARG, "null pointer argument");
  return TBE_OK;
}

int dispatch(const TbeBlockBucketizeArgs* a, hipStream_t s, void* ws, int64_t sums_off) {
  if (a->index_size == 4)
    return a->offset_size == 4 ? run<int32_t, int32_t>(a, s, ws, sums_off) : run<int32_t, int64_t>(a, s, ws, sums_off);
  return a->offset_size == 4 ? run<int64_t, int32_t>(a, s, ws, sums_off) : run<int64_t, int64_t>(a, s, ws, sums_off);
}

}  // namespace
}  // namespace tbe

extern "C" int tbe_block_bucketize_sparse_features(const TbeBlockBucketizeArgs* a, void* hip_stream) {
  clear_error();
  const int rc = check_args(a);
  if (rc != TBE_OK) return rc;
  int64_t sums_off = 0;
  const int64_t need = ws_layout(a->my_size, a->lengths_size, a->offset_size, &sums_off);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(TBE_ERR_INVALID_ARG, "workspace of %lld bytes needed", static_cast<long long>(need));
  if (check_pointers(a) != TBE_OK) return TBE_ERR_INVALID_ARG;
  return dispatch(a, static_cast<hipStream_t>(hip_stream), a->workspace, sums_off);
}

extern "C" int tbe_block_bucketize_sparse_features_noalloc(const TbeBlockBucketizeArgs* a, void* hip_stream) {
  clear_error();
  const int rc = check_args(a);
  if (rc != TBE_OK) return rc;
  int64_t sums_off = 0;
  const int64_t need = noalloc_need(a->my_size, a->lengths_size, a->offset_size, &sums_off);
  if (need > kNoAllocScratchBytes)
    return fail(TBE_ERR_UNSUPPORTED,
                "block_bucketize_sparse_features_noalloc: this call needs %lld bytes of scratch, more than the "
                "%lld the library holds per GPU (my_size * lengths_size too large); use "
                "tbe_block_bucketize_sparse_features with a workspace",
                static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
  if (check_pointers(a) != TBE_OK) return TBE_ERR_INVALID_ARG;
  const hipStream_t s = static_cast<hipStream_t>(hip_stream);
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoAllocDevice* d = noalloc_device();
  if (!d) return TBE_ERR_LAUNCH;
  // Eager calls wait for the previous call on this GPU.  Under graph capture the
  // graph orders the captured call; a wait on (or record of) an event from outside
  // the capture would break the capture, so neither is done there.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess)
    return fail(TBE_ERR_LAUNCH, "hipStreamIsCapturing failed");
  const bool eager = cs == hipStreamCaptureStatusNone;
  if (eager && d->recorded && hipStreamWaitEvent(s, d->done, 0) != hipSuccess)
    return fail(TBE_ERR_LAUNCH, "hipStreamWaitEvent on the previous call failed");
  const int rc2 = dispatch(a, s, d->scratch, sums_off);
  if (eager && rc2 == TBE_OK) {
    if (hipEventRecord(d->done, s) != hipSuccess) return fail(TBE_ERR_LAUNCH, "hipEventRecord failed");
    d->recorded = true;
  }
  return rc2;
}
