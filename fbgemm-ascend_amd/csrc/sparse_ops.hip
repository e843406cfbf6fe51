// sparse_ops.hip — gfx950 kernels and C ABI of block_bucketize_sparse_features
// (include/tbe_sparse_ops.h).
//
// Reference (paths relative to the reference repository root):
//   BA = src/sparse_ops/block_bucketize_sparse_features/block_bucketize_sparse_features.cpp
//   BK = src/sparse_ops/block_bucketize_sparse_features/c310/op_kernel/block_bucketize_sparse_features_kernel_full.h
//
// Three phases, as in BA:142-231: count the indices of every (bucket, row)
// segment, turn the counts into segment offsets with a device scan, scatter.  One
// 64-wide wavefront owns one row at a time and walks its indices 64 per step.
// For my_size <= 64 the row's per-bucket counters and write cursors live in one
// VGPR (lane b = bucket b) and a lane's rank among the lower lanes of its bucket
// comes from one ballot per bit of the bucket number (no pass per bucket, no
// memory); larger my_size groups the lanes of a bucket with a ballot loop (one
// pass per distinct bucket in the step) and advances in-memory counters with one
// atomic per group.  Only the owning wave touches a row's counters,
// so segments are filled in row order and the result is deterministic, including
// for sequence = 0 where the reference's per-lane atomics (BK:582-584) leave the
// order inside a segment unspecified.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "tbe_internal.h"
#include "tbe_nbit.h"
#include "tbe_sparse_ops.h"

namespace tbe {
namespace {

constexpr int kWaveBB = 64;
constexpr int kBBBlock = 256;
constexpr int kScanItems = 16;                       // elements per thread in the scan
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
  uint32_t* __restrict__ done;  // [my_size * L] write cursors of the scatter
  int64_t L;
  int64_t N;
  int64_t my_size;
  int64_t B;                    // rows per feature without batch_size_offsets
  int32_t F;
  int32_t keep;
  int32_t bucket_bits;          // ceil(log2(my_size)) when my_size <= 64
};

__device__ __forceinline__ int64_t uni(int64_t v) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v & 0xFFFFFFFF)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// What a wave needs to map the indices of one row (all values wave-uniform).
template <typename IT>
struct RowCtx {
  using UIT = std::make_unsigned_t<IT>;
  bool ok;
  int64_t s, e;
  IT blk;
  UIT gb, lbk, gsize, lsize, scalar;
  const IT* pos;
  int64_t pos_len;
};

// BK:322-347 (row -> feature) and BK:388-421 (per-feature parameters).
template <typename IT, typename OT>
__device__ __forceinline__ RowCtx<IT> row_ctx(const BBParams<IT, OT>& p, int64_t r) {
  using UIT = std::make_unsigned_t<IT>;
  RowCtx<IT> c{};
  int f;
  if (p.bso) {
    int lo = 0, hi = p.F;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (static_cast<int64_t>(uni(static_cast<int64_t>(p.bso[mid]))) <= r) lo = mid; else hi = mid - 1;
    }
    f = lo;
  } else {
    f = static_cast<int>(r / (p.B > 0 ? p.B : 1));
  }
  c.ok = f >= 0 && f < p.F;
  if (!c.ok) return c;
  const IT blk = static_cast<IT>(uni(static_cast<int64_t>(p.block_sizes[f])));
  c.ok = blk >= 0;
  if (!c.ok) return c;
  const IT my = static_cast<IT>(p.my_size);
  IT gb = p.tnb ? static_cast<IT>(uni(static_cast<int64_t>(p.tnb[f]))) : my;
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
    c.pos = reinterpret_cast<const IT*>(uni(reinterpret_cast<int64_t>(p.pos[f])));
    c.pos_len = uni(p.pos_len[f]);
    if (!c.pos || c.pos_len <= 0) {
      c.pos = nullptr;
      c.pos_len = 0;
    }
  }
  c.scalar = 1;
  if (c.pos && blk == 0) c.scalar = static_cast<UIT>(static_cast<UIT>(c.pos[c.pos_len - 1]) / c.gb);
  int64_t s = r == 0 ? 0 : static_cast<int64_t>(p.offsets[r - 1]);
  int64_t e = static_cast<int64_t>(p.offsets[r]);
  s = std::min<int64_t>(std::max<int64_t>(uni(s), 0), p.N);  // malformed offsets never read out of bounds
  e = std::min<int64_t>(std::max<int64_t>(uni(e), s), p.N);
  c.s = s;
  c.e = e;
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
      if (static_cast<UIT>(c.pos[mid]) <= adj) first = mid + 1; else last = mid;
    }
    const int64_t lb = first - 1;
    const bool in = lb >= 0 && static_cast<uint64_t>(lb) < my;
    bucket = in ? lb : static_cast<int64_t>(static_cast<uint64_t>(u) % my);
    if (keep) nidx = static_cast<IT>(u);
    else if (c.blk == 0) nidx = static_cast<IT>(u / c.gb);
    else if (in) nidx = static_cast<IT>(static_cast<UIT>(u - static_cast<UIT>(c.pos[lb])));
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

// Integer add on an int32 / int64 counter (two's complement: the unsigned add is the same).
__device__ __forceinline__ void add_count(int32_t* a, uint32_t v) { atomicAdd(reinterpret_cast<unsigned int*>(a), v); }
__device__ __forceinline__ void add_count(int64_t* a, uint32_t v) {
  atomicAdd(reinterpret_cast<unsigned long long*>(a), static_cast<unsigned long long>(v));
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & (kWaveBB - 1)); }

__device__ __forceinline__ uint64_t lanes_below() {
  return (uint64_t(1) << lane_id()) - 1;  // lane 0: 0
}

// Bucket ranks without a pass per bucket (my_size <= 64): one ballot per bit of
// the bucket number; the lanes whose bucket equals `key` are the valid lanes that
// agree with `key` on every bit.
constexpr int kMaxBucketBits = 6;

struct BucketBits {
  uint64_t valid;
  uint64_t bit[kMaxBucketBits];
};

__device__ __forceinline__ BucketBits bucket_bits(bool valid, uint32_t bucket, int nbits) {
  BucketBits r;
  r.valid = __builtin_amdgcn_ballot_w64(valid);
#pragma unroll
  for (int j = 0; j < kMaxBucketBits; ++j)
    r.bit[j] = j < nbits ? __builtin_amdgcn_ballot_w64(valid && ((bucket >> j) & 1u)) : 0;
  return r;
}

__device__ __forceinline__ uint64_t lanes_with_bucket(const BucketBits& bb, uint32_t key, int nbits) {
  uint64_t m = bb.valid;
#pragma unroll
  for (int j = 0; j < kMaxBucketBits; ++j)
    if (j < nbits) m &= ((key >> j) & 1u) ? bb.bit[j] : ~bb.bit[j];
  return m;
}

template <typename T>
__global__ __launch_bounds__(kBBBlock) void bb_fill_zero(T* __restrict__ a, int64_t n, uint32_t* __restrict__ b,
                                                        int64_t nb) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * kBBBlock;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kBBBlock) + threadIdx.x; i < n; i += step) a[i] = T(0);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kBBBlock) + threadIdx.x; i < nb; i += step) b[i] = 0u;
}

// Phase 1 (BK:350-456): new_lengths[bucket * L + r] for every row r.  With
// REG (my_size <= 64) lane b of one VGPR counts bucket b of the current row and
// every row stores all its my_size counts; otherwise counts go to new_lengths
// (zero-filled first) with one atomic per (step, bucket).
template <typename IT, typename OT, bool REG>
__global__ __launch_bounds__(kBBBlock) void bb_count(BBParams<IT, OT> p) {
  using UIT = std::make_unsigned_t<IT>;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kBBBlock / kWaveBB);
  const int64_t w0 = blockIdx.x * static_cast<int64_t>(kBBBlock / kWaveBB) + (threadIdx.x >> 6);
  for (int64_t r = w0; r < p.L; r += waves) {
    const RowCtx<IT> c = row_ctx(p, r);
    uint32_t cnt = 0;  // REG: this lane's bucket
    if (c.ok) {
      for (int64_t base = c.s; base < c.e; base += kWaveBB) {
        const int64_t i = base + lane_id();
        int64_t b = 0;
        IT v;
        bool valid = i < c.e && map_index<IT>(c, static_cast<UIT>(p.indices[i]), p.my_size, p.keep, b, v);
        if constexpr (REG) {
          // lane l counts the indices of bucket l
          const BucketBits bb = bucket_bits(valid, static_cast<uint32_t>(b), p.bucket_bits);
          cnt += static_cast<uint32_t>(__builtin_popcountll(lanes_with_bucket(bb, lane_id(), p.bucket_bits)));
          continue;
        }
        uint64_t pending = __builtin_amdgcn_ballot_w64(valid);
        while (pending) {
          const int leader = __builtin_ctzll(pending);
          const int64_t bl = uni(__builtin_amdgcn_readlane(static_cast<int>(b), leader)) & 0xFFFFFFFFll;
          const bool mine = valid && b == bl;
          const uint64_t m = __builtin_amdgcn_ballot_w64(mine);
          const uint32_t k = static_cast<uint32_t>(__builtin_popcountll(m));
          if (lane_id() == leader) add_count(p.new_lengths + bl * p.L + r, k);
          pending &= ~m;
          valid = valid && !mine;
        }
      }
    }
    if constexpr (REG) {
      if (lane_id() < p.my_size) p.new_lengths[lane_id() * p.L + r] = static_cast<OT>(cnt);
    }
  }
}

// Phase 3 (BK:458-606 and 608-762): write every index to its segment, in row
// order.  With REG lane b of one register holds the next write position of
// bucket b of the current row; otherwise the cursors are per-segment counters in
// the workspace, advanced with one atomic per (step, bucket).
template <typename IT, typename OT, bool REG>
__global__ __launch_bounds__(kBBBlock) void bb_scatter(BBParams<IT, OT> p) {
  using UIT = std::make_unsigned_t<IT>;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kBBBlock / kWaveBB);
  const int64_t w0 = blockIdx.x * static_cast<int64_t>(kBBBlock / kWaveBB) + (threadIdx.x >> 6);
  for (int64_t r = w0; r < p.L; r += waves) {
    const RowCtx<IT> c = row_ctx(p, r);
    if (!c.ok) continue;
    int64_t cur = 0;  // REG: write position of this lane's bucket
    if constexpr (REG) {
      if (lane_id() < p.my_size) cur = static_cast<int64_t>(p.new_offsets[lane_id() * p.L + r]);
    }
    for (int64_t base = c.s; base < c.e; base += kWaveBB) {
      const int64_t i = base + lane_id();
      int64_t b = 0;
      IT v = 0;
      const bool valid0 = i < c.e && map_index<IT>(c, static_cast<UIT>(p.indices[i]), p.my_size, p.keep, b, v);
      bool valid = valid0;
      int64_t w = 0;
      uint64_t pending = 0;
      if constexpr (REG) {
        // rank among the lower lanes of the same bucket, after the bucket's cursor
        // (lane b holds it); lane l then advances bucket l's cursor
        const BucketBits bb = bucket_bits(valid0, static_cast<uint32_t>(b), p.bucket_bits);
        const uint64_t mine = lanes_with_bucket(bb, static_cast<uint32_t>(b), p.bucket_bits);
        const int src = static_cast<int>(b & 63) * 4;
        const int64_t seg0 = static_cast<int64_t>(
            (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(cur >> 32)))) << 32) |
            static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(cur & 0xFFFFFFFF))));
        w = seg0 + __builtin_popcountll(mine & lanes_below());
        cur += __builtin_popcountll(lanes_with_bucket(bb, lane_id(), p.bucket_bits));
      } else {
        pending = __builtin_amdgcn_ballot_w64(valid);
      }
      while (pending) {
        const int leader = __builtin_ctzll(pending);
        const int64_t bl = uni(__builtin_amdgcn_readlane(static_cast<int>(b), leader)) & 0xFFFFFFFFll;
        const bool mine = valid && b == bl;
        const uint64_t m = __builtin_amdgcn_ballot_w64(mine);
        const uint32_t k = static_cast<uint32_t>(__builtin_popcountll(m));
        uint32_t old = 0;
        if (lane_id() == leader) old = atomicAdd(p.done + bl * p.L + r, k);
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
  __shared__ T lds[kBBBlock / kWaveBB];
  T carry = 0;
  for (int64_t t0 = 0; t0 < m; t0 += kBBBlock) {
    const int64_t i = t0 + threadIdx.x;
    const T v = i < m ? sums[i] : T(0);
    T total;
    const T ex = block_exclusive_scan(v, lds, total);
    if (i < m) sums[i] = carry + ex;
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

int64_t scan_tiles_of(int64_t n) { return (n + kScanTile - 1) / kScanTile; }

int64_t ws_layout(int64_t my, int64_t L, int32_t os, int64_t* sums_off) {
  // [done: my*L uint32][pad to 256][tile sums: tiles * os]
  const int64_t done_bytes = my * L * 4;
  const int64_t so = (done_bytes + 255) / 256 * 256;
  if (sums_off) *sums_off = so;
  return so + std::max<int64_t>(1, scan_tiles_of(my * L)) * os;
}

template <typename IT, typename OT>
int run(const TbeBlockBucketizeArgs* a, hipStream_t s) {
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
  int64_t sums_off = 0;
  ws_layout(a->my_size, a->lengths_size, a->offset_size, &sums_off);
  p.done = static_cast<uint32_t*>(a->workspace);
  OT* sums = reinterpret_cast<OT*>(static_cast<uint8_t*>(a->workspace) + sums_off);
  p.L = a->lengths_size;
  p.N = a->num_indices;
  p.my_size = a->my_size;
  p.B = a->batch_size_offsets ? 0 : a->lengths_size / a->num_features;
  p.F = a->num_features;
  p.keep = a->keep_orig_idx;
  p.bucket_bits = 0;
  while (p.bucket_bits < kMaxBucketBits && (int64_t(1) << p.bucket_bits) < a->my_size) ++p.bucket_bits;
  const int64_t nseg = a->my_size * a->lengths_size;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const int64_t fill_blocks = std::min<int64_t>(std::max<int64_t>(1, (nseg + kBBBlock - 1) / kBBBlock), 8LL * cus);
  const int64_t row_blocks = std::min<int64_t>(std::max<int64_t>(1, (p.L + 3) / 4), 16LL * cus);
  const int64_t tiles = std::max<int64_t>(1, scan_tiles_of(nseg));
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
  hipLaunchKernelGGL(scan_sums_exclusive<OT>, dim3(1), dim3(kBBBlock), 0, s, sums, tiles);
  hipLaunchKernelGGL(scan_tiles<OT>, dim3(static_cast<uint32_t>(tiles)), dim3(kBBBlock), 0, s,
                     const_cast<const OT*>(p.new_lengths), nseg, const_cast<const OT*>(sums),
                     static_cast<OT*>(a->new_offsets));
  if (p.N > 0) {
    if (reg)
      hipLaunchKernelGGL((bb_scatter<IT, OT, true>), dim3(static_cast<uint32_t>(row_blocks)), dim3(kBBBlock), 0, s, p);
    else
      hipLaunchKernelGGL((bb_scatter<IT, OT, false>), dim3(static_cast<uint32_t>(row_blocks)), dim3(kBBBlock), 0, s, p);
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

extern "C" int tbe_block_bucketize_sparse_features(const TbeBlockBucketizeArgs* a, void* hip_stream) {
  clear_error();
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
  const int64_t need = ws_layout(a->my_size, a->lengths_size, a->offset_size, nullptr);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(TBE_ERR_INVALID_ARG, "workspace of %lld bytes needed", static_cast<long long>(need));
  if (!a->new_lengths || !a->new_offsets || (a->lengths_size > 0 && (!a->offsets || !a->block_sizes)) ||
      (a->num_indices > 0 && (!a->indices || !a->new_indices)))
    return fail(TBE_ERR_INVALID_ARG, "null pointer argument");
  hipStream_t s = static_cast<hipStream_t>(hip_stream);
  if (a->index_size == 4)
    return a->offset_size == 4 ? run<int32_t, int32_t>(a, s) : run<int32_t, int64_t>(a, s);
  return a->offset_size == 4 ? run<int64_t, int32_t>(a, s) : run<int64_t, int64_t>(a, s);
}
