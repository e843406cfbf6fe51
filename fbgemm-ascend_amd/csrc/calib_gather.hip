// calib_gather.hip — measurement kernel of bench.py --gather-calibration (libtbe_calib.so;
// not part of the operator or of its C ABI).
//
// It moves the memory traffic of one TBE forward without its arithmetic or bag
// structure: every lookup's unpadded row is read (one row per lane, 16-byte loads
// covering the row's bytes, in index order, so the same 128-byte lines are fetched in
// the same order as by the operator), and a buffer the size of the operator's output is
// written, interleaved with the reads as the operator's output stores are (each lookup
// writes its share of the output right after its row).  Its time is the practical floor of the operator on that
// workload: what the memory system takes for the same lines with as many loads in flight
// as the GPU holds.  Rows are read in 16-byte pieces from their start, so row strides must
// be multiples of 16 (row_alignment 16, as in every benchmark configuration), and every
// table's rows must have the same number of pieces (row_bytes), at most 512 bytes.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {


// KC: 16-byte pieces of every row (all KC loads issued unconditionally: loads under
// per-piece predicates were measured to serialise and take 1.3x as long)
template <int KC>
__global__ __launch_bounds__(256) void calib_gather_kernel(const uint8_t* __restrict__ weights,
                                                           const void* __restrict__ indices, int index_size,
                                                           const int64_t* __restrict__ table_first,  // [T + 1]
                                                           const uint4* __restrict__ table_desc,     // [T]
                                                           const int4* __restrict__ chunk,           // [ceil(n/64)]
                                                           int64_t n, uint2* __restrict__ out, int64_t out_units,
                                                           uint32_t* __restrict__ sink) {
  // blocks of one XCD (block i runs on XCD i % 8; the grid is a multiple of 8) take one
  // contiguous eighth of the blocks, as the operator's kernels take their items
  const uint32_t nb = gridDim.x >> 3;
  const int64_t blk = static_cast<int64_t>(blockIdx.x & 7) * nb + (blockIdx.x >> 3);
  const int64_t i = blk * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // the index and its chunk's table record load together: one round trip before the row
  const int64_t row = index_size == 8 ? static_cast<const int64_t*>(indices)[i] : static_cast<const int32_t*>(indices)[i];
  const int4 c = chunk[i >> 6];  // {table at the chunk's first lookup, next table, its first lane, more}
  const int lane = static_cast<int>(i & 63);
  int t = lane < c.z ? c.x : c.y;
  if (c.w && lane >= c.z)  // a third table starts inside this chunk (small tables): walk
    while (table_first[t + 1] <= i) ++t;
  // {table byte base lo, hi, row stride | unpadded row bytes << 16, rows}
  const uint4 d = table_desc[t];
  uint32_t acc = 0;
  if (row >= 0 && row < static_cast<int64_t>(d.w)) {
    const uint8_t* p = weights + ((static_cast<uint64_t>(d.y) << 32) | d.x) + row * (d.z & 0xFFFFu);
    uint4 v[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k)  // every load issued before any is used
      v[k] = *reinterpret_cast<const uint4*>(p + 16 * k);
#pragma unroll
    for (int k = 0; k < KC; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  // the output-sized write, in 8-byte units: the wave's 64 lookups own units
  // [k i0, k (i0 + 64)) with k = out_units / n (an output row per lookup when k is whole:
  // nobag), written by the wave's lanes together, one coalesced store per 64 units; then
  // units n k + i, n k + i + n, ... of the remainder (pooled outputs: about one unit per lookup)
  const int64_t k = out_units / n;
  const int64_t i0 = i & ~int64_t(63);
  for (int64_t j = 0; j < k; ++j) {
    const int64_t u = i0 * k + j * 64 + lane;
    if (u < n * k) out[u] = make_uint2(acc, static_cast<uint32_t>(j));
  }
  for (int64_t u = n * k + i; u < out_units; u += n) out[u] = make_uint2(acc, static_cast<uint32_t>(u));
  if (acc == 0x9E3779B9u) sink[0] = acc;  // keeps the loads
}

}  // namespace

// table_first[T + 1]: first lookup of every table (table_first[T] = n); table_desc[t] =
// {byte base (low, high word), row stride | unpadded row bytes << 16, rows}; chunk[c] for
// lookups [64 c, 64 c + 64): {table of lookup 64 c, the next table, the lane where it
// starts (64: none), 1 if a further table starts inside the chunk}; row_bytes: the unpadded
// row size of every table; out: out_units 8-byte units.
extern "C" int tbe_calib_gather(const void* weights, const void* indices, int index_size, const int64_t* table_first,
                                const void* table_desc, const void* chunk, int32_t row_bytes, int64_t n,
                                void* out, int64_t out_units, void* sink, void* stream) {
  if (n <= 0) return 0;
  if (out_units < 0 || row_bytes <= 0 || row_bytes > 512) return -1;
  const int64_t blocks = 8 * ((n + 2047) / 2048);  // a multiple of 8 covering n lookups
  decltype(&calib_gather_kernel<1>) kern = nullptr;
  switch ((row_bytes + 15) >> 4) {
#define TBE_CALIB_PIECES(C) case C: kern = calib_gather_kernel<C>; break;
    TBE_CALIB_PIECES(1) TBE_CALIB_PIECES(2) TBE_CALIB_PIECES(3) TBE_CALIB_PIECES(4) TBE_CALIB_PIECES(5)
    TBE_CALIB_PIECES(6) TBE_CALIB_PIECES(8) TBE_CALIB_PIECES(9) TBE_CALIB_PIECES(16) TBE_CALIB_PIECES(17)
    TBE_CALIB_PIECES(32)
#undef TBE_CALIB_PIECES
    default: return -1;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(weights), indices, index_size, table_first,
                     static_cast<const uint4*>(table_desc), static_cast<const int4*>(chunk), n,
                     static_cast<uint2*>(out), out_units, static_cast<uint32_t*>(sink));
  return static_cast<int>(hipGetLastError());
}
