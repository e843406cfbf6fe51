// pooled_ops.hip — gfx950 kernels and C ABI of the operators next to the TBE
// inference forward (include/tbe_pooled_ops.h).
//
// Reference (paths relative to the reference repository root):
//   PA = src/pooled_embedding_ops/permute_pooled_embs/permute_pooled_embs.cpp
//   PK = src/pooled_embedding_ops/permute_pooled_embs/v220/op_kernel/permute_pooled_embs_kernel.h
//
// permute_pooled_embs is a strided column copy: HBM-bound, 2 * B * total_D *
// elem_size bytes per call.  One work-group copies one segment (a feature's
// columns) for a block of rows; the segment's source/destination columns come
// from the three device lists, so the host never reads them (the reference
// reads offset_dim_list[T] on the host, PA:82).  Rows of a segment are copied
// with 16-byte vectors when every address of the segment is 16-byte aligned,
// else with 4-byte words, else element by element; consecutive lanes take
// consecutive vectors of a row, so each row is read and written contiguously.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>

#include "tbe_internal.h"
#include "tbe_nbit.h"
#include "tbe_pooled_ops.h"

namespace tbe {
namespace {

constexpr int kPermBlock = 256;
constexpr int kPermRows = 64;  // rows of one segment per work-group

struct PermParams {
  const uint8_t* __restrict__ in;
  uint8_t* __restrict__ out;
  const int64_t* __restrict__ off;
  const int64_t* __restrict__ perm;
  const int64_t* __restrict__ inv;
  int64_t B;
  int64_t total_D;
  int64_t col_bytes;   // bytes of one column of one row (inner * elem_size)
  int32_t es;
  int32_t T;
  int32_t row_blocks;  // ceil(B / kPermRows)
};

// 64-bit value at a wave-uniform address, kept in SGPRs.
__device__ __forceinline__ int64_t uniform_load(const int64_t* p) {
  const uint64_t v = static_cast<uint64_t>(*p);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v & 0xFFFFFFFFu)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// n / d for a block-uniform d >= 1 with one multiply-high (Granlund & Montgomery,
// PLDI 1994), set up once per work-group.
struct UDiv {
  uint32_t mul, shift;
  __device__ explicit UDiv(uint32_t d) {
    uint32_t l = 0;
    while ((uint64_t(1) << l) < d) ++l;
    shift = l;
    mul = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  }
  __device__ uint32_t operator()(uint32_t n) const {
    return static_cast<uint32_t>((static_cast<uint64_t>(__umulhi(n, mul)) + n) >> shift);
  }
};

// Copy (or zero) `nbytes` per row for rows [r0, r1): src/dst are byte offsets of
// the segment in row 0; `VB` is the vector width in bytes.
template <int VB>
__device__ __forceinline__ void copy_rows(const PermParams& p, int64_t r0, int64_t r1, int64_t src, int64_t dst,
                                          int64_t nbytes, bool zero) {
  using V = typename std::conditional<VB == 16, uint4,
            typename std::conditional<VB == 4, uint32_t, uint16_t>::type>::type;
  const int64_t row_bytes = p.total_D * p.col_bytes;
  const uint32_t nv = static_cast<uint32_t>(nbytes / VB);
  if (nv == 0) return;
  const uint32_t items = static_cast<uint32_t>(r1 - r0) * nv;
  const UDiv div(nv);
  for (uint32_t it = threadIdx.x; it < items; it += kPermBlock) {
    const uint32_t r = div(it);
    const uint32_t v = it - r * nv;
    const int64_t row = r0 + r;
    V* o = reinterpret_cast<V*>(p.out + row * row_bytes + dst) + v;
    if (zero) {
      *o = V{};
    } else {
      *o = *(reinterpret_cast<const V*>(p.in + row * row_bytes + src) + v);
    }
  }
}

// PK:173-211 (segment walk) and PK:140-170 (row-blocked column copy).
__global__ __launch_bounds__(kPermBlock) void permute_pooled_kernel(PermParams p) {
  const int seg = static_cast<int>(blockIdx.x / static_cast<uint32_t>(p.row_blocks));
  const int rb = static_cast<int>(blockIdx.x - static_cast<uint32_t>(seg) * static_cast<uint32_t>(p.row_blocks));
  const int64_t r0 = static_cast<int64_t>(rb) * kPermRows;
  const int64_t r1 = std::min<int64_t>(r0 + kPermRows, p.B);
  const int64_t pi = uniform_load(p.perm + seg);
  const int64_t dst = uniform_load(p.inv + seg);
  const int64_t dst_end = uniform_load(p.inv + seg + 1);
  if (dst < 0 || dst_end < dst || dst_end > p.total_D) return;  // nothing we may write
  const int64_t len = dst_end - dst;
  bool zero = pi < 0 || pi >= p.T;
  int64_t src = 0;
  if (!zero) {
    src = uniform_load(p.off + pi);
    zero = src < 0 || src + len > p.total_D;
  }
  const int64_t cb = p.col_bytes;
  const int64_t sb = src * cb, db = dst * cb, nb = len * cb, rowb = p.total_D * cb;
  const uintptr_t base = reinterpret_cast<uintptr_t>(p.in) | reinterpret_cast<uintptr_t>(p.out);
  if (((sb | db | nb | rowb | static_cast<int64_t>(base)) & 15) == 0) {
    copy_rows<16>(p, r0, r1, sb, db, nb, zero);
  } else if (((sb | db | nb | rowb | static_cast<int64_t>(base)) & 3) == 0) {
    copy_rows<4>(p, r0, r1, sb, db, nb, zero);
  } else {
    // 2-byte elements (or, for misaligned fp32 buffers, half-words)
    copy_rows<2>(p, r0, r1, sb, db, nb, zero);
  }
}

}  // namespace
}  // namespace tbe

using namespace tbe;

extern "C" int tbe_permute_pooled_embs(const TbePermutePooledArgs* a, void* hip_stream) {
  clear_error();
  if (!a) return fail(TBE_ERR_INVALID_ARG, "null args");
  if (a->elem_size != 2 && a->elem_size != 4)
    return fail(TBE_ERR_INVALID_ARG, "pooled_embs must be float32, float16, or bfloat16 (elem_size %d)",
                a->elem_size);
  if (a->T <= 0) return fail(TBE_ERR_INVALID_ARG, "permute_list must not be empty");
  if (a->B < 0 || a->total_D < 0 || a->inner < 1) return fail(TBE_ERR_INVALID_ARG, "bad shape");
  if (a->B == 0 || a->total_D == 0) return TBE_OK;
  if (!a->pooled_embs || !a->output || !a->offset_dim_list || !a->permute_list || !a->inv_offset_dim_list)
    return fail(TBE_ERR_INVALID_ARG, "null pointer argument");
  const int64_t row_blocks = (a->B + kPermRows - 1) / kPermRows;
  if (row_blocks * a->T > 0x7FFFFFFF || a->total_D * a->inner * a->elem_size * kPermRows > 0x7FFFFFFF)
    return fail(TBE_ERR_UNSUPPORTED, "permute_pooled_embs shape too large for one launch");
  PermParams p{};
  p.in = static_cast<const uint8_t*>(a->pooled_embs);
  p.out = static_cast<uint8_t*>(a->output);
  p.off = a->offset_dim_list;
  p.perm = a->permute_list;
  p.inv = a->inv_offset_dim_list;
  p.B = a->B;
  p.total_D = a->total_D;
  p.col_bytes = a->inner * a->elem_size;
  p.es = a->elem_size;
  p.T = a->T;
  p.row_blocks = static_cast<int32_t>(row_blocks);
  void* args[] = {&p};
  const hipError_t err =
      hipLaunchKernel(reinterpret_cast<const void*>(permute_pooled_kernel),
                      dim3(static_cast<uint32_t>(row_blocks * a->T)), dim3(kPermBlock), args, 0,
                      static_cast<hipStream_t>(hip_stream));
  if (err != hipSuccess) return fail(TBE_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return TBE_OK;
}
