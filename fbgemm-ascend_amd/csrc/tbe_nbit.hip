// tbe_nbit.hip — gfx950 kernels and C ABI of the quantized table-batched-
// embedding inference forward (torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function).
//
// Reference (paths relative to the reference repository root):
//   A = src/tbe_inference/int_nbit_split_embedding_codegen_lookup_function/int_nbit_split_embedding_codegen_lookup_function.cpp
//   H = .../c310/op_host/int_nbit_split_embedding_codegen_lookup_function.cpp
//   C = .../c310/op_kernel/common.h
//   P = .../c310/op_kernel/int_nbit_split_embedding_pooling_kernel.h
//   N = .../c310/op_kernel/int_nbit_split_embedding_nobag_kernel.h
//
// Design (MI355X-first, not a port of the AscendC kernels):
//  * The path is an HBM-bound gather-reduce: no MFMA.  A work item is one bag
//    (table t, sample b) and, for rows wider than 256 bytes, one 256-byte column
//    tile of it; one 64-wide wavefront owns one item.  Launching one wave per
//    item lets the hardware dispatcher balance Poisson/Zipf bag lengths; the
//    reference instead splits bags statically by count over cores (P:119-131).
//  * A row's payload is split over G = 2^log2_lanes lanes, one 4-byte word per
//    lane, so one vector load instruction fetches R = 64/G rows; kUnroll such
//    loads are issued before any is consumed to keep many rows in flight.
//  * The bag's indices are staged 64 at a time with one coalesced load and
//    handed to the lanes that gather each row through the LDS crossbar
//    (ds_bpermute), so no lane re-reads an index.
//  * Dequantization is fused: INT rows carry an fp16 scale/bias header; each
//    lane accumulates scale*q per element and the bias once per row (summed
//    into the element at the end), so a code costs one convert and one FMA.
//  * Partial sums of the R row slots are reduced across the wavefront with
//    xor shuffles; slot 0 writes the D-wide output slice with vector stores.
//  * Blocks are renumbered so consecutive bags (which share a table) stay on
//    one XCD: each XCD's private L2 then caches the hot rows of a few tables
//    instead of all of them.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <type_traits>
#include <vector>

#include "tbe_nbit.h"

namespace tbe {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;
constexpr int kUnroll = 8;
constexpr int kNumXcd = 8;

struct Fp8Consts {
  uint32_t shift;      // exponent_bits + 16: body bits -> fp32 exponent/mantissa field (C:126)
  uint32_t mant_bits;  // 7 - exponent_bits
  float mult;          // 2^(127 - bias) (C:131)
  float sub_scale;     // 2^(1 - bias - mant_bits): value of one unit of a subnormal body
};

struct KParams {
  const uint8_t* __restrict__ weights;
  const TbeTableDesc* __restrict__ tables;
  const void* __restrict__ indices;
  const void* __restrict__ offsets;
  const float* __restrict__ psw;
  void* __restrict__ out;
  int64_t out_stride;
  int64_t B;
  int64_t num_items;
  int64_t num_indices;
  int32_t T;
  int32_t col_tiles;
  int32_t xcd_remap;
  int32_t num_blocks;
  int32_t mean;
  Fp8Consts fp8;
};

// ---------------------------------------------------------------- element decode

template <int WT> struct Traits;
template <> struct Traits<TBE_TY_FP32> { static constexpr int kEpd = 1;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_FP16> { static constexpr int kEpd = 2;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_BF16> { static constexpr int kEpd = 2;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_FP8>  { static constexpr int kEpd = 4;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_INT8> { static constexpr int kEpd = 4;  static constexpr bool kHdr = true; };
template <> struct Traits<TBE_TY_INT4> { static constexpr int kEpd = 8;  static constexpr bool kHdr = true; };
template <> struct Traits<TBE_TY_INT2> { static constexpr int kEpd = 16; static constexpr bool kHdr = true; };

__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h16)));
}

// byte k of x as float (the backend selects v_cvt_f32_ubyte{k})
template <int k>
__device__ __forceinline__ float ubyte_f(uint32_t x) {
  return static_cast<float>((x >> (8 * k)) & 0xFFu);
}

__device__ __forceinline__ float fp8_decode(uint32_t code, const Fp8Consts& c) {
  // Same value as C:136-167 (shift the 7 body bits into the fp32 exponent/mantissa
  // field, scale by 2^(127-bias), OR the sign back in).  Subnormal codes are formed
  // as body * 2^(1-bias-m) so no fp32 denormal operand is ever involved.
  const uint32_t body = code & 0x7Fu;
  const float vn = __uint_as_float(body << c.shift) * c.mult;
  const float vs = static_cast<float>(body) * c.sub_scale;
  const float v = (body >> c.mant_bits) ? vn : vs;
  return __uint_as_float(__float_as_uint(v) | ((code & 0x80u) << 24));
}

template <int WT>
__device__ __forceinline__ void decode(uint32_t d, float (&v)[Traits<WT>::kEpd], const Fp8Consts& c) {
  if constexpr (WT == TBE_TY_FP32) {
    v[0] = __uint_as_float(d);
  } else if constexpr (WT == TBE_TY_FP16) {
    v[0] = half_bits_to_float(d & 0xFFFFu);
    v[1] = half_bits_to_float(d >> 16);
  } else if constexpr (WT == TBE_TY_BF16) {
    v[0] = __uint_as_float(d << 16);
    v[1] = __uint_as_float(d & 0xFFFF0000u);
  } else if constexpr (WT == TBE_TY_FP8) {
    v[0] = fp8_decode(d & 0xFFu, c);
    v[1] = fp8_decode((d >> 8) & 0xFFu, c);
    v[2] = fp8_decode((d >> 16) & 0xFFu, c);
    v[3] = fp8_decode(d >> 24, c);
  } else if constexpr (WT == TBE_TY_INT8) {
    v[0] = ubyte_f<0>(d);
    v[1] = ubyte_f<1>(d);
    v[2] = ubyte_f<2>(d);
    v[3] = ubyte_f<3>(d);
  } else if constexpr (WT == TBE_TY_INT4) {
    // byte b holds element 2b in its low nibble and 2b+1 in its high nibble
    const uint32_t lo = d & 0x0F0F0F0Fu;
    const uint32_t hi = (d >> 4) & 0x0F0F0F0Fu;
    v[0] = ubyte_f<0>(lo); v[1] = ubyte_f<0>(hi);
    v[2] = ubyte_f<1>(lo); v[3] = ubyte_f<1>(hi);
    v[4] = ubyte_f<2>(lo); v[5] = ubyte_f<2>(hi);
    v[6] = ubyte_f<3>(lo); v[7] = ubyte_f<3>(hi);
  } else {  // INT2: byte b holds elements 4b..4b+3, bits 1:0 first
    const uint32_t m0 = d & 0x03030303u;
    const uint32_t m1 = (d >> 2) & 0x03030303u;
    const uint32_t m2 = (d >> 4) & 0x03030303u;
    const uint32_t m3 = (d >> 6) & 0x03030303u;
    v[0] = ubyte_f<0>(m0);  v[1] = ubyte_f<0>(m1);  v[2] = ubyte_f<0>(m2);  v[3] = ubyte_f<0>(m3);
    v[4] = ubyte_f<1>(m0);  v[5] = ubyte_f<1>(m1);  v[6] = ubyte_f<1>(m2);  v[7] = ubyte_f<1>(m3);
    v[8] = ubyte_f<2>(m0);  v[9] = ubyte_f<2>(m1);  v[10] = ubyte_f<2>(m2); v[11] = ubyte_f<2>(m3);
    v[12] = ubyte_f<3>(m0); v[13] = ubyte_f<3>(m1); v[14] = ubyte_f<3>(m2); v[15] = ubyte_f<3>(m3);
  }
}

// ---------------------------------------------------------------- output store

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  // round to nearest, ties to even; NaN stays a quiet NaN
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

struct Bf16Out { uint16_t bits; };

template <typename OutT, int E>
__device__ __forceinline__ void store_slice(OutT* dst, const float (&r)[E]) {
  if constexpr (sizeof(OutT) == 4) {
    float* o = reinterpret_cast<float*>(dst);
    const uintptr_t a = reinterpret_cast<uintptr_t>(o);
    if constexpr (E % 4 == 0) {
      if ((a & 15u) == 0) {
#pragma unroll
        for (int i = 0; i < E; i += 4)
          *reinterpret_cast<float4*>(o + i) = make_float4(r[i], r[i + 1], r[i + 2], r[i + 3]);
        return;
      }
    }
    if constexpr (E % 2 == 0) {
      if ((a & 7u) == 0) {
#pragma unroll
        for (int i = 0; i < E; i += 2) *reinterpret_cast<float2*>(o + i) = make_float2(r[i], r[i + 1]);
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < E; ++i) o[i] = r[i];
  } else {
    uint16_t b[E];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if constexpr (std::is_same<OutT, Bf16Out>::value) {
        b[i] = static_cast<uint16_t>(f32_to_bf16_bits(r[i]));
      } else {
        b[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(r[i]));  // RNE
      }
    }
    uint16_t* o = reinterpret_cast<uint16_t*>(dst);
    const uintptr_t a = reinterpret_cast<uintptr_t>(o);
    if constexpr (E % 8 == 0) {
      if ((a & 15u) == 0) {
#pragma unroll
        for (int i = 0; i < E; i += 8) {
          uint4 w;
          w.x = b[i] | (uint32_t(b[i + 1]) << 16);
          w.y = b[i + 2] | (uint32_t(b[i + 3]) << 16);
          w.z = b[i + 4] | (uint32_t(b[i + 5]) << 16);
          w.w = b[i + 6] | (uint32_t(b[i + 7]) << 16);
          *reinterpret_cast<uint4*>(o + i) = w;
        }
        return;
      }
    }
    if constexpr (E % 4 == 0) {
      if ((a & 7u) == 0) {
#pragma unroll
        for (int i = 0; i < E; i += 4) {
          uint2 w;
          w.x = b[i] | (uint32_t(b[i + 1]) << 16);
          w.y = b[i + 2] | (uint32_t(b[i + 3]) << 16);
          *reinterpret_cast<uint2*>(o + i) = w;
        }
        return;
      }
    }
    if constexpr (E % 2 == 0) {
      if ((a & 3u) == 0) {
#pragma unroll
        for (int i = 0; i < E; i += 2)
          *reinterpret_cast<uint32_t*>(o + i) = b[i] | (uint32_t(b[i + 1]) << 16);
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < E; ++i) o[i] = b[i];
  }
}

__device__ __forceinline__ uint32_t load_word(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

// Block renumbering: hardware hands block i to XCD i % 8; give XCD x a contiguous
// run of logical blocks so the bags it pools come from few tables.
__device__ __forceinline__ int remap_block(int bid, int nblk) {
  const int q = nblk / kNumXcd, r = nblk % kNumXcd;
  const int xcd = bid % kNumXcd, local = bid / kNumXcd;
  return (xcd < r) ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// ---------------------------------------------------------------- pooled (SUM / MEAN)

// One wavefront pools one bag [start, start+L) of table `td` over column tile `ct`.
// P:44-85 (bag walk), P:282-315 (pooling), P:346-394 (chunked bag), P:319-342 (cast/store).
template <int WT, typename IndexT, typename OutT, bool WEIGHTED>
__device__ __forceinline__ void pool_bag(const KParams& p, const TbeTableDesc& td, int64_t start,
                                         int L, int ct, int64_t b) {
  constexpr int E = Traits<WT>::kEpd;
  constexpr bool HDR = Traits<WT>::kHdr;
  const int lane = threadIdx.x & (kWave - 1);
  const int lg = td.log2_lanes;
  const int R = kWave >> lg;
  const int slot = lane >> lg;
  const int dw = ct * kWave + (lane & ((1 << lg) - 1));
  const bool col_ok = dw < td.data_dwords;
  const uint8_t* tbase = p.weights + td.weights_offset;
  const uint8_t* lane_base = tbase + td.data_offset + 4 * dw;
  const IndexT* ind = static_cast<const IndexT*>(p.indices) + start;
  const float* psw = WEIGHTED ? p.psw + start : nullptr;
  const int64_t rows = td.num_rows;
  const int stride = td.row_stride;

  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float bacc = 0.f;

  for (int base = 0; base < L; base += kWave) {
    const int n = min(kWave, L - base);
    // stage up to 64 indices (and weights) of the bag: one coalesced load
    int my_row = -1;
    float my_w = 0.f;
    if (lane < n) {
      const int64_t idx = static_cast<int64_t>(ind[base + lane]);
      if (idx >= 0 && idx < rows) my_row = static_cast<int>(idx);
      if constexpr (WEIGHTED) my_w = psw[base + lane];
    }
    for (int r0 = 0; r0 < n; r0 += R * kUnroll) {
      uint32_t d[kUnroll], h[kUnroll];
      float w[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        d[u] = 0u;
        h[u] = 0u;
        w[u] = 0.f;
        if (r0 + u * R < n) {  // wave-uniform
          const int i = r0 + u * R + slot;
          const int row = __shfl(my_row, i & (kWave - 1));
          float wi = 1.f;
          if constexpr (WEIGHTED) wi = __shfl(my_w, i & (kWave - 1));
          if (i < n && row >= 0) {
            const int64_t roff = static_cast<int64_t>(row) * stride;
            if (col_ok) d[u] = load_word(lane_base + roff);
            if constexpr (HDR) h[u] = load_word(tbase + roff);
            w[u] = wi;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        if (r0 + u * R < n) {
          float v[E];
          decode<WT>(d[u], v, p.fp8);
          if constexpr (HDR) {
            float s = half_bits_to_float(h[u] & 0xFFFFu);
            float bi = half_bits_to_float(h[u] >> 16);
            if constexpr (WEIGHTED) {
              s *= w[u];
              bi *= w[u];
            }
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] = fmaf(v[e], s, acc[e]);
            bacc += bi;
          } else if constexpr (WEIGHTED) {
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] = fmaf(v[e], w[u], acc[e]);
          } else {
#pragma unroll
            for (int e = 0; e < E; ++e) acc[e] += v[e];
          }
        }
      }
    }
  }

  // reduce the R row slots (lanes that differ in bits lg..5)
  for (int off = kWave >> 1; off >= (1 << lg); off >>= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] += __shfl_xor(acc[e], off);
    if constexpr (HDR) bacc += __shfl_xor(bacc, off);
  }

  if (slot == 0 && col_ok) {
    const float scale = (p.mean && L > 0) ? 1.0f / static_cast<float>(L) : 1.0f;  // P:355
    float r[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float x = HDR ? acc[e] + bacc : acc[e];
      r[e] = p.mean ? x * scale : x;
    }
    OutT* o = static_cast<OutT*>(p.out) + b * p.out_stride + td.D_offset + static_cast<int64_t>(dw) * E;
    store_slice<OutT, E>(o, r);
  }
}

template <typename IndexT, typename OutT, bool WEIGHTED>
__global__ __launch_bounds__(kBlock) void pooled_kernel(KParams p) {
  int blk = blockIdx.x;
  if (p.xcd_remap) blk = remap_block(blk, p.num_blocks);
  const int wv = uniform(threadIdx.x >> 6);
  const int64_t item = static_cast<int64_t>(blk) * kWavesPerBlock + wv;
  if (item >= p.num_items) return;
  const int64_t k = item / p.col_tiles;
  const int ct = static_cast<int>(item - k * p.col_tiles);
  const int t = static_cast<int>(k / p.B);
  const int64_t b = k - static_cast<int64_t>(t) * p.B;
  const TbeTableDesc td = p.tables[t];
  if (ct >= td.col_tiles) return;
  const IndexT* offs = static_cast<const IndexT*>(p.offsets);
  // clamp to the index array so malformed offsets can never read out of bounds
  const int64_t start = min(max(static_cast<int64_t>(offs[k]), int64_t(0)), p.num_indices);
  const int64_t end = min(max(static_cast<int64_t>(offs[k + 1]), start), p.num_indices);
  const int L = static_cast<int>(end - start);
  switch (td.weight_ty) {
    case TBE_TY_INT4: pool_bag<TBE_TY_INT4, IndexT, OutT, WEIGHTED>(p, td, start, L, ct, b); break;
    case TBE_TY_INT8: pool_bag<TBE_TY_INT8, IndexT, OutT, WEIGHTED>(p, td, start, L, ct, b); break;
    case TBE_TY_INT2: pool_bag<TBE_TY_INT2, IndexT, OutT, WEIGHTED>(p, td, start, L, ct, b); break;
    case TBE_TY_FP8:  pool_bag<TBE_TY_FP8,  IndexT, OutT, WEIGHTED>(p, td, start, L, ct, b); break;
    case TBE_TY_FP16: pool_bag<TBE_TY_FP16, IndexT, OutT, WEIGHTED>(p, td, start, L, ct, b); break;
    case TBE_TY_BF16: pool_bag<TBE_TY_BF16, IndexT, OutT, WEIGHTED>(p, td, start, L, ct, b); break;
    case TBE_TY_FP32: pool_bag<TBE_TY_FP32, IndexT, OutT, WEIGHTED>(p, td, start, L, ct, b); break;
    default: break;  // rejected by the planner
  }
}

// ---------------------------------------------------------------- nobag (pooling_mode NONE)

// Rows [i0, i1) of the global index array, all belonging to table td: output row i
// is the dequantized row of indices[i] (N:224-300).
template <int WT, typename IndexT, typename OutT>
__device__ __forceinline__ void nobag_rows(const KParams& p, const TbeTableDesc& td, int64_t i0,
                                           int64_t i1) {
  constexpr int E = Traits<WT>::kEpd;
  constexpr bool HDR = Traits<WT>::kHdr;
  const int lane = threadIdx.x & (kWave - 1);
  const int lg = td.log2_lanes;
  const int R = kWave >> lg;
  const int slot = lane >> lg;
  const uint8_t* tbase = p.weights + td.weights_offset;
  const IndexT* ind = static_cast<const IndexT*>(p.indices);
  for (int ct = 0; ct < td.col_tiles; ++ct) {
    const int dw = ct * kWave + (lane & ((1 << lg) - 1));
    const bool col_ok = dw < td.data_dwords;
    for (int64_t r0 = i0; r0 < i1; r0 += R) {
      const int64_t i = r0 + slot;
      if (i >= i1 || !col_ok) continue;
      const int64_t idx = static_cast<int64_t>(ind[i]);
      float v[E];
      float s = 1.f, bi = 0.f;
      if (idx >= 0 && idx < td.num_rows) {
        const uint8_t* row = tbase + idx * td.row_stride;
        decode<WT>(load_word(row + td.data_offset + 4 * dw), v, p.fp8);
        if constexpr (HDR) {
          const uint32_t h = load_word(row);
          s = half_bits_to_float(h & 0xFFFFu);
          bi = half_bits_to_float(h >> 16);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = 0.f;
        s = 0.f;
      }
      float r[E];
#pragma unroll
      for (int e = 0; e < E; ++e) r[e] = HDR ? fmaf(v[e], s, bi) : v[e];
      OutT* o = static_cast<OutT*>(p.out) + i * p.out_stride + static_cast<int64_t>(dw) * E;
      store_slice<OutT, E>(o, r);
    }
  }
}

template <typename IndexT>
__device__ __forceinline__ int64_t table_begin(const KParams& p, int t) {
  return static_cast<int64_t>(static_cast<const IndexT*>(p.offsets)[static_cast<int64_t>(t) * p.B]);
}

template <typename IndexT, typename OutT>
__global__ __launch_bounds__(kBlock) void nobag_kernel(KParams p) {
  const int wv = uniform(threadIdx.x >> 6);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wv;
  if (item >= p.num_items) return;
  const int64_t i0 = item * kWave;
  const int64_t i1 = min(i0 + kWave, p.num_indices);
  // last table whose first index is <= i0 (N:57-78 walks tables by offset_per_key)
  int lo = 0, hi = p.T - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (table_begin<IndexT>(p, mid) <= i0) lo = mid; else hi = mid - 1;
  }
  for (int t = lo; t < p.T; ++t) {
    const int64_t tb = table_begin<IndexT>(p, t);
    const int64_t te = table_begin<IndexT>(p, t + 1);
    if (tb >= i1) break;
    const int64_t a = max(tb, i0), e = min(te, i1);
    if (a >= e) continue;
    const TbeTableDesc td = p.tables[t];
    switch (td.weight_ty) {
      case TBE_TY_INT4: nobag_rows<TBE_TY_INT4, IndexT, OutT>(p, td, a, e); break;
      case TBE_TY_INT8: nobag_rows<TBE_TY_INT8, IndexT, OutT>(p, td, a, e); break;
      case TBE_TY_INT2: nobag_rows<TBE_TY_INT2, IndexT, OutT>(p, td, a, e); break;
      case TBE_TY_FP8:  nobag_rows<TBE_TY_FP8,  IndexT, OutT>(p, td, a, e); break;
      case TBE_TY_FP16: nobag_rows<TBE_TY_FP16, IndexT, OutT>(p, td, a, e); break;
      case TBE_TY_BF16: nobag_rows<TBE_TY_BF16, IndexT, OutT>(p, td, a, e); break;
      case TBE_TY_FP32: nobag_rows<TBE_TY_FP32, IndexT, OutT>(p, td, a, e); break;
      default: break;
    }
  }
}

// ---------------------------------------------------------------- host side

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int bits_of(int ty) {
  switch (ty) {
    case TBE_TY_FP32: return 32;
    case TBE_TY_FP16: case TBE_TY_BF16: return 16;
    case TBE_TY_INT8: case TBE_TY_FP8: return 8;
    case TBE_TY_INT4: return 4;
    case TBE_TY_INT2: return 2;
    default: return 0;
  }
}

Fp8Consts make_fp8(int bits, int bias) {
  Fp8Consts c{};
  if (bits < 1 || bits > 7 || bias < 0 || bias > 120) return c;
  c.shift = static_cast<uint32_t>(bits + 16);
  c.mant_bits = static_cast<uint32_t>(7 - bits);
  const uint32_t mult_bits = static_cast<uint32_t>(254 - bias) << 23;
  memcpy(&c.mult, &mult_bits, 4);
  c.sub_scale = ldexpf(1.0f, 1 - bias - (7 - bits));
  return c;
}

template <typename IndexT, typename OutT>
hipError_t launch_pooled(const KParams& p, bool weighted, hipStream_t s) {
  if (weighted)
    hipLaunchKernelGGL((pooled_kernel<IndexT, OutT, true>), dim3(p.num_blocks), dim3(kBlock), 0, s, p);
  else
    hipLaunchKernelGGL((pooled_kernel<IndexT, OutT, false>), dim3(p.num_blocks), dim3(kBlock), 0, s, p);
  return hipGetLastError();
}

template <typename IndexT>
hipError_t launch_pooled_out(const KParams& p, int out_ty, bool weighted, hipStream_t s) {
  switch (out_ty) {
    case TBE_TY_FP32: return launch_pooled<IndexT, float>(p, weighted, s);
    case TBE_TY_FP16: return launch_pooled<IndexT, _Float16>(p, weighted, s);
    default: return launch_pooled<IndexT, Bf16Out>(p, weighted, s);
  }
}

template <typename IndexT>
hipError_t launch_nobag_out(const KParams& p, int out_ty, hipStream_t s) {
  switch (out_ty) {
    case TBE_TY_FP32:
      hipLaunchKernelGGL((nobag_kernel<IndexT, float>), dim3(p.num_blocks), dim3(kBlock), 0, s, p);
      break;
    case TBE_TY_FP16:
      hipLaunchKernelGGL((nobag_kernel<IndexT, _Float16>), dim3(p.num_blocks), dim3(kBlock), 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((nobag_kernel<IndexT, Bf16Out>), dim3(p.num_blocks), dim3(kBlock), 0, s, p);
      break;
  }
  return hipGetLastError();
}

}  // namespace tbe

using namespace tbe;

extern "C" {

const char* tbe_last_error(void) { return g_last_error.c_str(); }

int tbe_nbit_abi_version(void) { return TBE_NBIT_ABI_VERSION; }

int tbe_nbit_plan(const TbePlanInput* in, TbeTableDesc* descs, TbePlanSummary* summary) {
  g_last_error.clear();
  if (!in || !descs || !summary) return fail(TBE_ERR_INVALID_ARG, "null argument to tbe_nbit_plan");
  const int T = in->T;
  // A:116, H:120-123
  if (T <= 0) return fail(TBE_ERR_INVALID_ARG, "weights_offsets size must be greater than 0 (got T=%d)", T);
  if (!in->weights_offsets || !in->weights_tys || !in->D_offsets)
    return fail(TBE_ERR_INVALID_ARG, "null table metadata");
  if (in->row_alignment <= 0 || in->row_alignment % 4 != 0)
    return fail(TBE_ERR_UNSUPPORTED, "row_alignment must be a positive multiple of 4 (got %d)",
                in->row_alignment);
  if (in->dev_weights_bytes < 0) return fail(TBE_ERR_INVALID_ARG, "negative dev_weights size");
  TbePlanSummary s{};
  s.max_col_tiles = 1;
  s.uniform_D = 1;
  s.covers_output = in->D_offsets[0] == 0;
  s.total_D = in->D_offsets[T];
  int has_fp8 = 0;
  for (int t = 0; t < T; ++t) {
    const int ty = in->weights_tys[t];
    const int bits = bits_of(ty);
    if (bits == 0) return fail(TBE_ERR_UNSUPPORTED, "table %d: unsupported weight type %d", t, ty);
    const int64_t D = static_cast<int64_t>(in->D_offsets[t + 1]) - in->D_offsets[t];
    if (D < 0) return fail(TBE_ERR_INVALID_ARG, "D_offsets must be non-decreasing (table %d)", t);
    if ((D * bits) % 32 != 0)
      return fail(TBE_ERR_UNSUPPORTED,
                  "table %d: D=%lld of weight type %d does not fill whole 4-byte words (D*bits %% 32 != 0)",
                  t, static_cast<long long>(D), ty);
    const int64_t wo = in->weights_offsets[t];
    if (wo < 0 || wo > in->dev_weights_bytes)
      return fail(TBE_ERR_INVALID_ARG, "table %d: weights_offset %lld outside dev_weights (%lld bytes)", t,
                  static_cast<long long>(wo), static_cast<long long>(in->dev_weights_bytes));
    if (wo % 4 != 0) return fail(TBE_ERR_UNSUPPORTED, "table %d: weights_offset not 4-byte aligned", t);
    const int hdr = (ty == TBE_TY_INT8 || ty == TBE_TY_INT4 || ty == TBE_TY_INT2) ? 4 : 0;
    const int64_t payload = D * bits / 8;
    const int64_t stride = (payload + hdr + in->row_alignment - 1) / in->row_alignment * in->row_alignment;
    const int64_t dwords = D * bits / 32;
    int lg = 0;
    while ((1LL << lg) < std::min<int64_t>(dwords, kWave)) ++lg;
    const int64_t tiles = std::max<int64_t>(1, (dwords + kWave - 1) / kWave);
    if (tiles > 255 || stride > (1LL << 30))
      return fail(TBE_ERR_UNSUPPORTED, "table %d: row too wide (D=%lld)", t, static_cast<long long>(D));
    TbeTableDesc& d = descs[t];
    memset(&d, 0, sizeof(d));
    d.weights_offset = wo;
    d.D = static_cast<int32_t>(D);
    d.D_offset = in->D_offsets[t];
    d.row_stride = static_cast<int32_t>(stride);
    d.data_offset = hdr;
    d.data_dwords = static_cast<int32_t>(dwords);
    d.weight_ty = static_cast<uint8_t>(ty);
    d.log2_lanes = static_cast<uint8_t>(lg);
    d.col_tiles = static_cast<uint8_t>(tiles);
    s.max_col_tiles = std::max<int32_t>(s.max_col_tiles, static_cast<int32_t>(tiles));
    s.max_D = std::max<int32_t>(s.max_D, static_cast<int32_t>(D));
    if (t > 0 && D != descs[0].D) s.uniform_D = 0;
    if (ty == TBE_TY_FP8) has_fp8 = 1;
  }
  // rows addressable by each table: up to the next table's first byte (or the end)
  std::vector<int64_t> starts(in->weights_offsets, in->weights_offsets + T);
  std::sort(starts.begin(), starts.end());
  starts.erase(std::unique(starts.begin(), starts.end()), starts.end());
  for (int t = 0; t < T; ++t) {
    auto it = std::upper_bound(starts.begin(), starts.end(), descs[t].weights_offset);
    const int64_t end = it == starts.end() ? in->dev_weights_bytes : *it;
    descs[t].num_rows = (end - descs[t].weights_offset) / descs[t].row_stride;
  }
  if (has_fp8) {
    const int eb = in->fp8_exponent_bits, bias = in->fp8_exponent_bias;
    if (eb < 1 || eb > 7 || bias < 0 || bias > 120)
      return fail(TBE_ERR_INVALID_ARG, "FP8 tables need fp8_exponent_bits in [1,7] and bias in [0,120] (got %d, %d)",
                  eb, bias);
  }
  s.has_fp8 = has_fp8;
  *summary = s;
  return TBE_OK;
}

int tbe_nbit_forward(const TbeNbitArgs* a, void* hip_stream) {
  g_last_error.clear();
  if (!a) return fail(TBE_ERR_INVALID_ARG, "null args");
  if (a->T <= 0) return fail(TBE_ERR_INVALID_ARG, "T must be positive");
  if (a->B < 0) return fail(TBE_ERR_INVALID_ARG, "B must be non-negative");
  if (a->index_size != 4 && a->index_size != 8)
    return fail(TBE_ERR_INVALID_ARG, "indices/offsets must be int32 or int64 (H:170-173)");
  if (a->pooling_mode < TBE_POOL_SUM || a->pooling_mode > TBE_POOL_NONE)
    return fail(TBE_ERR_INVALID_ARG, "invalid pooling mode %d: supported SUM(0), MEAN(1), NONE(2)",
                a->pooling_mode);
  if (a->output_dtype == TBE_TY_INT8)
    return fail(TBE_ERR_UNSUPPORTED, "INT8 output is not supported (the reference kernel asserts on it)");
  if (a->output_dtype != TBE_TY_FP32 && a->output_dtype != TBE_TY_FP16 && a->output_dtype != TBE_TY_BF16)
    return fail(TBE_ERR_INVALID_ARG, "unsupported output_dtype %d: supported 0(FP32), 1(FP16), 5(BF16)",
                a->output_dtype);
  if (a->max_col_tiles < 1 || a->max_col_tiles > 255) return fail(TBE_ERR_INVALID_ARG, "bad max_col_tiles");
  if (a->num_indices < 0) return fail(TBE_ERR_INVALID_ARG, "negative num_indices");
  KParams p{};
  p.weights = a->dev_weights;
  p.tables = a->tables;
  p.indices = a->indices;
  p.offsets = a->offsets;
  p.psw = a->indice_weights;
  p.out = a->output;
  p.out_stride = a->output_stride;
  p.B = a->B;
  p.num_indices = a->num_indices;
  p.T = a->T;
  p.col_tiles = a->max_col_tiles;
  p.xcd_remap = (a->flags & TBE_FLAG_NO_XCD_REMAP) ? 0 : 1;
  p.mean = a->pooling_mode == TBE_POOL_MEAN;
  p.fp8 = make_fp8(a->fp8_exponent_bits, a->fp8_exponent_bias);
  hipStream_t s = static_cast<hipStream_t>(hip_stream);
  hipError_t err;
  if (a->pooling_mode == TBE_POOL_NONE) {
    p.num_items = (a->num_indices + kWave - 1) / kWave;
    if (p.num_items == 0) return TBE_OK;
    const int64_t blocks = (p.num_items + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 0x7FFFFFFF) return fail(TBE_ERR_UNSUPPORTED, "too many indices for one launch");
    if (!a->dev_weights || !a->tables || !a->indices || !a->offsets || !a->output)
      return fail(TBE_ERR_INVALID_ARG, "null device pointer");
    p.num_blocks = static_cast<int32_t>(blocks);
    err = a->index_size == 8 ? launch_nobag_out<int64_t>(p, a->output_dtype, s)
                             : launch_nobag_out<int32_t>(p, a->output_dtype, s);
  } else {
    p.num_items = static_cast<int64_t>(a->T) * a->B * a->max_col_tiles;
    if (p.num_items == 0) return TBE_OK;
    const int64_t blocks = (p.num_items + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 0x7FFFFFFF) return fail(TBE_ERR_UNSUPPORTED, "too many bags for one launch");
    if (!a->dev_weights || !a->tables || !a->offsets || !a->output)
      return fail(TBE_ERR_INVALID_ARG, "null device pointer");
    if (a->num_indices > 0 && !a->indices) return fail(TBE_ERR_INVALID_ARG, "null indices");
    p.num_blocks = static_cast<int32_t>(blocks);
    const bool weighted = a->indice_weights != nullptr;
    err = a->index_size == 8 ? launch_pooled_out<int64_t>(p, a->output_dtype, weighted, s)
                             : launch_pooled_out<int32_t>(p, a->output_dtype, weighted, s);
  }
  if (err != hipSuccess) return fail(TBE_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  return TBE_OK;
}

}  // extern "C"
