// tbe_kernels.h — device code of the quantized table-batched-embedding inference
// forward, shared by the per-weight-type translation units (tbe_kern_*.hip) that
// instantiate its kernels and by tbe_nbit.hip (host side, nobag and 64-bit kernels).
// The operator is torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function.
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
//    tile of it; one 64-wide wavefront pools one item at a time.
//  * The host planner groups tables by (weight type, lanes per row).  Each group
//    launches a kernel compiled for exactly that shape, so the register budget
//    (and with it the number of resident waves) is that of one row format, not
//    of the worst one.  Kernels are persistent: the grid holds what the GPU keeps
//    resident and each wave walks items.
//  * Items of a group are split into one contiguous range per XCD (the hardware
//    places block i on XCD i % 8); the waves of an XCD interleave over its range.
//    Bags of one table are adjacent, so each XCD's L2 caches the hot rows of
//    about 1/8 of the tables instead of all of them.
//  * A row's payload is split over G = 2^LG lanes, one 4-byte word per lane, so
//    one load instruction fetches R = 64/G rows.  The bag's indices are staged 64
//    at a time with one coalesced load, each lane turns its index into a byte
//    offset, and the lanes that gather a row fetch that offset through the LDS
//    crossbar (ds_bpermute).  All row loads of a step are issued before any is
//    consumed; rows are read with buffer loads at 32-bit offsets from the table
//    base, and slots past the bag or rejected indices use an offset that fails
//    the buffer range check, which returns zero.  The load phase is therefore
//    straight-line code.
//  * Dequantization is fused: an INT code q is fed to v_fma_mix_f32 as the fp16
//    subnormal q*2^-24 (the code bits are the operand, no convert), multiplied by
//    the row's fp16 scale, accumulated in fp32; the bias is summed once per row.
//    Scaling by 2^24 at the end is exact, so the result is the plain fp32 sum.
//  * Partial sums of the R row slots are reduced with v_permlane32_swap /
//    v_permlane16_swap and DPP row rotations; slot 0 writes the output slice.
#ifndef TBE_KERNELS_H
#define TBE_KERNELS_H

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "tbe_internal.h"
#include "tbe_nbit.h"
namespace tbe {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;
constexpr int kNumXcd = 8;
constexpr int kUnrollWide = 8;

// Word 3 of a raw buffer resource on gfx9-family parts (32-bit data format, no swizzle).
constexpr int kRsrcWord3 = 0x00020000;
// Offset that fails the buffer range check, so the load returns zero (rows past
// the bag, rejected indices).  32-bit tables span at most kNoRow bytes, and a
// lane's column offset stays below 64 KiB, so kNoRow + column never wraps.
constexpr uint32_t kNoRow = 0xFFFE0000u;

// Unsigned division by a runtime-invariant divisor with one multiply-high
// (Granlund & Montgomery, PLDI 1994): q = (mulhi(n, mul) + n) >> shift,
// exact for n < 2^31.
struct FastDiv {
  uint32_t d, mul, shift;
};

struct Fp8Consts {
  uint32_t shift;      // exponent_bits + 16: body bits -> fp32 exponent/mantissa field (C:126)
  uint32_t mant_bits;  // 7 - exponent_bits
  float mult;          // 2^(127 - bias) (C:131)
  float sub_scale;     // 2^(1 - bias - mant_bits): value of one unit of a subnormal body
  uint32_t h16_shift;  // exponent_bits + 3: body bits -> fp16 exponent/mantissa field
  float h16_scale;     // 2^(15 - bias): fp16 reading of the placed body -> code value
  int32_t h16_ok;      // exponent_bits <= 4: every body fits a finite fp16
  float one;           // 1.0f (see accum_row)
};

struct KParams {
  const uint8_t* __restrict__ weights;
  const TbeTableDesc* __restrict__ tables;
  const int32_t* __restrict__ order;  // group's table ids: order[group_first + i]
  const void* __restrict__ indices;
  const void* __restrict__ offsets;
  const float* __restrict__ psw;
  void* __restrict__ out;
  int64_t out_stride;
  int64_t num_indices;
  int32_t B;
  int32_t T;
  int32_t group_first;
  int32_t group_count;
  int32_t col_tiles;    // of the group
  int32_t num_items;    // group_count * B * col_tiles (bag modes), index chunks (nobag)
  int32_t index64;
  int32_t out_ty;
  int32_t mean;
  int32_t xcd;            // bit 0: XCD-aware item split; bit 1: progress-ordered wave priority
  int32_t ranges;         // bag ranges per table (stream kernel)
  int32_t bags_per_wave;  // bags of one range
  int32_t zero_gaps;      // nobag: this launch zeroes output rows outside every table's segment
  FastDiv div_B;
  FastDiv div_tiles;
  FastDiv div_ranges;
  Fp8Consts fp8;
};

// ---------------------------------------------------------------- small helpers

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
  const uint64_t hi = (static_cast<uint64_t>(n) * f.mul) >> 32;
  return static_cast<uint32_t>((hi + n) >> f.shift);
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Generic pointer -> constant address space, so loads at wave-uniform addresses
// become scalar loads (device pass only; the host pass of hipcc parses device
// functions but never emits them).
#if defined(__HIP_DEVICE_COMPILE__)
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* as_constant(const T* p) {
  return (const __attribute__((address_space(4))) T*)(p);
}
#else
template <typename T>
__device__ __forceinline__ const T* as_constant(const T* p) { return p; }
#endif

template <typename T>
__device__ __forceinline__ T load_uniform(const T* ptr) {
  return *as_constant(ptr);
}

struct DescWords {
  uint32_t w[sizeof(TbeTableDesc) / 4];
};
static_assert(sizeof(TbeTableDesc) == 40, "TbeTableDesc layout");

// Table descriptor at a wave-uniform address, read as dwords and kept in SGPRs.
__device__ __forceinline__ TbeTableDesc load_desc(const TbeTableDesc* ptr) {
  DescWords x = *as_constant(reinterpret_cast<const DescWords*>(ptr));
#pragma unroll
  for (int i = 0; i < static_cast<int>(sizeof(TbeTableDesc) / 4); ++i)
    x.w[i] = static_cast<uint32_t>(uniform(static_cast<int>(x.w[i])));
  TbeTableDesc d;
  d.weights_offset = static_cast<int64_t>(x.w[0] | (static_cast<uint64_t>(x.w[1]) << 32));
  d.num_rows = static_cast<int64_t>(x.w[2] | (static_cast<uint64_t>(x.w[3]) << 32));
  d.D = static_cast<int32_t>(x.w[4]);
  d.D_offset = static_cast<int32_t>(x.w[5]);
  d.row_stride = static_cast<int32_t>(x.w[6]);
  d.data_offset = static_cast<int32_t>(x.w[7]);
  d.data_dwords = static_cast<int32_t>(x.w[8]);
  d.weight_ty = static_cast<uint8_t>(x.w[9]);
  d.log2_lanes = static_cast<uint8_t>(x.w[9] >> 8);
  d.col_tiles = static_cast<uint8_t>(x.w[9] >> 16);
  d.flags = static_cast<uint8_t>(x.w[9] >> 24);
  return d;
}

// Entry i of the indices / offsets array (int32 or int64), any address.
__device__ __forceinline__ int64_t load_index(const KParams& p, const void* base, int64_t i) {
  return p.index64 ? static_cast<const int64_t*>(base)[i]
                   : static_cast<int64_t>(static_cast<const int32_t*>(base)[i]);
}

// Entry i of the offsets array at a wave-uniform position (scalar load).
__device__ __forceinline__ int64_t load_offset(const KParams& p, int64_t i) {
  return p.index64 ? load_uniform(static_cast<const int64_t*>(p.offsets) + i)
                   : static_cast<int64_t>(load_uniform(static_cast<const int32_t*>(p.offsets) + i));
}

// A word of device memory through a global (not flat) load: flat loads also count
// as LDS operations, so every ds_bpermute wait would wait for them too.
__device__ __forceinline__ uint32_t load_word(const uint8_t* p) {
  using GlobalWord = const __attribute__((address_space(1))) uint32_t;
  return *(GlobalWord*)(p);
}

// ---------------------------------------------------------------- element decode

template <int WT> struct Traits;
template <> struct Traits<TBE_TY_FP32> { static constexpr int kEpd = 1;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_FP16> { static constexpr int kEpd = 2;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_BF16> { static constexpr int kEpd = 2;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_FP8>  { static constexpr int kEpd = 4;  static constexpr bool kHdr = false; };
template <> struct Traits<TBE_TY_INT8> { static constexpr int kEpd = 4;  static constexpr bool kHdr = true; };
template <> struct Traits<TBE_TY_INT4> { static constexpr int kEpd = 8;  static constexpr bool kHdr = true; };
template <> struct Traits<TBE_TY_INT2> { static constexpr int kEpd = 16; static constexpr bool kHdr = true; };

// Halves of a word read as fp16 (the backend folds these into v_fma_mix_f32 operands).
__device__ __forceinline__ float h16lo(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x & 0xFFFFu)));
}
__device__ __forceinline__ float h16hi(uint32_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x >> 16)));
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

// Exact element values of one payload word (scale/bias not applied).
template <int WT>
__device__ __forceinline__ void decode(uint32_t d, float (&v)[Traits<WT>::kEpd], const Fp8Consts& c) {
  if constexpr (WT == TBE_TY_FP32) {
    v[0] = __uint_as_float(d);
  } else if constexpr (WT == TBE_TY_FP16) {
    v[0] = h16lo(d);
    v[1] = h16hi(d);
  } else if constexpr (WT == TBE_TY_BF16) {
    v[0] = __uint_as_float(d << 16);
    v[1] = __uint_as_float(d & 0xFFFF0000u);
  } else if constexpr (WT == TBE_TY_FP8) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = fp8_decode((d >> (8 * e)) & 0xFFu, c);
  } else {
    // INT8/INT4/INT2: element e sits at bits [e*bits, (e+1)*bits), low bits first
    constexpr int bits = 32 / Traits<WT>::kEpd;
#pragma unroll
    for (int e = 0; e < Traits<WT>::kEpd; ++e) v[e] = static_cast<float>((d >> (bits * e)) & ((1u << bits) - 1));
  }
}

// ---------------------------------------------------------------- fused dequant + accumulate

// Factor applied to the element accumulators after the last row.  INT codes q are
// accumulated as the fp16 subnormal q * 2^-24 (the code itself is the bit pattern,
// so no conversion instruction is needed and every product is exact in fp32);
// scaling by a power of two commutes with rounding, so the result equals the
// plain fp32 sum of scale*q.
//
// INT4 words are split with two masks per byte pair (no shift for the odd
// nibbles), so odd elements arrive as (16q) * 2^-24 and take 2^20 instead.
template <int WT>
__device__ __forceinline__ float acc_post_scale(int e) {
  if constexpr (WT == TBE_TY_INT4) return (e & 1) ? 1048576.0f : 16777216.0f;
  if constexpr (WT == TBE_TY_INT2) {
    // field j of a half-word reads as 4^j' x 2^-24 (j' = j for j < 5, j - 5 after the 10-bit shift)
    const int j = e & 7;
    const int jp = j < 5 ? j : j - 5;
    return __int_as_float((127 + 24 - 2 * jp) << 23);
  }
  return WT == TBE_TY_INT8 ? 16777216.0f : 1.0f;
}

// Add one row's contribution: acc[e] += w * value[e] (value = scale*q + bias for INT
// rows: the scale part goes to acc, the bias to bacc once per row).
// `d` is the lane's payload word, `h` the row's header word (INT rows).
template <int WT, bool WEIGHTED>
__device__ __forceinline__ void accum_row(float (&acc)[Traits<WT>::kEpd], float& bacc, uint32_t d,
                                          uint32_t h, float w, const Fp8Consts& c) {
  constexpr int E = Traits<WT>::kEpd;
  if constexpr (Traits<WT>::kHdr) {
    float s = h16lo(h);
    if constexpr (WEIGHTED) {
      s *= w;
      bacc = fmaf(h16hi(h), w, bacc);
    } else {
      // c.one is 1.0f; as an opaque operand it keeps this a single v_fma_mix_f32
      // reading the bias half of the header in place (no separate convert)
      bacc = fmaf(h16hi(h), c.one, bacc);
    }
    if constexpr (WT == TBE_TY_INT8) {
      // halves of p0 hold bytes 0 and 2, of p1 bytes 1 and 3
      const uint32_t p0 = d & 0x00FF00FFu, p1 = (d >> 8) & 0x00FF00FFu;
      acc[0] = fmaf(h16lo(p0), s, acc[0]);
      acc[2] = fmaf(h16hi(p0), s, acc[2]);
      acc[1] = fmaf(h16lo(p1), s, acc[1]);
      acc[3] = fmaf(h16hi(p1), s, acc[3]);
    } else if constexpr (WT == TBE_TY_INT4) {
      // nibble n of the word is element n; halves of p0..p3 hold elements (0,4),
      // (1,5) x16, (2,6), (3,7) x16 (see acc_post_scale)
      const uint32_t d8 = d >> 8;
      const uint32_t p0 = d & 0x000F000Fu, p1 = d & 0x00F000F0u, p2 = d8 & 0x000F000Fu, p3 = d8 & 0x00F000F0u;
      acc[0] = fmaf(h16lo(p0), s, acc[0]);
      acc[4] = fmaf(h16hi(p0), s, acc[4]);
      acc[1] = fmaf(h16lo(p1), s, acc[1]);
      acc[5] = fmaf(h16hi(p1), s, acc[5]);
      acc[2] = fmaf(h16lo(p2), s, acc[2]);
      acc[6] = fmaf(h16hi(p2), s, acc[6]);
      acc[3] = fmaf(h16lo(p3), s, acc[3]);
      acc[7] = fmaf(h16hi(p3), s, acc[7]);
    } else {  // INT2: 2-bit fields j and j+8 of the halves are elements j and j+8
      // fields 0-4 are masked in place (a subnormal half's mantissa holds bits 0-9:
      // value 4^j x field x 2^-24), fields 5-7 after one 10-bit shift; acc_post_scale
      // removes the 4^j'
      const uint32_t d10 = d >> 10;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t pj = j < 5 ? (d & (0x00030003u << (2 * j))) : (d10 & (0x00030003u << (2 * (j - 5))));
        acc[j] = fmaf(h16lo(pj), s, acc[j]);
        acc[j + 8] = fmaf(h16hi(pj), s, acc[j + 8]);
      }
    }
  } else if constexpr (WT == TBE_TY_FP16) {
    if constexpr (WEIGHTED) {
      acc[0] = fmaf(h16lo(d), w, acc[0]);
      acc[1] = fmaf(h16hi(d), w, acc[1]);
    } else {
      acc[0] += h16lo(d);
      acc[1] += h16hi(d);
    }
  } else if constexpr (WT == TBE_TY_FP8) {
    if (c.h16_ok) {
      // place each 7-bit body into an fp16 exponent/mantissa field, sign to bit 15:
      // fp16 value * 2^(15-bias) is the code's value (subnormal codes included)
      const float m = WEIGHTED ? c.h16_scale * w : c.h16_scale;
      const uint32_t x0 = d & 0x00FF00FFu, x1 = (d >> 8) & 0x00FF00FFu;
      const uint32_t p0 = ((x0 & 0x007F007Fu) << c.h16_shift) | ((x0 & 0x00800080u) << 8);
      const uint32_t p1 = ((x1 & 0x007F007Fu) << c.h16_shift) | ((x1 & 0x00800080u) << 8);
      acc[0] = fmaf(h16lo(p0), m, acc[0]);
      acc[2] = fmaf(h16hi(p0), m, acc[2]);
      acc[1] = fmaf(h16lo(p1), m, acc[1]);
      acc[3] = fmaf(h16hi(p1), m, acc[3]);
    } else {
      float v[E];
      decode<WT>(d, v, c);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = WEIGHTED ? fmaf(v[e], w, acc[e]) : acc[e] + v[e];
    }
  } else {  // FP32, BF16
    float v[E];
    decode<WT>(d, v, c);
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = WEIGHTED ? fmaf(v[e], w, acc[e]) : acc[e] + v[e];
  }
}

// Two rows at once, unweighted INT8 / INT4: byte k of both rows' words is placed
// in the two halves of one register (v_perm_b32: {row 1 byte k, 0, row 2 byte k, 0}),
// so one v_dot2_f32_f16 adds element e of both rows, each times its own fp16 scale
// (the halves read as q x 2^-24 subnormals, as in accum_row; the products are exact
// in fp32).  The two biases are summed into bacc by one more dot2 with {1, 1}.
// Same element order and post-scale as accum_row.
template <int WT>
constexpr bool kPairDot = WT == TBE_TY_INT8 || WT == TBE_TY_INT4;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

template <int WT>
__device__ __forceinline__ void accum_row_pair(float (&acc)[Traits<WT>::kEpd], float& bacc, uint32_t d1, uint32_t d2,
                                               uint32_t h1, uint32_t h2) {
  static_assert(kPairDot<WT>, "INT8 and INT4 rows");
  const uint32_t s2 = __builtin_amdgcn_perm(h2, h1, 0x05040100u);  // {scale 1, scale 2}
  const uint32_t b2 = __builtin_amdgcn_perm(h2, h1, 0x07060302u);  // {bias 1, bias 2}
  bacc = dot2(b2, 0x3C003C00u, bacc);                              // + bias 1 + bias 2
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t x = __builtin_amdgcn_perm(d2, d1, 0x0C000C00u | (static_cast<uint32_t>(4 + k) << 16) | k);
    if constexpr (WT == TBE_TY_INT8) {
      acc[k] = dot2(x, s2, acc[k]);
    } else {  // byte k holds elements 2k (low nibble) and 2k+1 (high nibble, x16)
      acc[2 * k] = dot2(x & 0x000F000Fu, s2, acc[2 * k]);
      acc[2 * k + 1] = dot2(x & 0x00F000F0u, s2, acc[2 * k + 1]);
    }
  }
}

// ---------------------------------------------------------------- output store

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  // round to nearest, ties to even; NaN stays a quiet NaN
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

typedef uint32_t tbe_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t tbe_u32x4 __attribute__((ext_vector_type(4)));

// Output stores: the output is written once and never read back here, so it is
// stored non-temporally and does not evict from L2 the embedding rows that bags
// share (config 2: 123 -> 121 us, config 3: 876 -> 857 us).  Index chunks keep
// plain loads: consecutive chunks share cache lines.
template <typename T>
__device__ __forceinline__ void out_store(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}

template <int E>
__device__ __forceinline__ void store_f32(float* o, const float (&r)[E]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(o);
  if constexpr (E % 4 == 0) {
    if ((a & 15u) == 0) {
#pragma unroll
      for (int i = 0; i < E; i += 4)
        out_store(reinterpret_cast<tbe_u32x4*>(o + i), tbe_u32x4{__float_as_uint(r[i]), __float_as_uint(r[i + 1]),
                                                             __float_as_uint(r[i + 2]), __float_as_uint(r[i + 3])});
      return;
    }
  }
  if constexpr (E % 2 == 0) {
    if ((a & 7u) == 0) {
#pragma unroll
      for (int i = 0; i < E; i += 2)
        out_store(reinterpret_cast<tbe_u32x2*>(o + i), tbe_u32x2{__float_as_uint(r[i]), __float_as_uint(r[i + 1])});
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < E; ++i) out_store(o + i, r[i]);
}

template <int E>
__device__ __forceinline__ void store_b16(uint16_t* o, const uint16_t (&b)[E]) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(o);
  if constexpr (E % 8 == 0) {
    if ((a & 15u) == 0) {
#pragma unroll
      for (int i = 0; i < E; i += 8) {
        const tbe_u32x4 w{b[i] | (uint32_t(b[i + 1]) << 16), b[i + 2] | (uint32_t(b[i + 3]) << 16),
                          b[i + 4] | (uint32_t(b[i + 5]) << 16), b[i + 6] | (uint32_t(b[i + 7]) << 16)};
        out_store(reinterpret_cast<tbe_u32x4*>(o + i), w);
      }
      return;
    }
  }
  if constexpr (E % 4 == 0) {
    if ((a & 7u) == 0) {
#pragma unroll
      for (int i = 0; i < E; i += 4) {
        out_store(reinterpret_cast<tbe_u32x2*>(o + i),
                  tbe_u32x2{b[i] | (uint32_t(b[i + 1]) << 16), b[i + 2] | (uint32_t(b[i + 3]) << 16)});
      }
      return;
    }
  }
  if constexpr (E % 2 == 0) {
    if ((a & 3u) == 0) {
#pragma unroll
      for (int i = 0; i < E; i += 2)
        out_store(reinterpret_cast<uint32_t*>(o + i), b[i] | (uint32_t(b[i + 1]) << 16));
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < E; ++i) out_store(o + i, b[i]);
}

// Write E consecutive output elements starting at element `pos` of the output,
// converting to the output dtype (fp16 / bf16 round to nearest even, P:330).
template <int E>
__device__ __forceinline__ void store_out(const KParams& p, int64_t pos, const float (&r)[E]) {
  if (p.out_ty == TBE_TY_FP32) {
    store_f32<E>(static_cast<float*>(p.out) + pos, r);
  } else {
    uint16_t b[E];
    if (p.out_ty == TBE_TY_FP16) {
#pragma unroll
      for (int i = 0; i < E; ++i) b[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(r[i]));
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) b[i] = static_cast<uint16_t>(f32_to_bf16_bits(r[i]));
    }
    store_b16<E>(static_cast<uint16_t*>(p.out) + pos, b);
  }
}

// store_out with the alignment decided by the caller: `vec` says the slice start
// is E-element aligned (one or two wide stores), else element by element.
template <int E>
__device__ __forceinline__ void store_slice(const KParams& p, int64_t pos, const float (&r)[E], bool vec) {
  if (p.out_ty == TBE_TY_FP32) {
    float* o = static_cast<float*>(p.out) + pos;
    if (vec && E % 4 == 0) {
#pragma unroll
      for (int i = 0; i < E; i += 4)
        out_store(reinterpret_cast<tbe_u32x4*>(o + i), tbe_u32x4{__float_as_uint(r[i]), __float_as_uint(r[i + 1]),
                                                             __float_as_uint(r[i + 2]), __float_as_uint(r[i + 3])});
    } else if (vec && E == 2) {
      out_store(reinterpret_cast<tbe_u32x2*>(o), tbe_u32x2{__float_as_uint(r[0]), __float_as_uint(r[1])});
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) out_store(o + i, r[i]);
    }
    return;
  }
  uint16_t b[E];
  if (p.out_ty == TBE_TY_FP16) {
#pragma unroll
    for (int i = 0; i < E; ++i) b[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(r[i]));
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) b[i] = static_cast<uint16_t>(f32_to_bf16_bits(r[i]));
  }
  uint16_t* o = static_cast<uint16_t*>(p.out) + pos;
  if constexpr (E >= 2) {
    if (!vec) {
#pragma unroll
      for (int i = 0; i < E; ++i) out_store(o + i, b[i]);
      return;
    }
    uint32_t w[E / 2];
#pragma unroll
    for (int i = 0; i < E / 2; ++i) w[i] = b[2 * i] | (uint32_t(b[2 * i + 1]) << 16);
    if constexpr (E % 8 == 0) {
#pragma unroll
      for (int i = 0; i < E / 2; i += 4)
        out_store(reinterpret_cast<tbe_u32x4*>(o + 2 * i), tbe_u32x4{w[i], w[i + 1], w[i + 2], w[i + 3]});
    } else if constexpr (E == 4) {
      out_store(reinterpret_cast<tbe_u32x2*>(o), tbe_u32x2{w[0], w[1]});
    } else {
      out_store(reinterpret_cast<uint32_t*>(o), w[0]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < E; ++i) out_store(o + i, b[i]);
  }
}

// ---------------------------------------------------------------- cross-lane sums

__device__ __forceinline__ float sum_xor32(float v) {
  // v_permlane32_swap exchanges the two 32-lane halves; adding both results
  // gives every lane v[l] + v[l ^ 32]
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v[l] + v[(l + n) mod 16 within the lane's row of 16]; applied for n = 8,4,2,1 in
// that order it sums lanes that differ in the low bits
template <int n>
__device__ __forceinline__ float add_row_ror(float v) {
  const int r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + n, 0xF, 0xF, false);
  return v + __int_as_float(r);
}

__device__ __forceinline__ float sum_slots(float v, int lg) {
  if (lg <= 5) v = sum_xor32(v);
  if (lg <= 4) v = sum_xor16(v);
  if (lg <= 3) v = add_row_ror<8>(v);
  if (lg <= 2) v = add_row_ror<4>(v);
  if (lg <= 1) v = add_row_ror<2>(v);
  if (lg == 0) v = add_row_ror<1>(v);
  return v;
}

// Sum over the row slots: lanes that agree in bits [0, lg) and differ above.
template <int E, bool HDR>
__device__ __forceinline__ void reduce_slots(float (&acc)[E], float& bacc, int lg) {
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = sum_slots(acc[e], lg);
  if (HDR) bacc = sum_slots(bacc, lg);
}

// Final value of the lane's E elements and their store (slot 0 lanes only).
template <int WT>
__device__ __forceinline__ void finish_bag(const KParams& p, const TbeTableDesc& td, int L, int dw, int64_t b,
                                           const float (&acc)[Traits<WT>::kEpd], float bacc) {
  constexpr int E = Traits<WT>::kEpd;
  const float scale = (p.mean && L > 0) ? 1.0f / static_cast<float>(L) : 1.0f;  // P:355
  float r[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float x = Traits<WT>::kHdr ? fmaf(acc[e], acc_post_scale<WT>(e), bacc) : acc[e];
    r[e] = p.mean ? x * scale : x;
  }
  store_out<E>(p, b * p.out_stride + td.D_offset + static_cast<int64_t>(dw) * E, r);
}

// ---------------------------------------------------------------- work items

// Work item -> bag of the group: table, sample, column tile and the bag's index
// range.  Returns false when the item's column tile does not exist for its table.
template <typename IndexT>
__device__ __forceinline__ bool item_bag(const KParams& p, uint32_t item, TbeTableDesc& td, int64_t& start,
                                         int& L, int& ct, int64_t& b, int32_t& t) {
  uint32_t k = item;
  ct = 0;
  if (p.col_tiles > 1) {
    k = fast_div(item, p.div_tiles);
    ct = static_cast<int>(item - k * static_cast<uint32_t>(p.col_tiles));
  }
  const uint32_t gt = static_cast<uint32_t>(uniform(static_cast<int>(fast_div(k, p.div_B))));
  b = static_cast<int64_t>(k - gt * static_cast<uint32_t>(p.B));
  t = p.order ? load_uniform(p.order + p.group_first + gt) : static_cast<int32_t>(gt);
  td = load_desc(p.tables + t);
  if (ct >= td.col_tiles) return false;
  const int64_t bag = static_cast<int64_t>(t) * p.B + b;
  // clamp to the index array so malformed offsets can never read out of bounds
  const IndexT* offs = static_cast<const IndexT*>(p.offsets);
  start = min(max(static_cast<int64_t>(load_uniform(offs + bag)), int64_t(0)), p.num_indices);
  const int64_t end = min(max(static_cast<int64_t>(load_uniform(offs + bag + 1)), start), p.num_indices);
  L = static_cast<int>(end - start);
  return true;
}

// Items [first, end) of this wave, stepping by `step`: one contiguous range per
// XCD, interleaved over the XCD's waves.
struct WaveItems {
  uint32_t first, end, step;
};

__device__ __forceinline__ WaveItems wave_items(const KParams& p) {
  const uint32_t wv = static_cast<uint32_t>(uniform(threadIdx.x >> 6));
  // every partition must own at least one block
  const uint32_t nparts = (p.xcd & 1) ? min(static_cast<uint32_t>(kNumXcd), gridDim.x) : 1u;
  const uint32_t part = blockIdx.x % nparts;
  const uint32_t lblk = blockIdx.x / nparts;
  const uint32_t nblk = (gridDim.x - part + nparts - 1) / nparts;  // blocks of this partition
  const uint32_t I = static_cast<uint32_t>(p.num_items);
  WaveItems w;
  w.first = static_cast<uint32_t>(static_cast<uint64_t>(I) * part / nparts) + lblk * kWavesPerBlock + wv;
  w.end = static_cast<uint32_t>(static_cast<uint64_t>(I) * (part + 1) / nparts);
  w.step = nblk * kWavesPerBlock;
  return w;
}

// ---------------------------------------------------------------- pooled bag, 32-bit tables

// Steps (of R = 64 >> LG rows each) whose loads are issued back to back before
// any is consumed: 8-32 rows in flight per wave for wide rows, a whole 64-index
// chunk for short rows.  U*R always divides 64, so slot r0 + u*R + slot of a
// step never passes lane 63 and slots past the bag read lanes holding kNoRow.
// Rows of 32 or more lanes take 8 per lane rather than 16: the two register sets
// shrink (INT8 D=128: 127 -> 95 VGPRs, 4 -> 5 waves per SIMD) and config 1 runs
// 43.1 -> 41.3 us, config 3 0.716 -> 0.698 ms; 4 per lane is slower on config 3,
// and 4 per lane for 16-lane rows (INT4 D=128) takes config 2 from 122 to 140 us.
template <int LG, int VW = 1>
constexpr int unroll_for() {
  return LG >= 5 ? 8 / VW : (LG == 4 ? 8 : kWave / (kWave >> LG));
}

// A bag whose first index chunk has been requested: the kernels issue the index
// load of the next bag before pooling the current one, so that load's latency
// hides behind the current bag's row loads.  Index chunks are read with buffer
// loads over exactly the chunk's bytes, so lanes past the chunk get zero from
// the range check: every path issues the same loads, which keeps the wait
// counts exact across the software pipeline.
struct StagedBag {
  int64_t start;
  int64_t b;
  int L;
  int ct;
  int32_t t;
  int valid;
  uint64_t idx;  // this lane's raw index of chunk 0 (meaningful for lane < min(L, 64))
  float w;       // its per-sample weight
};

template <typename IndexT>
__device__ __forceinline__ uint64_t load_index_chunk(const KParams& p, int64_t first, int n) {
  // n >= 0 indices from position `first`; lane >= n reads zero
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<IndexT*>(static_cast<const IndexT*>(p.indices) + first), 0,
      n * static_cast<int>(sizeof(IndexT)), kRsrcWord3);
  const int lane = threadIdx.x & (kWave - 1);
  if constexpr (sizeof(IndexT) == 8) {
    const int lo = __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 8, 0, 0);
    const int hi = __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 8 + 4, 0, 0);
    return static_cast<uint64_t>(static_cast<uint32_t>(lo)) | (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32);
  } else {
    // sign-extended so a negative int32 index is rejected like a negative int64
    return static_cast<uint64_t>(static_cast<int64_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4, 0, 0)));
  }
}

__device__ __forceinline__ float load_weight_chunk(const KParams& p, int64_t first, int n) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.psw + first), 0, n * 4, kRsrcWord3);
  return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (threadIdx.x & (kWave - 1)) * 4, 0, 0));
}

// Per-lane bag table: lane l describes item l of the current batch of the wave's
// items, gathered with vector loads once per 64 items so that no chain of
// dependent scalar loads (table order -> descriptor -> offsets) sits on the
// per-bag path.  Requires num_indices < 2^31.
struct BagTable {
  int32_t tct;    // table id | column tile << 24, or -1 (no such item / tile)
  int32_t b;      // sample
  uint32_t start; // first index position
  int32_t L;      // bag length
};

template <typename IndexT>
__device__ __forceinline__ BagTable load_bag_table(const KParams& p, uint32_t item, bool ok) {
  BagTable r;
  r.tct = -1;
  r.b = 0;
  r.start = 0;
  r.L = 0;
  if (ok) {
    uint32_t k = item;
    int ct = 0;
    if (p.col_tiles > 1) {
      k = fast_div(item, p.div_tiles);
      ct = static_cast<int>(item - k * static_cast<uint32_t>(p.col_tiles));
    }
    const uint32_t gt = fast_div(k, p.div_B);
    const int32_t b = static_cast<int32_t>(k - gt * static_cast<uint32_t>(p.B));
    const int32_t t = p.order[p.group_first + gt];
    const int tiles = static_cast<int>((reinterpret_cast<const uint32_t*>(p.tables + t)[9] >> 16) & 0xFFu);
    if (ct < tiles) {
      const int64_t bag = static_cast<int64_t>(t) * p.B + b;
      const IndexT* offs = static_cast<const IndexT*>(p.offsets);
      // clamp to the index array so malformed offsets can never read out of bounds
      const int64_t start = min(max(static_cast<int64_t>(offs[bag]), int64_t(0)), p.num_indices);
      const int64_t end = min(max(static_cast<int64_t>(offs[bag + 1]), start), p.num_indices);
      r.tct = t | (ct << 24);
      r.b = b;
      r.start = static_cast<uint32_t>(start);
      r.L = static_cast<int32_t>(end - start);
    }
  }
  return r;
}

// Stage the wave's item g (items are staged in order g = 0, 1, 2, ...): the bag
// table is (re)loaded when g starts a new batch of 64.
template <typename IndexT, bool WEIGHTED>
__device__ __forceinline__ StagedBag stage_bag(const KParams& p, const WaveItems& w, uint32_t nitems, BagTable& tab,
                                               uint32_t g) {
  if ((g & (kWave - 1)) == 0 && g < nitems) {  // wave-uniform
    const uint32_t l = g + (threadIdx.x & (kWave - 1));
    tab = load_bag_table<IndexT>(p, w.first + l * w.step, l < nitems);
  }
  StagedBag s;
  // every value goes through readfirstlane: selects on uniform values are
  // otherwise materialised in VGPRs and the buffer descriptors built from them
  // become waterfall loops
  const int kk = static_cast<int>(g & (kWave - 1));
  const int tct = uniform(g < nitems ? __builtin_amdgcn_readlane(tab.tct, kk) : -1);
  s.valid = tct >= 0;
  s.t = uniform(s.valid ? (tct & 0xFFFFFF) : 0);
  s.ct = uniform(s.valid ? (tct >> 24) : 0);
  s.b = __builtin_amdgcn_readlane(tab.b, kk);
  s.start = static_cast<uint32_t>(uniform(s.valid ? __builtin_amdgcn_readlane(static_cast<int>(tab.start), kk) : 0));
  s.L = uniform(s.valid ? __builtin_amdgcn_readlane(tab.L, kk) : 0);
  const int n = min(s.L, kWave);
  s.idx = load_index_chunk<IndexT>(p, s.start, n);
  s.w = WEIGHTED ? load_weight_chunk(p, s.start, n) : 0.f;
  return s;
}

// Reduce the R row slots of each element and store the bag's output slice.
// Slot bits 5 and 4 are reduce-scattered with permlane swaps: each swap+add
// finishes one element in each half of the lane pair, so after those levels a
// lane holds E>>k fully-summed elements and every slot stores its share; the
// slot bits below 4 are summed with DPP row rotations.
template <int WT, int LG, int E = Traits<WT>::kEpd>
__device__ __forceinline__ void reduce_store(const KParams& p, const TbeTableDesc& td, int L, int dw, bool col_ok,
                                             int64_t b, const float (&acc)[E], float bacc) {
  constexpr int EW = Traits<WT>::kEpd;  // elements per word; E = EW x words per lane
  constexpr bool HDR = Traits<WT>::kHdr;
  constexpr bool S5 = LG <= 5 && E >= 2;
  constexpr int E1 = S5 ? E / 2 : E;
  constexpr bool S4 = LG <= 4 && E1 >= 2;
  constexpr int E2 = S4 ? E1 / 2 : E1;
  const int lane = threadIdx.x & (kWave - 1);
  float a1[E1];
  if constexpr (S5) {
#pragma unroll
    for (int e = 0; e < E1; ++e) {
      // lanes 0-31 finish element e, lanes 32-63 element e + E1
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[e]), __float_as_uint(acc[e + E1]),
                                                      false, false);
      a1[e] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E1; ++e) a1[e] = LG <= 5 ? sum_xor32(acc[e]) : acc[e];
  }
  float a2[E2];
  if constexpr (S4) {
#pragma unroll
    for (int e = 0; e < E2; ++e) {
      // even rows of 16 finish element e, odd rows element e + E2
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a1[e]), __float_as_uint(a1[e + E2]),
                                                      false, false);
      a2[e] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < E2; ++e) a2[e] = LG <= 4 ? sum_xor16(a1[e]) : a1[e];
  }
#pragma unroll
  for (int e = 0; e < E2; ++e) {
    if constexpr (LG <= 3) a2[e] = add_row_ror<8>(a2[e]);
    if constexpr (LG <= 2) a2[e] = add_row_ror<4>(a2[e]);
    if constexpr (LG <= 1) a2[e] = add_row_ror<2>(a2[e]);
    if constexpr (LG == 0) a2[e] = add_row_ror<1>(a2[e]);
  }
  if constexpr (HDR) bacc = sum_slots(bacc, LG);

  // which lanes store: slot bits reduced by butterflies must be zero
  uint32_t need_zero = 0;
  if constexpr (LG < 4) need_zero |= (0xFu >> LG) << LG;  // bits [LG, 4)
  if constexpr (LG <= 4 && !S4) need_zero |= 0x10u;
  if constexpr (LG <= 5 && !S5) need_zero |= 0x20u;
  if (!col_ok || (static_cast<uint32_t>(lane) & need_zero)) return;
  int e0 = 0;
  if constexpr (S5) e0 += (lane & 32) ? E1 : 0;
  if constexpr (S4) e0 += (lane & 16) ? E2 : 0;
  const float scale = (p.mean && L > 0) ? 1.0f / static_cast<float>(L) : 1.0f;  // P:355
  float r[E2];
#pragma unroll
  for (int e = 0; e < E2; ++e) {
    const float x = HDR ? fmaf(a2[e], acc_post_scale<WT>((e0 + e) % EW), bacc) : a2[e];
    r[e] = p.mean ? x * scale : x;
  }
  store_out<E2>(p, b * p.out_stride + td.D_offset + static_cast<int64_t>(dw) * EW + e0, r);
}

// Zeros that a lane without a row reads in its place under 64-bit addressing (no
// range check there): a zero header and zero words add nothing.  Covers every
// column offset a lane of a row reads (255 tiles of 64 words after the header).
constexpr int kZeroRowWords = 256 * kWave + 4;
static __device__ __align__(16) const uint32_t g_zero_row[kZeroRowWords] = {};

// What a lane needs to gather rows of one bag's table.
struct BagCtx {
  __amdgpu_buffer_rsrc_t rs;  // the table's rows; range = rows * stride bytes
  const uint8_t* tbase;       // row 0 (64-bit addressing)
  const uint8_t* zero;        // the zero row (64-bit addressing)
  TbeTableDesc td;
  uint32_t col;               // byte offset of this lane's payload word in a row
  int dw;                     // payload word of this lane
  bool col_ok;                // that word exists (rows narrower than the lanes)
};

template <int LG, int VW = 1>
__device__ __forceinline__ BagCtx bag_ctx(const KParams& p, const StagedBag& sb) {
  BagCtx c;
  c.td = load_desc(p.tables + sb.t);
  const int lane = threadIdx.x & (kWave - 1);
  c.dw = sb.ct * kWave + (lane & ((1 << LG) - 1)) * VW;
  c.col_ok = c.dw < c.td.data_dwords;
  c.col = static_cast<uint32_t>(c.td.data_offset + (c.col_ok ? 4 * c.dw : 0));
  c.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.weights + c.td.weights_offset), 0,
                                           static_cast<int>(static_cast<uint32_t>(c.td.num_rows) *
                                                            static_cast<uint32_t>(c.td.row_stride)),
                                           kRsrcWord3);
  c.tbase = p.weights + c.td.weights_offset;
  c.zero = reinterpret_cast<const uint8_t*>(g_zero_row);
  return c;
}

// This lane's index of a chunk as a byte offset into the table (kNoRow for a
// rejected index or a lane past the chunk's n indices).  A64 (tables past 32-bit
// byte offsets, fewer than 2^32 - 1 rows): the row index itself, kNoRow64 for none.
constexpr uint32_t kNoRow64 = 0xFFFFFFFFu;
template <bool A64 = false>
__device__ __forceinline__ uint32_t row_offset(const BagCtx& c, uint64_t idx, int n) {
  const int lane = threadIdx.x & (kWave - 1);
  if constexpr (A64) {
    return (lane < n && idx < static_cast<uint64_t>(c.td.num_rows)) ? static_cast<uint32_t>(idx) : kNoRow64;
  } else {
    const uint32_t rows = static_cast<uint32_t>(c.td.num_rows);
    return (lane < n && idx < rows) ? static_cast<uint32_t>(idx) * static_cast<uint32_t>(c.td.row_stride) : kNoRow;
  }
}


// VW consecutive words at byte offset `off` of a buffer.
template <int VW>
__device__ __forceinline__ void load_words(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t (&w)[VW]) {
  if constexpr (VW == 1) {
    w[0] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(off), 0, 0));
  } else if constexpr (VW == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, static_cast<int>(off), 0, 0);
    w[0] = v[0];
    w[1] = v[1];
  } else {
    static_assert(VW == 4, "1, 2 or 4 words per lane");
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0);
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
    w[3] = v[3];
  }
}

// Registers of one gather step: U rows per lane slot.
template <int U, int VW = 1>
struct StepRegs {
  uint32_t d[U][VW], h[U];
  float w[U];
};

// Issue the loads of step `st` of a chunk (rows st*R*U .. st*R*U + R*U - 1).
// Slot st*R*U + u*R + slot < 64 because R*U divides 64; slots past the chunk
// read lanes that hold kNoRow and load zero.
template <int WT, int LG, bool WEIGHTED, int VW, bool A64 = false>
__device__ __forceinline__ void issue_step(const BagCtx& c, uint32_t my_off, float my_w, int st,
                                           StepRegs<unroll_for<LG, VW>(), VW>& r) {
  constexpr int R = kWave >> LG;
  constexpr int U = unroll_for<LG, VW>();
  const int slot4 = ((threadIdx.x & (kWave - 1)) >> LG) * 4;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int src = (st * R * U + u * R) * 4 + slot4;
    const uint32_t off = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(my_off)));
    if constexpr (A64) {
      static_assert(VW == 1, "64-bit addressing: one word per lane");
      // off is a row index; a lane without a row reads the zero row (the address
      // is selected, not the loaded value, so no wait is forced here)
      // selected with a mask rather than a branch
      const uint64_t hit = reinterpret_cast<uint64_t>(c.tbase) +
                           static_cast<uint64_t>(off) * static_cast<uint32_t>(c.td.row_stride);
      const uint64_t zr = reinterpret_cast<uint64_t>(c.zero);
      const uint64_t keep = 0ull - static_cast<uint64_t>(off != kNoRow64);
      const uint8_t* rp = reinterpret_cast<const uint8_t*>(zr ^ ((hit ^ zr) & keep));
      r.d[u][0] = load_word(rp + c.col);
      if constexpr (Traits<WT>::kHdr) r.h[u] = load_word(rp);
      else r.h[u] = 0u;
    } else {
      load_words<VW>(c.rs, off + c.col, r.d[u]);
      if constexpr (Traits<WT>::kHdr) r.h[u] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(c.rs, static_cast<int>(off), 0, 0));
      else r.h[u] = 0u;
    }
    if constexpr (WEIGHTED) r.w[u] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(my_w)));
    else r.w[u] = 1.f;
  }
}

template <int WT, int LG, bool WEIGHTED, int VW>
__device__ __forceinline__ void consume_step(const KParams& p, const StepRegs<unroll_for<LG, VW>(), VW>& r, int st, int n,
                                             float (&acc)[Traits<WT>::kEpd * VW], float& bacc) {
  constexpr int R = kWave >> LG;
  constexpr int U = unroll_for<LG, VW>();
  constexpr int EW = Traits<WT>::kEpd;
  if constexpr (!WEIGHTED && kPairDot<WT> && VW == 1 && U % 2 == 0) {
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      // wave-uniform; a row past the bag read zero words and a zero header, so it adds 0
      if (st * R * U + u * R < n) accum_row_pair<WT>(acc, bacc, r.d[u][0], r.d[u + 1][0], r.h[u], r.h[u + 1]);
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (st * R * U + u * R < n) {  // wave-uniform
#pragma unroll
      for (int v = 0; v < VW; ++v) {  // the row's bias once, with its first word
        float unused = 0.f;
        accum_row<WT, WEIGHTED>(*reinterpret_cast<float(*)[EW]>(&acc[v * EW]), v == 0 ? bacc : unused, r.d[u][v],
                                r.h[u], r.w[u], p.fp8);
      }
    }
  }
}

// Steps st0.. of one chunk of <= 64 indices, each issued then consumed.
template <int WT, int LG, bool WEIGHTED, int VW, bool A64>
__device__ __forceinline__ void pool_steps(const KParams& p, const BagCtx& c, uint32_t my_off, float my_w, int n,
                                           int st0, float (&acc)[Traits<WT>::kEpd * VW], float& bacc) {
  constexpr int kSteps = kWave / ((kWave >> LG) * unroll_for<LG, VW>());
#pragma unroll
  for (int st = 1; st < kSteps; ++st) {
    if (st >= st0 && st * (kWave / kSteps) < n) {  // wave-uniform
      StepRegs<unroll_for<LG, VW>(), VW> r;
      issue_step<WT, LG, WEIGHTED, VW, A64>(c, my_off, my_w, st, r);
      // keep the step's loads together, ahead of the guarded accumulations
      __builtin_amdgcn_sched_barrier(0);
      consume_step<WT, LG, WEIGHTED, VW>(p, r, st, n, acc, bacc);
    }
  }
}

// Finish a bag whose step 0 rows are in `r0`: consume them, gather the rest of
// the bag (longer than one step or one chunk), reduce and store (P:44-85 bag
// walk, P:282-315 pooling, P:346-394 chunked bag, P:319-342 store).
template <int WT, int LG, typename IndexT, bool WEIGHTED, int VW, bool A64>
__device__ __forceinline__ void finish_bag_fast(const KParams& p, const StagedBag& sb, const BagCtx& c,
                                                uint32_t my_off, const StepRegs<unroll_for<LG, VW>(), VW>& r0) {
  constexpr int E = Traits<WT>::kEpd * VW;
  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float bacc = 0.f;
  const int L = sb.L;
  const int n0 = min(L, kWave);
  consume_step<WT, LG, WEIGHTED, VW>(p, r0, 0, n0, acc, bacc);
  pool_steps<WT, LG, WEIGHTED, VW, A64>(p, c, my_off, sb.w, n0, 1, acc, bacc);
  for (int base = kWave; base < L; base += kWave) {
    const int n = min(kWave, L - base);
    const uint64_t idx = load_index_chunk<IndexT>(p, sb.start + base, n);
    const float w = WEIGHTED ? load_weight_chunk(p, sb.start + base, n) : 0.f;
    const uint32_t off = row_offset<A64>(c, idx, n);
    StepRegs<unroll_for<LG, VW>(), VW> r;
    issue_step<WT, LG, WEIGHTED, VW, A64>(c, off, w, 0, r);
    __builtin_amdgcn_sched_barrier(0);
    consume_step<WT, LG, WEIGHTED, VW>(p, r, 0, n, acc, bacc);
    pool_steps<WT, LG, WEIGHTED, VW, A64>(p, c, off, w, n, 1, acc, bacc);
  }
  if (sb.valid) reduce_store<WT, LG, E>(p, c.td, L, c.dw, c.col_ok, sb.b, acc, bacc);
}

// ---------------------------------------------------------------- pooled bag, 64-bit tables

// Same contract for tables whose rows span more than kNoRow bytes: 64-bit addresses and
// explicit masks instead of the buffer range check.  Lanes per row are a runtime
// value here.
template <int WT, bool WEIGHTED>
__device__ __forceinline__ void pool_bag_wide(const KParams& p, const TbeTableDesc& td, int64_t start, int L,
                                              int ct, int64_t b) {
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
  const int64_t rows = td.num_rows;
  const int64_t stride = td.row_stride;

  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float bacc = 0.f;

  for (int base = 0; base < L; base += kWave) {
    const int n = min(kWave, L - base);
    int64_t my_row = -1;
    float my_w = 0.f;
    if (lane < n) {
      const int64_t idx = load_index(p, p.indices, start + base + lane);
      if (idx >= 0 && idx < rows) my_row = idx;
      if constexpr (WEIGHTED) my_w = p.psw[start + base + lane];
    }
    const int32_t row_lo = static_cast<int32_t>(my_row);
    const int32_t row_hi = static_cast<int32_t>(my_row >> 32);
    for (int r0 = 0; r0 < n; r0 += R * kUnrollWide) {
      uint32_t d[kUnrollWide], h[kUnrollWide];
      float w[kUnrollWide];
#pragma unroll
      for (int u = 0; u < kUnrollWide; ++u) {
        d[u] = 0u;
        h[u] = 0u;
        w[u] = 0.f;
        if (r0 + u * R < n) {  // wave-uniform
          const int i = r0 + u * R + slot;
          const int src = (i & (kWave - 1)) * 4;
          const int64_t row = static_cast<int64_t>(
              (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, row_hi))) << 32) |
              static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, row_lo)));
          float wi = 1.f;
          if constexpr (WEIGHTED) wi = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(my_w)));
          if (i < n && row >= 0) {
            const int64_t roff = row * stride;
            if (col_ok) d[u] = load_word(lane_base + roff);
            if constexpr (HDR) h[u] = load_word(tbase + roff);
            w[u] = wi;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kUnrollWide; ++u)
        if (r0 + u * R < n) accum_row<WT, WEIGHTED>(acc, bacc, d[u], h[u], w[u], p.fp8);
    }
  }

  reduce_slots<E, HDR>(acc, bacc, lg);
  if (slot == 0 && col_ok) finish_bag<WT>(p, td, L, dw, b, acc, bacc);
}

// ---------------------------------------------------------------- pooled bags, row streams

// Rows of 8 or more payload words (LG >= 3).  A wave owns up to 63 consecutive
// bags of one table and splits them, at bag boundaries, into S slots of about
// equal row count.  The bags' index ranges are adjacent, so each slot walks ONE
// contiguous run of the index array: every step, every slot gathers its next
// row, whatever bag it belongs to.  No lane idles at bag ends, the wave does no
// per-bag setup, and no sum crosses slots: a slot's lanes own distinct columns,
// and a slot stores a bag's pooled slice the step its last row is consumed.
//  * A lane gathers VW = 2 consecutive words (8 bytes) of a row (1 for INT2):
//    the more rows one load instruction reaches, the more misses the vector
//    L1 keeps in flight, and random-row throughput follows.  A slot is
//    SL = 2^LG / VW lanes, so a wave gathers 64/SL rows per step.
//  * Row byte offsets are computed once per index chunk: lane l holds entry
//    l mod C (C = min(SL, 8)) of its slot's next C indices.  Step J hands
//    entry J's offset to the slot's lanes with a DPP row broadcast (SL >= 16)
//    or an LDS crossbar read at a constant offset (SL < 16).
//  * Rows are read with raw buffer loads from the table base; rejected indices
//    and slots past their run use an offset that fails the range check, which
//    reads zero.
//  * Loads run one chunk (C steps) ahead of the accumulation through a
//    C-entry register ring: 8 steps of 8-byte lanes, 4 KiB in flight per wave.

constexpr int kMaxBagsPerWave = kWave - 1;  // the wave keeps its bags' offsets in one VGPR
constexpr int32_t kNever = 0x40000000;      // `rel` of a slot that has no bag left
#ifndef TBE_STREAM_RING
#define TBE_STREAM_RING 8
#endif
constexpr int kStreamRing = TBE_STREAM_RING;  // steps of loads in flight per wave
// Payload words a lane gathers per row (2^LG words per row): 2 (8-byte lanes)
// while a slot keeps at least 4 lanes and a lane at most 16 accumulators; 1
// otherwise.  (16-byte lanes reach more rows per load instruction, but their
// 32 accumulators per lane make the per-bag epilogue, run by 4 of 64 lanes,
// cost more than the wider loads save.)
constexpr int stream_vw_for(int elems_per_word, int lg) {
  return (lg >= 3 && elems_per_word <= 8) ? 2 : 1;
}
template <int WT, int LG>
constexpr int stream_vw() {
  return stream_vw_for(Traits<WT>::kEpd, LG);
}
// Words per lane of the per-bag kernel.  Two words (8 bytes) for INT4 rows of
// 17-32 payload words: the row then takes 16 lanes, a load instruction reaches 4
// rows instead of 2, and a lane's 16 elements share one row's address and weight
// work (config 3's INT4 D=256 tables: 148 -> 105 us).  Measured and kept at one
// word elsewhere: 16-word rows (INT4/INT8/FP16, 3-10 % slower), INT8 and FP16
// rows of 17-32 words (no gain or up to 6 % slower), 33-64-word rows (15-40 %
// slower at 2 words with 16 rows per lane in flight, 3-5 % with 8).
template <int WT, int LG>
constexpr int fast_vw() {
  return (LG == 5 && WT == TBE_TY_INT4) ? 2 : 1;
}
inline int stream_vw_of(int weight_ty, int lg) {
  static const int epw[] = {1, 2, 4, 8, 16, 2, 4};  // elements per word by TbeSparseType
  return stream_vw_for(epw[weight_ty], lg);
}

template <int J, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (J < N) {
    f(std::integral_constant<int, J>{});
    static_for<J + 1, N>(f);
  }
}

// Value of lane J of the caller's 16-lane row, in every lane of that row.
template <int J>
__device__ __forceinline__ uint32_t row_bcast(uint32_t v) {
  // every lane has a valid source lane, so bound_ctrl needs no "old" operand
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x150 + J, 0xF, 0xF, true));
}

// Entry J of the caller's slot (2^SLG lanes; entries at lanes slot_first + J).
template <int SLG, int J>
__device__ __forceinline__ uint32_t slot_bcast(uint32_t v) {
  if constexpr (SLG >= 4) {
    return row_bcast<J>(v);
  } else if constexpr (SLG == 2) {
    // quad_perm [J, J, J, J]
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), J * 0x55, 0xF, 0xF, true));
  } else {
    const int base = static_cast<int>((threadIdx.x & (kWave - 1)) >> SLG) << (SLG + 2);
    return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(base + 4 * J, static_cast<int>(v)));
  }
}


// Entry l mod C of a slot's index chunk starting at position q0 (-1 past the
// slot's run) and its per-sample weight.  The raw index is kept until the chunk
// is used, a chunk later: computing with it here would make the wave wait for
// this load, and with it for every row load issued before it.
template <typename IndexT, bool WEIGHTED, int C>
__device__ __forceinline__ void load_stream_chunk(const KParams& p, uint32_t q0, uint32_t end, IndexT& idx, float& w) {
  const uint32_t q = q0 + (threadIdx.x & (C - 1));
  idx = -1;
  w = 0.f;
  if (q < end) {
    // plain loads: a slot's consecutive chunks share cache lines
    idx = static_cast<const IndexT*>(p.indices)[q];
    if constexpr (WEIGHTED) w = p.psw[q];
  }
}

// Row byte offset of a raw chunk index (kNoRow outside [0, rows)).
template <typename IndexT>
__device__ __forceinline__ uint32_t row_byte_offset(IndexT idx, uint32_t rows, uint32_t stride) {
  const int64_t v = static_cast<int64_t>(idx);
  return (v >= 0 && v < static_cast<int64_t>(rows)) ? static_cast<uint32_t>(v) * stride : kNoRow;
}

template <int WT, int LG, typename IndexT, bool WEIGHTED>
__global__ __launch_bounds__(kBlock) void pooled_stream_kernel(KParams p) {
  constexpr int VW = stream_vw<WT, LG>();
  constexpr int EW = Traits<WT>::kEpd;  // elements per word
  constexpr int E = EW * VW;            // elements per lane
  constexpr bool HDR = Traits<WT>::kHdr;
  constexpr int SLG = LG - (VW == 4 ? 2 : VW == 2 ? 1 : 0);  // log2 lanes per slot
  constexpr int SL = 1 << SLG;
  constexpr int S = kWave / SL;         // slots per wave
  constexpr int C = SL < kStreamRing ? SL : kStreamRing;  // index entries per slot per chunk = ring depth
  static_assert(SLG >= 2, "a slot spans at least 4 lanes");
  __shared__ int32_t lds_off[kWavesPerBlock][kWave];
  __shared__ float lds_inv[kWavesPerBlock][kWave];

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = uniform(threadIdx.x >> 6);
  // XCD-aware block order: the hardware deals blocks to the 8 XCDs round-robin;
  // renumber so each XCD runs one contiguous range of items (adjacent bags of the
  // same tables share that XCD's L2)
  uint32_t lblk = blockIdx.x;
  if (p.xcd & 1) {
    const uint32_t nb = gridDim.x, x = blockIdx.x % kNumXcd;
    lblk = x * (nb / kNumXcd) + min(x, nb % kNumXcd) + blockIdx.x / kNumXcd;
  }
  const uint32_t item = lblk * kWavesPerBlock + wv;
  if (item >= static_cast<uint32_t>(p.num_items)) return;
  uint32_t k = item;
  int ct = 0;
  if (p.col_tiles > 1) {
    k = fast_div(item, p.div_tiles);
    ct = static_cast<int>(item - k * static_cast<uint32_t>(p.col_tiles));
  }
  const uint32_t gt = uniform(static_cast<int>(fast_div(k, p.div_ranges)));
  const int32_t rng = static_cast<int32_t>(k - gt * static_cast<uint32_t>(p.ranges));
  const int32_t t = load_uniform(p.order + p.group_first + gt);
  const TbeTableDesc td = load_desc(p.tables + t);
  if (ct >= td.col_tiles) return;
  const int32_t b0 = rng * p.bags_per_wave;
  const int nb = min(p.bags_per_wave, p.B - b0);
  const int64_t bag0 = static_cast<int64_t>(t) * p.B + b0;

  // offsets of bags b0 .. b0+nb, clamped to the index array (lane l: start of bag
  // l).  Offsets must not decrease; if they do (invalid input) the running
  // maximum is used, so every read stays inside the index array.
  int32_t o = 0;
  if (lane <= nb) {
    const int64_t v = static_cast<int64_t>(static_cast<const IndexT*>(p.offsets)[bag0 + lane]);
    o = static_cast<int32_t>(min(max(v, int64_t(0)), p.num_indices));
  }
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int32_t x = __builtin_amdgcn_ds_bpermute((lane - d) * 4, o);
    if (lane >= d) o = max(o, x);
  }
  lds_off[wv][lane] = o;
  {
    // 1/L of bag `lane` for MEAN (P:355: float(1)/float(L)), else 1
    const int32_t L = __builtin_amdgcn_ds_bpermute((lane + 1) * 4, o) - o;
    lds_inv[wv][lane] = (p.mean && L > 0) ? 1.0f / static_cast<float>(L) : 1.0f;
  }
  // the wave's stores are E-element vectors when every slice start is aligned
  const bool vec_out = (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0 && p.out_stride % E == 0 && td.D_offset % E == 0;

  // split the bags into S slots of about equal rows: slot s takes the bags whose
  // first index lies in [first + total*s/S, first + total*(s+1)/S)
  const int slot = lane >> SLG;
  const int32_t first = __builtin_amdgcn_readlane(o, 0);
  const int32_t total = __builtin_amdgcn_readlane(o, nb) - first;
  int kbeg = 0, kend = nb;
#pragma unroll
  for (int s = 1; s < S; ++s) {
    const int32_t target = first + static_cast<int32_t>(static_cast<int64_t>(total) * s / S);
    const int c = __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < nb && o < target));
    if (slot >= s) kbeg = c;
    if (slot == s - 1) kend = c;
  }
  __builtin_amdgcn_wave_barrier();
  uint32_t pos = static_cast<uint32_t>(lds_off[wv][kbeg]);        // first row of the chunk being consumed
  const uint32_t end = static_cast<uint32_t>(lds_off[wv][kend]);  // end of the slot's run
  int kc = kbeg;                                                  // bag being pooled
  int32_t rel = kc < kend ? lds_off[wv][kc + 1] - static_cast<int32_t>(pos) - 1 : kNever;
  // longest run of the wave's slots (slot s starts at lane s * SL)
  const uint32_t run = end - pos;
  uint32_t longest = 0;
#pragma unroll
  for (int s = 0; s < S; ++s) longest = max(longest, static_cast<uint32_t>(__builtin_amdgcn_readlane(run, s * SL)));
  const int nchunks = static_cast<int>((longest + C - 1) / C);

  const int dw = ct * kWave + VW * (lane & (SL - 1));  // first payload word of this lane
  const bool col_ok = dw < td.data_dwords;
  const uint32_t col = static_cast<uint32_t>(col_ok ? td.data_offset + 4 * dw : 0);
  const uint32_t rows = static_cast<uint32_t>(td.num_rows);
  const uint32_t stride = static_cast<uint32_t>(td.row_stride);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(p.weights + td.weights_offset), 0, static_cast<int>(rows * stride), kRsrcWord3);

  float acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.f;
  float bacc = 0.f;

  // store the pooled slice of bag kc and move to the next bag, for every slot
  // whose bag ends at row pos + J (J = -1: empty bags before the first row)
  auto finish = [&](int J) __attribute__((always_inline)) {
    do {
      if (col_ok) {
        const float scale = lds_inv[wv][kc];
        float r[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float x = HDR ? fmaf(acc[e], acc_post_scale<WT>(e % EW), bacc) : acc[e];
          r[e] = x;
        }
        if (p.mean) {
#pragma unroll
          for (int e = 0; e < E; ++e) r[e] *= scale;
        }
        store_slice<E>(p, static_cast<int64_t>(b0 + kc) * p.out_stride + td.D_offset + static_cast<int64_t>(dw) * EW,
                       r, vec_out);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] = 0.f;
      bacc = 0.f;
      ++kc;
      rel = kc < kend ? lds_off[wv][kc + 1] - static_cast<int32_t>(pos) - 1 : kNever;
    } while (rel == J);
  };
  if (rel == -1) finish(-1);

  // accumulate one row: VW words, the bias once
  auto accum = [&](const uint32_t (&d)[VW], uint32_t h, float w) {
#pragma unroll
    for (int v = 0; v < VW; ++v) {
      float dummy = 0.f;
      accum_row<WT, WEIGHTED>(*reinterpret_cast<float(*)[EW]>(&acc[v * EW]), v == 0 ? bacc : dummy, d[v], h, w,
                              p.fp8);
    }
  };

  IndexT i1, i2;
  float w0, w1, w2;
  load_stream_chunk<IndexT, WEIGHTED, C>(p, pos, end, i1, w0);
  const uint32_t off0 = row_byte_offset(i1, rows, stride);
  load_stream_chunk<IndexT, WEIGHTED, C>(p, pos + C, end, i1, w1);
  uint32_t rd[C][VW], rh[C];
  // the row's header word (fp16 scale, fp16 bias) is read in the same step as
  // its payload: same cache line, so the L1 merges the two requests
  auto issue = [&](auto jc, uint32_t offc) __attribute__((always_inline)) {
    constexpr int J = decltype(jc)::value;
    const uint32_t r = slot_bcast<SLG, J>(offc);
    load_words<VW>(rs, r + col, rd[J]);
    rh[J] = HDR ? static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(r), 0, 0)) : 0u;
  };
  static_for<0, C>([&](auto jc) __attribute__((always_inline)) { issue(jc, off0); });
  i2 = -1;

  // consume the chunk in the ring; when ISSUE, refill each entry with the next
  // chunk's row as soon as it is consumed
  auto chunk_step = [&](auto issue_tag) __attribute__((always_inline)) {
    constexpr bool ISSUE = decltype(issue_tag)::value;
    uint32_t off1 = 0;
    if constexpr (ISSUE) {
      off1 = row_byte_offset(i1, rows, stride);
      load_stream_chunk<IndexT, WEIGHTED, C>(p, pos + 2 * C, end, i2, w2);
    }
    static_for<0, C>([&](auto jc) __attribute__((always_inline)) {
      constexpr int J = decltype(jc)::value;
      const float w = WEIGHTED ? __uint_as_float(slot_bcast<SLG, J>(__float_as_uint(w0))) : 1.f;
      accum(rd[J], rh[J], w);
      if constexpr (ISSUE) issue(jc, off1);
      if (rel == J) finish(J);
    });
    pos += C;
    rel -= C;
    w0 = w1;
    if constexpr (ISSUE) {
      i1 = i2;
      w1 = w2;
    }
  };
  for (int c = 0; c + 1 < nchunks; ++c) chunk_step(std::true_type{});
  if (nchunks > 0) chunk_step(std::false_type{});
}

// ---------------------------------------------------------------- nobag, 32-bit tables

// pooling_mode NONE (N:224-300): output row i is the dequantised row of
// indices[i].  One wave takes 64 consecutive positions; per table segment the 64
// indices arrive with one coalesced load, their row offsets reach the row lanes
// by ds_bpermute, and every row load of the segment is issued before the first
// is decoded.  Specialised per (weight type, lanes per row) like the pooled
// kernels; segments of other tables are left to their own group's launch.

// Decoded (exact) values of one payload word, INT4 through byte conversions.
template <int WT>
__device__ __forceinline__ void decode_word(uint32_t d, float (&v)[Traits<WT>::kEpd], const Fp8Consts& c) {
  if constexpr (WT == TBE_TY_INT4) {
    const uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = static_cast<float>((lo >> (8 * k)) & 0xFFu);
      v[2 * k + 1] = static_cast<float>((hi >> (8 * k)) & 0xFFu);
    }
  } else {
    decode<WT>(d, v, c);
  }
}

template <int WT, int LG, typename IndexT, bool A64>
__device__ __forceinline__ void nobag_segment(const KParams& p, const TbeTableDesc& td, int64_t a, int n) {
  constexpr int E = Traits<WT>::kEpd;
  constexpr bool HDR = Traits<WT>::kHdr;
  constexpr int R = kWave >> LG;               // rows per load instruction
  constexpr int U = kWave / R;                 // load instructions per 64 rows
  constexpr int UB = U < 16 ? U : 16;          // issued together
  const int lane = threadIdx.x & (kWave - 1);
  const int slot = lane >> LG;
  const uint32_t rows = static_cast<uint32_t>(td.num_rows);
  const uint32_t stride = static_cast<uint32_t>(td.row_stride);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(p.weights + td.weights_offset), 0, static_cast<int>(rows * stride), kRsrcWord3);
  const uint64_t raw = load_index_chunk<IndexT>(p, a, n);
  const int64_t iv = sizeof(IndexT) == 8 ? static_cast<int64_t>(raw) : static_cast<int64_t>(static_cast<int32_t>(raw));
  // A64: the row index (kNoRow64 for none); else the row's byte offset (kNoRow)
  const bool has_row = lane < n && iv >= 0 && iv < static_cast<int64_t>(td.num_rows);
  const uint32_t off = A64 ? (has_row ? static_cast<uint32_t>(iv) : kNoRow64)
                           : (has_row ? static_cast<uint32_t>(iv) * stride : kNoRow);
  const uint8_t* tbase = p.weights + td.weights_offset;
  const bool vec = (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0 && p.out_stride % E == 0;
  for (int ct = 0; ct < td.col_tiles; ++ct) {
    const int dw = ct * kWave + (lane & ((1 << LG) - 1));
    const bool col_ok = dw < td.data_dwords;
    const uint32_t col = static_cast<uint32_t>(td.data_offset + (col_ok ? 4 * dw : 0));
#pragma unroll
    for (int u0 = 0; u0 < U; u0 += UB) {
      if (u0 * R >= n) break;  // wave-uniform
      uint32_t d[UB], h[UB];
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        const uint32_t o = static_cast<uint32_t>(
            __builtin_amdgcn_ds_bpermute(((u0 + u) * R + slot) * 4, static_cast<int>(off)));
        if constexpr (A64) {  // a lane without a row reads the zero row
          const uint8_t* rp = o != kNoRow64 ? tbase + static_cast<uint64_t>(o) * stride
                                            : reinterpret_cast<const uint8_t*>(g_zero_row);
          d[u] = load_word(rp + col);
          h[u] = HDR ? load_word(rp) : 0u;
        } else {
          d[u] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(o + col), 0, 0));
          h[u] = HDR ? static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(o), 0, 0)) : 0u;
        }
      }
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        const int row = (u0 + u) * R + slot;
        if (row < n && col_ok) {
          float v[E], r[E];
          decode_word<WT>(d[u], v, p.fp8);
          // a rejected index reads a zero word and header: scale 0, bias 0 -> zeros
          const float sc = HDR ? h16lo(h[u]) : 1.f, bi = HDR ? h16hi(h[u]) : 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) r[e] = HDR ? fmaf(sc, v[e], bi) : v[e];
          store_slice<E>(p, (a + row) * p.out_stride + static_cast<int64_t>(dw) * E, r, vec);
        }
      }
    }
  }
}

// Output rows of positions that no table's segment covers (before offsets[0], or
// from offsets[T*B] on, e.g. when len(offsets)-1 is not a multiple of T) are
// zero, as the reference's zero-initialised output leaves them (A:135).  One
// launch of a forward (p.zero_gaps) writes them.
__device__ __forceinline__ void nobag_zero_gaps(const KParams& p, int64_t i0, int64_t i1) {
  const int64_t first = load_offset(p, 0);
  const int64_t last = load_offset(p, static_cast<int64_t>(p.T) * p.B);
  if (i0 >= first && i1 <= last) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);
  for (int64_t i = i0; i < i1; ++i) {
    if (i >= first && i < last) continue;
    for (int64_t c = lane; c < p.out_stride; c += kWave) {
      if (p.out_ty == TBE_TY_FP32) static_cast<float*>(p.out)[i * p.out_stride + c] = 0.f;
      else static_cast<uint16_t*>(p.out)[i * p.out_stride + c] = 0;
    }
  }
}

// A64: the group's tables are past 32-bit byte offsets (64-bit row addresses).
template <int WT, int LG, typename IndexT, bool A64 = false>
__global__ __launch_bounds__(kBlock) void nobag_fast_kernel(KParams p) {
  const int wv = uniform(threadIdx.x >> 6);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wv;
  if (item >= p.num_items) return;
  const int64_t i0 = item * kWave;
  const int64_t i1 = min(i0 + kWave, p.num_indices);
  if (p.zero_gaps) nobag_zero_gaps(p, i0, i1);
  // last table whose first index is <= i0 (N:57-78 walks tables by offset_per_key)
  int lo = 0, hi = p.T - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (load_offset(p, static_cast<int64_t>(mid) * p.B) <= i0) lo = mid; else hi = mid - 1;
  }
  for (int t = lo; t < p.T; ++t) {
    const int64_t tb = load_offset(p, static_cast<int64_t>(t) * p.B);
    const int64_t te = load_offset(p, static_cast<int64_t>(t + 1) * p.B);
    if (tb >= i1) break;
    const int64_t a = max(tb, i0), e = min(te, i1);
    if (a >= e) continue;
    const TbeTableDesc td = load_desc(p.tables + t);
    if (td.weight_ty != WT || td.log2_lanes != LG || ((td.flags & TBE_TABLE_OFFSET32) != 0) == A64) continue;
    if (A64 && td.num_rows >= static_cast<int64_t>(kNoRow64)) continue;  // the generic kernel's
    nobag_segment<WT, LG, IndexT, A64>(p, td, a, static_cast<int>(e - a));
  }
}

// ---------------------------------------------------------------- pooled kernels


// Kernel for one group of tables with weight type WT and 2^LG lanes per row, rows
// read with range-checked buffer loads at 32-bit byte offsets, or (A64, tables
// past 4 GiB) with 64-bit addresses, a lane without a row reading the zero row.
// Software pipeline over the wave's items: while bag i is consumed, the rows of
// bag i+1 are in flight and the index chunk of bag i+2 is being fetched.  The
// loop body is unrolled twice so the two row buffers swap roles without copies.
template <int WT, int LG, typename IndexT, bool WEIGHTED, int VW, bool A64 = false>
__global__ __launch_bounds__(kBlock) void pooled_fast_kernel(KParams p) {
  // VW words per lane: 2^LGE lanes cover a row's 2^LG words of this column tile
  constexpr int LGE = VW == 2 ? LG - 1 : LG;
  constexpr int U = unroll_for<LGE, VW>();
  const WaveItems w = wave_items(p);
  if (w.first >= w.end) return;
  const uint32_t nitems = (w.end - w.first + w.step - 1) / w.step;
  BagTable tab;
  uint32_t g = 0;
  StagedBag s0 = stage_bag<IndexT, WEIGHTED>(p, w, nitems, tab, 0);
  StagedBag s1 = stage_bag<IndexT, WEIGHTED>(p, w, nitems, tab, 1);
  BagCtx c0 = bag_ctx<LGE, VW>(p, s0);
  uint32_t off0 = row_offset<A64>(c0, s0.idx, min(s0.L, kWave));
  StepRegs<U, VW> ra, rb;
  issue_step<WT, LGE, WEIGHTED, VW, A64>(c0, off0, s0.w, 0, ra);
  // Wave priority by progress (when the launch runs alone, xcd bit 1): every wave
  // starts at priority 3 and drops one level per quarter of its items, so at any
  // moment the waves that are behind issue first, and the kernel's last waves are
  // the ones that were slowest (config 2 123.6 -> 117.9 us, config 1 42.0 -> 39.9 us).
  // Next to other groups' kernels on other streams it is off: the thresholds are
  // all zero, so the first check (g = 0) drops the wave to priority 0 before its
  // first bag (a separate branch around the first s_setprio costs the INT4 kernel
  // 20 VGPRs and a wave per SIMD); at priority 3 throughout, fresh waves of the
  // next kernel held back the previous kernel's last waves (config 3 0.70 -> 0.72 ms).
  const uint32_t on_q = (p.xcd & 2) ? 0xFFFFFFFFu : 0u;
  const uint32_t q1 = uniform(static_cast<int>((nitems >> 2) & on_q));
  const uint32_t q2 = uniform(static_cast<int>((nitems >> 1) & on_q));
  const uint32_t q3 = uniform(static_cast<int>(((nitems >> 2) + (nitems >> 1)) & on_q));
  __builtin_amdgcn_s_setprio(3);
  while (true) {
    if ((g & 3) == 0) {
      if (g >= q3) __builtin_amdgcn_s_setprio(0);
      else if (g >= q2) __builtin_amdgcn_s_setprio(1);
      else if (g >= q1) __builtin_amdgcn_s_setprio(2);
    }
    StagedBag s2 = stage_bag<IndexT, WEIGHTED>(p, w, nitems, tab, g + 2);
    BagCtx c1 = bag_ctx<LGE, VW>(p, s1);
    uint32_t off1 = row_offset<A64>(c1, s1.idx, min(s1.L, kWave));
    issue_step<WT, LGE, WEIGHTED, VW, A64>(c1, off1, s1.w, 0, rb);
    __builtin_amdgcn_sched_barrier(0);
    finish_bag_fast<WT, LGE, IndexT, WEIGHTED, VW, A64>(p, s0, c0, off0, ra);
    if (++g >= nitems) break;
    s0 = s1;
    c0 = c1;
    off0 = off1;
    s1 = s2;

    s2 = stage_bag<IndexT, WEIGHTED>(p, w, nitems, tab, g + 2);
    c1 = bag_ctx<LGE, VW>(p, s1);
    off1 = row_offset<A64>(c1, s1.idx, min(s1.L, kWave));
    issue_step<WT, LGE, WEIGHTED, VW, A64>(c1, off1, s1.w, 0, ra);
    __builtin_amdgcn_sched_barrier(0);
    finish_bag_fast<WT, LGE, IndexT, WEIGHTED, VW, A64>(p, s0, c0, off0, rb);
    if (++g >= nitems) break;
    s0 = s1;
    c0 = c1;
    off0 = off1;
    s1 = s2;
  }
}

// Kernel for a group of 64-bit tables (any weight type, runtime lanes per row).
template <bool WEIGHTED>
__global__ __launch_bounds__(kBlock) void pooled_wide_kernel(KParams p) {
  const WaveItems w = wave_items(p);
  for (uint32_t item = w.first; item < w.end; item += w.step) {
    TbeTableDesc td;
    int64_t start, b;
    int L, ct;
    int32_t t;
    const bool ok = p.index64 ? item_bag<int64_t>(p, item, td, start, L, ct, b, t)
                              : item_bag<int32_t>(p, item, td, start, L, ct, b, t);
    if (!ok) continue;
    switch (td.weight_ty) {
      case TBE_TY_INT4: pool_bag_wide<TBE_TY_INT4, WEIGHTED>(p, td, start, L, ct, b); break;
      case TBE_TY_INT8: pool_bag_wide<TBE_TY_INT8, WEIGHTED>(p, td, start, L, ct, b); break;
      case TBE_TY_INT2: pool_bag_wide<TBE_TY_INT2, WEIGHTED>(p, td, start, L, ct, b); break;
      case TBE_TY_FP8:  pool_bag_wide<TBE_TY_FP8,  WEIGHTED>(p, td, start, L, ct, b); break;
      case TBE_TY_FP16: pool_bag_wide<TBE_TY_FP16, WEIGHTED>(p, td, start, L, ct, b); break;
      case TBE_TY_BF16: pool_bag_wide<TBE_TY_BF16, WEIGHTED>(p, td, start, L, ct, b); break;
      case TBE_TY_FP32: pool_bag_wide<TBE_TY_FP32, WEIGHTED>(p, td, start, L, ct, b); break;
      default: break;  // rejected by the planner
    }
  }
}

using KernelFn = void (*)(KParams);

template <int WT, int LG, int VW>
KernelFn fast_kernel_vw(bool index64, bool weighted) {
  if (index64)
    return weighted ? pooled_fast_kernel<WT, LG, int64_t, true, VW> : pooled_fast_kernel<WT, LG, int64_t, false, VW>;
  return weighted ? pooled_fast_kernel<WT, LG, int32_t, true, VW> : pooled_fast_kernel<WT, LG, int32_t, false, VW>;
}

template <int WT, int LG>
KernelFn fast_kernel_for(bool index64, bool weighted, bool wide_words) {
  if constexpr (fast_vw<WT, LG>() == 2) {
    if (wide_words) return fast_kernel_vw<WT, LG, 2>(index64, weighted);
  }
  return fast_kernel_vw<WT, LG, 1>(index64, weighted);
}

// The per-bag kernel with 64-bit row addresses (one word per lane), for tables
// past 32-bit byte offsets that still have fewer than 2^32 - 1 rows.
template <int WT, int LG>
KernelFn fast_kernel_a64_for(bool index64, bool weighted) {
  if (index64)
    return weighted ? pooled_fast_kernel<WT, LG, int64_t, true, 1, true> : pooled_fast_kernel<WT, LG, int64_t, false, 1, true>;
  return weighted ? pooled_fast_kernel<WT, LG, int32_t, true, 1, true> : pooled_fast_kernel<WT, LG, int32_t, false, 1, true>;
}

template <int WT>
KernelFn fast_kernel_a64_lg(int lg, bool index64, bool weighted) {
  switch (lg) {
    case 0: return fast_kernel_a64_for<WT, 0>(index64, weighted);
    case 1: return fast_kernel_a64_for<WT, 1>(index64, weighted);
    case 2: return fast_kernel_a64_for<WT, 2>(index64, weighted);
    case 3: return fast_kernel_a64_for<WT, 3>(index64, weighted);
    case 4: return fast_kernel_a64_for<WT, 4>(index64, weighted);
    case 5: return fast_kernel_a64_for<WT, 5>(index64, weighted);
    default: return fast_kernel_a64_for<WT, 6>(index64, weighted);
  }
}

// wide_words: every table of the group has an even number of payload words
// (TBE_TABLE_STREAM), so lanes may read two words at a time.
template <int WT>
KernelFn fast_kernel_lg(int lg, bool index64, bool weighted, bool wide_words) {
  switch (lg) {
    case 0: return fast_kernel_for<WT, 0>(index64, weighted, wide_words);
    case 1: return fast_kernel_for<WT, 1>(index64, weighted, wide_words);
    case 2: return fast_kernel_for<WT, 2>(index64, weighted, wide_words);
    case 3: return fast_kernel_for<WT, 3>(index64, weighted, wide_words);
    case 4: return fast_kernel_for<WT, 4>(index64, weighted, wide_words);
    case 5: return fast_kernel_for<WT, 5>(index64, weighted, wide_words);
    default: return fast_kernel_for<WT, 6>(index64, weighted, wide_words);
  }
}

template <int WT, int LG>
KernelFn stream_kernel_for(bool index64, bool weighted) {
  if (index64)
    return weighted ? pooled_stream_kernel<WT, LG, int64_t, true> : pooled_stream_kernel<WT, LG, int64_t, false>;
  return weighted ? pooled_stream_kernel<WT, LG, int32_t, true> : pooled_stream_kernel<WT, LG, int32_t, false>;
}

template <int WT>
KernelFn nobag_kernel_lg(int lg, bool index64, bool a64) {
  switch (lg) {
#define TBE_NOBAG_CASE(L)                                                                \
    case L:                                                                              \
      if (a64) return index64 ? nobag_fast_kernel<WT, L, int64_t, true> : nobag_fast_kernel<WT, L, int32_t, true>; \
      return index64 ? nobag_fast_kernel<WT, L, int64_t> : nobag_fast_kernel<WT, L, int32_t>;
    TBE_NOBAG_CASE(0) TBE_NOBAG_CASE(1) TBE_NOBAG_CASE(2) TBE_NOBAG_CASE(3) TBE_NOBAG_CASE(4) TBE_NOBAG_CASE(5)
#undef TBE_NOBAG_CASE
    default:
      if (a64) return index64 ? nobag_fast_kernel<WT, 6, int64_t, true> : nobag_fast_kernel<WT, 6, int32_t, true>;
      return index64 ? nobag_fast_kernel<WT, 6, int64_t> : nobag_fast_kernel<WT, 6, int32_t>;
  }
}

template <int WT>
KernelFn stream_kernel_lg(int lg, bool index64, bool weighted) {
  switch (lg) {
    case 2: return stream_kernel_for<WT, 2>(index64, weighted);
    case 3: return stream_kernel_for<WT, 3>(index64, weighted);
    case 4: return stream_kernel_for<WT, 4>(index64, weighted);
    case 5: return stream_kernel_for<WT, 5>(index64, weighted);
    default: return stream_kernel_for<WT, 6>(index64, weighted);
  }
}

}  // namespace tbe

#endif  // TBE_KERNELS_H
