/*
 * tbe_oracle.c — CPU restatement of the reference's quantized TBE inference
 * forward.  TEST INFRASTRUCTURE ONLY: the GPU product never links, loads or
 * calls this file.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker (and the timed CPU baseline).
 *
 * Citations are relative to the reference repository root.
 *   A = src/tbe_inference/int_nbit_split_embedding_codegen_lookup_function/
 *       int_nbit_split_embedding_codegen_lookup_function.cpp
 *   C = .../c310/op_kernel/common.h
 *   P = .../c310/op_kernel/int_nbit_split_embedding_pooling_kernel.h
 *   N = .../c310/op_kernel/int_nbit_split_embedding_nobag_kernel.h
 *   R = .../c310/README.md
 *
 * The reference device kernel implements FP8 rows only (P:226-232); the
 * INT8/INT4/INT2/FP16/FP32 row formats follow the upstream fbgemm_gpu layout
 * that the reference's test uses as its golden (fbgemm_gpu 1.2.0, not vendored):
 * INT rows are [fp16 scale][fp16 bias][packed codes], codes packed low bits
 * first, row length rounded up to row_alignment bytes; value = scale*q + bias.
 *
 * Order of operations per bag (P:346-394, P:282-315): fp32 accumulator,
 * rows added in index order, weighted rows as acc += w*row, MEAN multiplies by
 * float(1)/float(L) after the last row (P:355, P:307-310), then the cast to the
 * output dtype with round-to-nearest-even (P:330, CAST_RINT).
 *
 * Beyond the reference: an index outside [0, rows of its table) contributes
 * nothing (fbgemm_gpu's pruned-row convention for -1); MEAN still divides by L.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { TY_FP32 = 0, TY_FP16 = 1, TY_INT8 = 2, TY_INT4 = 3, TY_INT2 = 4, TY_BF16 = 5, TY_FP8 = 6 };

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* IEEE binary16 -> binary32, exact (every half is representable). */
float oracle_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u;
  int32_t exp = (h >> 10) & 0x1F;
  uint32_t mant = h & 0x3FFu;
  float mag;
  if (exp == 0) {
    mag = ldexpf((float)mant, -24); /* subnormal: mant * 2^-24 */
  } else if (exp == 31) {
    mag = mant ? NAN : INFINITY;
  } else {
    mag = ldexpf((float)(mant | 0x400u), exp - 25); /* (1024+mant) * 2^(exp-15-10) */
  }
  return sign ? -mag : mag;
}

/* binary32 -> binary16, round to nearest, ties to even. */
uint16_t oracle_float_to_half(float f) {
  uint32_t u = f32_to_bits(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t aexp = (u >> 23) & 0xFFu;
  uint32_t mant = u & 0x7FFFFFu;
  if (aexp == 0xFF) return sign | (mant ? 0x7E00u : 0x7C00u);
  float a = fabsf(f);
  if (a >= 65520.0f) return sign | 0x7C00u; /* rounds to infinity */
  if (a < ldexpf(1.0f, -14)) {
    /* subnormal half: value = k * 2^-24, k = rint(a * 2^24) (exact scaling) */
    float k = nearbyintf(a * 16777216.0f); /* default rounding mode: ties-to-even */
    return sign | (uint16_t)k;             /* k == 1024 becomes the smallest normal */
  }
  int e = (int)aexp - 127;           /* a in [2^e, 2^(e+1)), e in [-14, 15] */
  float scaled = ldexpf(a, 10 - e);  /* in [1024, 2048), exact */
  float k = nearbyintf(scaled);      /* ties-to-even */
  uint32_t ki = (uint32_t)k;
  if (ki == 2048u) { ki = 1024u; e += 1; }
  if (e > 15) return sign | 0x7C00u;
  return sign | (uint16_t)(((uint32_t)(e + 15) << 10) | (ki - 1024u));
}

/* binary32 -> bfloat16, round to nearest, ties to even (NaN kept quiet). */
uint16_t oracle_float_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

/* FP8 code -> fp32 with exponent_bits / exponent_bias, restating C:120-167:
 * body bits shifted into the fp32 exponent/mantissa field, multiplied by
 * 2^(127-bias), sign OR-ed back in.  Subnormal codes (exponent field 0) are
 * computed here as body * 2^(1-bias-m) so the result never depends on the
 * host's handling of fp32 denormal operands. */
float oracle_fp8_to_float(uint8_t code, int exp_bits, int exp_bias) {
  int m = 7 - exp_bits;
  uint32_t body = code & 0x7Fu;
  float v;
  if ((body >> m) == 0) {
    v = ldexpf((float)body, 1 - exp_bias - m);
  } else {
    float raw = bits_to_f32(body << (exp_bits + 16)); /* C:126, C:162-163 */
    float mult = bits_to_f32((uint32_t)(254 - exp_bias) << 23); /* C:131 */
    v = raw * mult;                                              /* C:165 */
  }
  return bits_to_f32(f32_to_bits(v) | ((uint32_t)(code & 0x80u) << 24)); /* C:166 */
}

static int bits_of(int ty) {
  switch (ty) {
    case TY_FP32: return 32;
    case TY_FP16: case TY_BF16: return 16;
    case TY_INT8: case TY_FP8: return 8;
    case TY_INT4: return 4;
    case TY_INT2: return 2;
    default: return 0;
  }
}

/* Bytes of one row before padding (fbgemm_gpu layout, and P:241 for FP8). */
int64_t oracle_unpadded_row_bytes(int ty, int64_t D) {
  int b = bits_of(ty);
  int64_t payload = (D * b + 7) / 8;
  int hdr = (ty == TY_INT8 || ty == TY_INT4 || ty == TY_INT2) ? 4 : 0;
  return payload + hdr;
}

int64_t oracle_row_stride(int ty, int64_t D, int64_t row_alignment) {
  int64_t u = oracle_unpadded_row_bytes(ty, D);
  return (u + row_alignment - 1) / row_alignment * row_alignment; /* P:241 */
}

/* Dequantize element d of one row. */
static float dequant(const uint8_t* row, int ty, int64_t d, int fp8_bits, int fp8_bias) {
  switch (ty) {
    case TY_FP32: {
      float v;
      memcpy(&v, row + 4 * d, 4);
      return v;
    }
    case TY_FP16: {
      uint16_t h;
      memcpy(&h, row + 2 * d, 2);
      return oracle_half_to_float(h);
    }
    case TY_BF16: {
      uint16_t h;
      memcpy(&h, row + 2 * d, 2);
      return bits_to_f32((uint32_t)h << 16);
    }
    case TY_FP8:
      return oracle_fp8_to_float(row[d], fp8_bits, fp8_bias);
    default: break;
  }
  uint16_t sh, bh;
  memcpy(&sh, row, 2);
  memcpy(&bh, row + 2, 2);
  float scale = oracle_half_to_float(sh), bias = oracle_half_to_float(bh);
  const uint8_t* q = row + 4;
  uint32_t code;
  if (ty == TY_INT8) code = q[d];
  else if (ty == TY_INT4) code = (q[d >> 1] >> (4 * (d & 1))) & 0xFu;
  else code = (q[d >> 2] >> (2 * (d & 3))) & 0x3u;
  return fmaf(scale, (float)code, bias);
}

static void store_out(void* out, int out_ty, int64_t pos, float v) {
  if (out_ty == TY_FP32) ((float*)out)[pos] = v;
  else if (out_ty == TY_FP16) ((uint16_t*)out)[pos] = oracle_float_to_half(v);
  else ((uint16_t*)out)[pos] = oracle_float_to_bf16(v);
}

static int64_t load_index(const void* p, int index_size, int64_t i) {
  return index_size == 8 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

/*
 * The op.  Host arrays throughout.  Returns 0, or -1 on an argument error.
 *   table_rows[t]: rows of table t that may be addressed (indices outside are skipped).
 *   out:     [B, total_D] (bag) or [N, max_D] (nobag) in out_ty; when out_f32 is
 *            non-NULL the fp32 value before the cast is stored there too.
 * Bag decomposition (P:44-85, R:40-57): bag k = t*B + b covers
 * indices[offsets[k], offsets[k+1]) and writes out[b, D_offsets[t] : D_offsets[t+1]).
 * Nobag (N:44-81, A:132-146): indices of table t are offsets[t*B]..offsets[(t+1)*B];
 * out row i = dequantized row of indices[i]; columns past D stay zero.
 */
int oracle_tbe_forward(const uint8_t* weights, int T, const int64_t* weights_offsets,
                       const uint8_t* weights_tys, const int32_t* D_offsets,
                       const int64_t* table_rows, const void* indices, const void* offsets,
                       int index_size, int64_t num_indices, int64_t B, int pooling_mode,
                       const float* indice_weights, int out_ty, int64_t row_alignment,
                       int fp8_bits, int fp8_bias, void* out, float* out_f32,
                       int64_t out_stride, int num_threads) {
  if (T <= 0 || B < 0 || row_alignment <= 0) return -1;
  if (index_size != 4 && index_size != 8) return -1;
  if (out_ty != TY_FP32 && out_ty != TY_FP16 && out_ty != TY_BF16) return -1;
  if (pooling_mode < 0 || pooling_mode > 2) return -1;
  for (int t = 0; t < T; ++t)
    if (D_offsets[t + 1] - D_offsets[t] > 8192) return -1; /* acc_buf bound */
  (void)num_indices;
  if (pooling_mode == 2) {
    for (int t = 0; t < T; ++t) {
      int64_t lo = load_index(offsets, index_size, (int64_t)t * B);
      int64_t hi = load_index(offsets, index_size, (int64_t)(t + 1) * B);
      int ty = weights_tys[t];
      int64_t D = D_offsets[t + 1] - D_offsets[t];
      int64_t stride = oracle_row_stride(ty, D, row_alignment);
#pragma omp parallel for schedule(static) num_threads(num_threads)
      for (int64_t i = lo; i < hi; ++i) {
        int64_t idx = load_index(indices, index_size, i);
        int ok = idx >= 0 && idx < table_rows[t];
        const uint8_t* row = weights + weights_offsets[t] + (ok ? idx : 0) * stride;
        for (int64_t d = 0; d < out_stride; ++d) {
          float v = (ok && d < D) ? dequant(row, ty, d, fp8_bits, fp8_bias) : 0.0f;
          store_out(out, out_ty, i * out_stride + d, v);
          if (out_f32) out_f32[i * out_stride + d] = v;
        }
      }
    }
    return 0;
  }
  int64_t nbags = (int64_t)T * B;
#pragma omp parallel num_threads(num_threads)
  {
    float acc_buf[8192];
#pragma omp for schedule(dynamic, 64)
    for (int64_t k = 0; k < nbags; ++k) {
      int t = (int)(k / B);
      int64_t b = k - (int64_t)t * B;
      int64_t start = load_index(offsets, index_size, k);
      int64_t end = load_index(offsets, index_size, k + 1);
      int32_t L = (int32_t)(end - start);
      int ty = weights_tys[t];
      int64_t D = D_offsets[t + 1] - D_offsets[t];
      int64_t stride = oracle_row_stride(ty, D, row_alignment);
      const uint8_t* tbase = weights + weights_offsets[t];
      for (int64_t d = 0; d < D; ++d) acc_buf[d] = 0.0f;
      for (int64_t i = start; i < end; ++i) {
        int64_t idx = load_index(indices, index_size, i);
        if (idx < 0 || idx >= table_rows[t]) continue;
        const uint8_t* row = tbase + idx * stride;
        if (indice_weights) {
          float w = indice_weights[i];
          for (int64_t d = 0; d < D; ++d)
            acc_buf[d] = fmaf(w, dequant(row, ty, d, fp8_bits, fp8_bias), acc_buf[d]);
        } else {
          for (int64_t d = 0; d < D; ++d) acc_buf[d] += dequant(row, ty, d, fp8_bits, fp8_bias);
        }
      }
      if (pooling_mode == 1 && L > 0) {
        float inv = (float)1 / (float)L; /* P:355 */
        for (int64_t d = 0; d < D; ++d) acc_buf[d] *= inv;
      }
      int64_t base = b * out_stride + D_offsets[t];
      for (int64_t d = 0; d < D; ++d) {
        store_out(out, out_ty, base + d, acc_buf[d]);
        if (out_f32) out_f32[base + d] = acc_buf[d];
      }
    }
  }
  return 0;
}

/* Batch helpers used by the tests to pin the element decoders exhaustively. */
void oracle_decode_fp8_table(int exp_bits, int exp_bias, float* out256) {
  for (int c = 0; c < 256; ++c) out256[c] = oracle_fp8_to_float((uint8_t)c, exp_bits, exp_bias);
}
void oracle_half_to_float_n(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_half_to_float(in[i]);
}
void oracle_float_to_half_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_float_to_half(in[i]);
}
void oracle_float_to_bf16_n(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_float_to_bf16(in[i]);
}

/*
 * permute_pooled_embs: output[:, inv[i] : inv[i+1]] = input[:, off[p] : off[p] + that
 * width], p = perm[i], for i in [0, T) (reference permute_pooled_embs.cpp:83-98,
 * the host path that builds the column list and index_selects dim 1, and the
 * kernel's segment walk permute_pooled_embs_kernel.h:173-211).  Rows are
 * [total_D, inner] elements of `es` bytes.  Beyond the reference (which does not
 * check these on its device path): a destination segment with p outside [0, T) or
 * source columns outside [0, total_D) is zero-filled; one whose own columns leave
 * [0, total_D) is left untouched.
 */
void oracle_permute_pooled_embs(const uint8_t* in, uint8_t* out, int64_t B, int64_t total_D, int64_t inner,
                                int es, int T, const int64_t* off, const int64_t* perm, const int64_t* inv) {
  const int64_t cb = inner * es;
  const int64_t rb = total_D * cb;
  for (int i = 0; i < T; ++i) {
    const int64_t dst = inv[i], dst_end = inv[i + 1];
    if (dst < 0 || dst_end < dst || dst_end > total_D) continue;
    const int64_t len = dst_end - dst;
    const int64_t p = perm[i];
    int zero = p < 0 || p >= T;
    int64_t src = 0;
    if (!zero) {
      src = off[p];
      zero = src < 0 || src + len > total_D;
    }
    for (int64_t b = 0; b < B; ++b) {
      uint8_t* o = out + b * rb + dst * cb;
      if (zero)
        memset(o, 0, (size_t)(len * cb));
      else
        memcpy(o, in + b * rb + src * cb, (size_t)(len * cb));
    }
  }
}

/*
 * block_bucketize_sparse_features (reference
 * src/sparse_ops/block_bucketize_sparse_features/block_bucketize_sparse_features.cpp:93-246
 * and c310/op_kernel/block_bucketize_sparse_features_kernel_full.h: bucket rule 387-455,
 * new index rule 560-603, sequential write cursor 730-760).
 *
 * Row r of `offsets` (inclusive cumsum of lengths, L rows) belongs to feature
 * r / (L / F), or with batch_size_offsets (complete cumsum of
 * batch_size_per_feature, F+1 entries) to the last f with bso[f] <= r.  Each index
 * of the row goes to a bucket in [0, my_size) and is written, in row order, to
 * segment (bucket, r) of the output, which starts at new_offsets[bucket*L + r]
 * (new_offsets = complete cumsum of new_lengths).  Index widths: `is` (indices,
 * block_sizes, total_num_blocks, pos lists), `os` (offsets, new_lengths,
 * batch_size_offsets), 4 or 8 bytes.  Rows of a feature with a negative block
 * size, and indices whose bucket would be >= my_size (possible only with
 * total_num_blocks not a multiple of my_size), are left out (the reference writes
 * those out of bounds).  Pass new_lengths only (new_indices NULL) to count.
 */
static int64_t ld_i(const void* p, int64_t i, int sz) {
  return sz == 8 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}
static void st_i(void* p, int64_t i, int sz, int64_t v) {
  if (sz == 8) ((int64_t*)p)[i] = v; else ((int32_t*)p)[i] = (int32_t)v;
}

static int bb_feature(int64_t r, int64_t L, int F, const void* bso, int os) {
  if (!bso) {
    const int64_t B = L / F;
    return (int)(r / (B > 0 ? B : 1));
  }
  int lo = 0, hi = F;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ld_i(bso, mid, os) <= r) lo = mid; else hi = mid - 1;
  }
  return lo;
}

/* bucket and new index of one index value; returns 0 if the index is left out */
static int bb_map(uint64_t u, int is, int64_t blk, int64_t gb, int64_t lbk, uint64_t my, int keep,
                  const void* pos, int64_t pos_len, int64_t* bucket, int64_t* nidx) {
  if (is == 4) u = (uint32_t)u;
  const uint64_t mask = is == 4 ? 0xFFFFFFFFull : ~0ull;
  if (pos && pos_len > 0) {
    uint64_t adj = u;
    if (blk == 0 && gb > 0) {
      const uint64_t scalar = ((uint64_t)ld_i(pos, pos_len - 1, is) & mask) / (uint64_t)gb;
      adj = ((u % (uint64_t)gb) * scalar) & mask;
    }
    int64_t first = 0, last = pos_len;
    while (first < last) {
      const int64_t mid = first + ((last - first) >> 1);
      if (((uint64_t)ld_i(pos, mid, is) & mask) <= adj) first = mid + 1; else last = mid;
    }
    const int64_t lb = first - 1;
    *bucket = (lb >= 0 && (uint64_t)lb < my) ? lb : (int64_t)(u % my);
    if (keep) *nidx = (int64_t)u;
    else if (blk == 0 && gb > 0) *nidx = (int64_t)(u / (uint64_t)gb);
    else if (lb >= 0 && (uint64_t)lb < my) *nidx = (int64_t)((u - ((uint64_t)ld_i(pos, lb, is) & mask)) & mask);
    else *nidx = (int64_t)(u / my);
  } else {
    const uint64_t gsize = ((uint64_t)blk * (uint64_t)gb) & mask, lsize = ((uint64_t)blk * (uint64_t)lbk) & mask;
    if (blk != 0 && u < gsize) {
      *bucket = (int64_t)(u / lsize);
      *nidx = keep ? (int64_t)u : (int64_t)(u % lsize);
    } else {
      *bucket = (int64_t)((u % (uint64_t)gb) / (uint64_t)lbk);
      *nidx = keep ? (int64_t)u : (int64_t)(u / (uint64_t)gb);
    }
  }
  return (uint64_t)*bucket < my;
}

int oracle_block_bucketize(const void* indices, int64_t n, int is, const void* offsets, int os, int64_t L,
                           const void* block_sizes, int F, int64_t my_size, const float* weights,
                           const void* bso, const void* tnb, const void* const* pos, const int64_t* pos_len,
                           int keep, void* new_lengths, const void* new_offsets, void* new_indices,
                           float* new_weights, void* new_pos, void* unbucketize_permute) {
  int64_t* cursor = NULL;
  if (new_indices) {
    cursor = (int64_t*)malloc(sizeof(int64_t) * (size_t)(my_size * L));
    if (!cursor) return -1;
    for (int64_t k = 0; k < my_size * L; ++k) cursor[k] = ld_i(new_offsets, k, os);
  } else {
    for (int64_t k = 0; k < my_size * L; ++k) st_i(new_lengths, k, os, 0);
  }
  for (int64_t r = 0; r < L; ++r) {
    const int f = bb_feature(r, L, F, bso, os);
    if (f < 0 || f >= F) continue;
    const int64_t blk = ld_i(block_sizes, f, is);
    if (blk < 0) continue;
    int64_t gb = tnb ? ld_i(tnb, f, is) : my_size;
    if (gb <= 0) gb = my_size;
    int64_t lbk = tnb ? gb / my_size : 1;
    if (lbk <= 0) lbk = 1;
    const void* pp = pos ? pos[f] : NULL;
    const int64_t pl = pos ? pos_len[f] : 0;
    int64_t s = r == 0 ? 0 : ld_i(offsets, r - 1, os), e = ld_i(offsets, r, os);
    /* clamp to the index array so malformed offsets never read out of bounds */
    s = s < 0 ? 0 : (s > n ? n : s);
    e = e < s ? s : (e > n ? n : e);
    for (int64_t i = s; i < e; ++i) {
      int64_t b, v;
      if (!bb_map((uint64_t)ld_i(indices, i, is), is, blk, gb, lbk, (uint64_t)my_size, keep, pp, pl, &b, &v))
        continue;
      const int64_t slot = b * L + r;
      if (!new_indices) {
        st_i(new_lengths, slot, os, ld_i(new_lengths, slot, os) + 1);
        continue;
      }
      const int64_t w = cursor[slot]++;
      st_i(new_indices, w, is, v);
      if (new_weights) new_weights[w] = weights[i];
      if (new_pos) st_i(new_pos, w, is, i - s);
      if (unbucketize_permute) st_i(unbucketize_permute, i, is, w);
    }
  }
  free(cursor);
  return 0;
}
