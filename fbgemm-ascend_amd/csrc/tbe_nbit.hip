// tbe_nbit.hip — host side and C ABI of the quantized table-batched-embedding
// inference forward (torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function):
// planner, launcher, and the kernels that are not specialised per weight type
// (nobag, 64-bit tables).  The per-type pooled kernels live in tbe_kern_*.hip;
// the design notes are at the top of tbe_kernels.h.
//
// Reference (paths relative to the reference repository root):
//   A = src/tbe_inference/int_nbit_split_embedding_codegen_lookup_function/int_nbit_split_embedding_codegen_lookup_function.cpp
//   H = .../c310/op_host/int_nbit_split_embedding_codegen_lookup_function.cpp
//   C = .../c310/op_kernel/common.h
//   P = .../c310/op_kernel/int_nbit_split_embedding_pooling_kernel.h
//   N = .../c310/op_kernel/int_nbit_split_embedding_nobag_kernel.h
//
#include <cmath>

#include "tbe_kernels.h"

namespace tbe {

// instantiated once, in tbe_kern_<type>.hip
extern template KernelFn fast_kernel_lg<TBE_TY_FP32>(int, bool, bool, bool);
extern template KernelFn fast_kernel_a64_lg<TBE_TY_FP32>(int, bool, bool);
extern template KernelFn stream_kernel_lg<TBE_TY_FP32>(int, bool, bool);
extern template KernelFn nobag_kernel_lg<TBE_TY_FP32>(int, bool, bool);
extern template KernelFn fast_kernel_lg<TBE_TY_FP16>(int, bool, bool, bool);
extern template KernelFn fast_kernel_a64_lg<TBE_TY_FP16>(int, bool, bool);
extern template KernelFn stream_kernel_lg<TBE_TY_FP16>(int, bool, bool);
extern template KernelFn nobag_kernel_lg<TBE_TY_FP16>(int, bool, bool);
extern template KernelFn fast_kernel_lg<TBE_TY_BF16>(int, bool, bool, bool);
extern template KernelFn fast_kernel_a64_lg<TBE_TY_BF16>(int, bool, bool);
extern template KernelFn stream_kernel_lg<TBE_TY_BF16>(int, bool, bool);
extern template KernelFn nobag_kernel_lg<TBE_TY_BF16>(int, bool, bool);
extern template KernelFn fast_kernel_lg<TBE_TY_FP8>(int, bool, bool, bool);
extern template KernelFn fast_kernel_a64_lg<TBE_TY_FP8>(int, bool, bool);
extern template KernelFn stream_kernel_lg<TBE_TY_FP8>(int, bool, bool);
extern template KernelFn nobag_kernel_lg<TBE_TY_FP8>(int, bool, bool);
extern template KernelFn fast_kernel_lg<TBE_TY_INT8>(int, bool, bool, bool);
extern template KernelFn fast_kernel_a64_lg<TBE_TY_INT8>(int, bool, bool);
extern template KernelFn stream_kernel_lg<TBE_TY_INT8>(int, bool, bool);
extern template KernelFn nobag_kernel_lg<TBE_TY_INT8>(int, bool, bool);
extern template KernelFn fast_kernel_lg<TBE_TY_INT4>(int, bool, bool, bool);
extern template KernelFn fast_kernel_a64_lg<TBE_TY_INT4>(int, bool, bool);
extern template KernelFn stream_kernel_lg<TBE_TY_INT4>(int, bool, bool);
extern template KernelFn nobag_kernel_lg<TBE_TY_INT4>(int, bool, bool);
extern template KernelFn fast_kernel_lg<TBE_TY_INT2>(int, bool, bool, bool);
extern template KernelFn fast_kernel_a64_lg<TBE_TY_INT2>(int, bool, bool);
extern template KernelFn stream_kernel_lg<TBE_TY_INT2>(int, bool, bool);
extern template KernelFn nobag_kernel_lg<TBE_TY_INT2>(int, bool, bool);

// ---------------------------------------------------------------- nobag (pooling_mode NONE)

// Rows [i0, i1) of the global index array, all belonging to table td: output row i
// is the dequantized row of indices[i] (N:224-300).  Generic path of tables beyond
// 32-bit addressing (64-bit addresses, runtime lanes per row).
template <int WT>
__device__ __forceinline__ void nobag_rows(const KParams& p, const TbeTableDesc& td, int64_t i0, int64_t i1) {
  constexpr int E = Traits<WT>::kEpd;
  constexpr bool HDR = Traits<WT>::kHdr;
  const int lane = threadIdx.x & (kWave - 1);
  const int lg = td.log2_lanes;
  const int R = kWave >> lg;
  const int slot = lane >> lg;
  const uint8_t* tbase = p.weights + td.weights_offset;
  for (int ct = 0; ct < td.col_tiles; ++ct) {
    const int dw = ct * kWave + (lane & ((1 << lg) - 1));
    const bool col_ok = dw < td.data_dwords;
    for (int64_t r0 = i0; r0 < i1; r0 += R) {
      const int64_t i = r0 + slot;
      if (i >= i1 || !col_ok) continue;
      const int64_t idx = load_index(p, p.indices, i);
      float v[E];
      float s = 1.f, bi = 0.f;
      if (idx >= 0 && idx < td.num_rows) {
        const uint8_t* row = tbase + idx * td.row_stride;
        decode<WT>(load_word(row + td.data_offset + 4 * dw), v, p.fp8);
        if constexpr (HDR) {
          const uint32_t h = load_word(row);
          s = h16lo(h);
          bi = h16hi(h);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = 0.f;
        s = 0.f;
      }
      float r[E];
#pragma unroll
      for (int e = 0; e < E; ++e) r[e] = HDR ? fmaf(s, v[e], bi) : v[e];
      store_out<E>(p, i * p.out_stride + static_cast<int64_t>(dw) * E, r);
    }
  }
}

__global__ __launch_bounds__(kBlock) void nobag_kernel(KParams p) {
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
    // done by the group's specialised kernel (32-bit offsets or 64-bit row addresses)
    if ((td.flags & TBE_TABLE_OFFSET32) || td.num_rows < static_cast<int64_t>(kNoRow64)) continue;
    switch (td.weight_ty) {
      case TBE_TY_INT4: nobag_rows<TBE_TY_INT4>(p, td, a, e); break;
      case TBE_TY_INT8: nobag_rows<TBE_TY_INT8>(p, td, a, e); break;
      case TBE_TY_INT2: nobag_rows<TBE_TY_INT2>(p, td, a, e); break;
      case TBE_TY_FP8:  nobag_rows<TBE_TY_FP8>(p, td, a, e); break;
      case TBE_TY_FP16: nobag_rows<TBE_TY_FP16>(p, td, a, e); break;
      case TBE_TY_BF16: nobag_rows<TBE_TY_BF16>(p, td, a, e); break;
      case TBE_TY_FP32: nobag_rows<TBE_TY_FP32>(p, td, a, e); break;
      default: break;
    }
  }
}

// ---------------------------------------------------------------- host side

thread_local std::string g_last_error;

void clear_error() { g_last_error.clear(); }

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
  c.one = 1.0f;
  if (bits < 1 || bits > 7 || bias < 0 || bias > 120) return c;
  c.shift = static_cast<uint32_t>(bits + 16);
  c.mant_bits = static_cast<uint32_t>(7 - bits);
  const uint32_t mult_bits = static_cast<uint32_t>(254 - bias) << 23;
  memcpy(&c.mult, &mult_bits, 4);
  c.sub_scale = ldexpf(1.0f, 1 - bias - (7 - bits));
  c.h16_shift = static_cast<uint32_t>(bits + 3);
  c.h16_scale = ldexpf(1.0f, 15 - bias);
  c.h16_ok = bits <= 4;
  return c;
}

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{};
  f.d = d;
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  f.shift = l;
  f.mul = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  return f;
}

// Row-stream kernel of a group (rows of >= 16 lanes, 32-bit table offsets).
KernelFn stream_kernel_group(const TbePlanGroup& g, bool index64, bool weighted) {
  switch (g.weight_ty) {
    case TBE_TY_FP32: return stream_kernel_lg<TBE_TY_FP32>(g.log2_lanes, index64, weighted);
    case TBE_TY_FP16: return stream_kernel_lg<TBE_TY_FP16>(g.log2_lanes, index64, weighted);
    case TBE_TY_BF16: return stream_kernel_lg<TBE_TY_BF16>(g.log2_lanes, index64, weighted);
    case TBE_TY_FP8:  return stream_kernel_lg<TBE_TY_FP8>(g.log2_lanes, index64, weighted);
    case TBE_TY_INT8: return stream_kernel_lg<TBE_TY_INT8>(g.log2_lanes, index64, weighted);
    case TBE_TY_INT4: return stream_kernel_lg<TBE_TY_INT4>(g.log2_lanes, index64, weighted);
    default:          return stream_kernel_lg<TBE_TY_INT2>(g.log2_lanes, index64, weighted);
  }
}

// Groups of at least this many (table, sample, column tile) items use the
// row-stream kernel by default.
constexpr int64_t kStreamMinBags = int64_t(1) << 20;

// Rows a wave of the row-stream kernel should walk: measured on 200 INT4 tables x
// 32768 bags of ~40 rows, 32 bags per wave (1280 rows) ran 3.14 ms, 24 or 40 bags
// 3.16 ms, 63 bags 3.20 ms and 16 bags 3.27 ms.
constexpr int64_t kStreamRowsPerWave = 1280;

// Bags per wave of the row-stream kernel for a group of `bags` (table, sample)
// pairs: enough waves for about `rounds` waves per resident wave slot, so the
// hardware balances the waves' uneven run times, and no more bags than hold about
// kStreamRowsPerWave rows at the call's mean bag length, within [4, 63] bags.
// TBE_STREAM_BAGS_PER_WAVE / TBE_STREAM_ROUNDS override (tuning).
int stream_bags_per_wave(int64_t bags, int64_t resident_waves, double rows_per_bag) {
  static const int fixed = [] {
    const char* e = getenv("TBE_STREAM_BAGS_PER_WAVE");
    const int x = e ? atoi(e) : 0;
    return (x >= 1 && x <= kMaxBagsPerWave) ? x : 0;
  }();
  static const int rounds = [] {
    const char* e = getenv("TBE_STREAM_ROUNDS");
    const int x = e ? atoi(e) : 0;
    return x >= 1 ? x : 3;
  }();
  if (fixed) return fixed;
  // enough waves for `rounds` rounds of the resident ones, and about
  // kStreamRowsPerWave rows per wave
  const int64_t want = std::max<int64_t>(1, resident_waves) * rounds;
  int64_t bpw = (bags + want - 1) / want;
  if (rows_per_bag > 0)
    bpw = std::min<int64_t>(bpw, static_cast<int64_t>(std::ceil(kStreamRowsPerWave / rows_per_bag)));
  return static_cast<int>(std::min<int64_t>(kMaxBagsPerWave, std::max<int64_t>(4, bpw)));
}

// Specialised nobag kernel of a 32-bit group.
KernelFn nobag_kernel_group(const TbePlanGroup& g, bool index64) {
  switch (g.weight_ty) {
    case TBE_TY_FP32: return nobag_kernel_lg<TBE_TY_FP32>(g.log2_lanes, index64, !g.offset32);
    case TBE_TY_FP16: return nobag_kernel_lg<TBE_TY_FP16>(g.log2_lanes, index64, !g.offset32);
    case TBE_TY_BF16: return nobag_kernel_lg<TBE_TY_BF16>(g.log2_lanes, index64, !g.offset32);
    case TBE_TY_FP8:  return nobag_kernel_lg<TBE_TY_FP8>(g.log2_lanes, index64, !g.offset32);
    case TBE_TY_INT8: return nobag_kernel_lg<TBE_TY_INT8>(g.log2_lanes, index64, !g.offset32);
    case TBE_TY_INT4: return nobag_kernel_lg<TBE_TY_INT4>(g.log2_lanes, index64, !g.offset32);
    default:          return nobag_kernel_lg<TBE_TY_INT2>(g.log2_lanes, index64, !g.offset32);
  }
}

KernelFn pooled_kernel_for(const TbePlanGroup& g, bool index64, bool weighted, bool wide, bool wide_words) {
  if (wide || g.weight_ty < 0) return weighted ? pooled_wide_kernel<true> : pooled_wide_kernel<false>;
  if (!g.offset32) {  // past 32-bit byte offsets: 64-bit row addresses
    switch (g.weight_ty) {
      case TBE_TY_FP32: return fast_kernel_a64_lg<TBE_TY_FP32>(g.log2_lanes, index64, weighted);
      case TBE_TY_FP16: return fast_kernel_a64_lg<TBE_TY_FP16>(g.log2_lanes, index64, weighted);
      case TBE_TY_BF16: return fast_kernel_a64_lg<TBE_TY_BF16>(g.log2_lanes, index64, weighted);
      case TBE_TY_FP8:  return fast_kernel_a64_lg<TBE_TY_FP8>(g.log2_lanes, index64, weighted);
      case TBE_TY_INT8: return fast_kernel_a64_lg<TBE_TY_INT8>(g.log2_lanes, index64, weighted);
      case TBE_TY_INT4: return fast_kernel_a64_lg<TBE_TY_INT4>(g.log2_lanes, index64, weighted);
      default:          return fast_kernel_a64_lg<TBE_TY_INT2>(g.log2_lanes, index64, weighted);
    }
  }
  switch (g.weight_ty) {
    case TBE_TY_FP32: return fast_kernel_lg<TBE_TY_FP32>(g.log2_lanes, index64, weighted, wide_words);
    case TBE_TY_FP16: return fast_kernel_lg<TBE_TY_FP16>(g.log2_lanes, index64, weighted, wide_words);
    case TBE_TY_BF16: return fast_kernel_lg<TBE_TY_BF16>(g.log2_lanes, index64, weighted, wide_words);
    case TBE_TY_FP8:  return fast_kernel_lg<TBE_TY_FP8>(g.log2_lanes, index64, weighted, wide_words);
    case TBE_TY_INT8: return fast_kernel_lg<TBE_TY_INT8>(g.log2_lanes, index64, weighted, wide_words);
    case TBE_TY_INT4: return fast_kernel_lg<TBE_TY_INT4>(g.log2_lanes, index64, weighted, wide_words);
    default:          return fast_kernel_lg<TBE_TY_INT2>(g.log2_lanes, index64, weighted, wide_words);
  }
}

// Blocks of `fn` the whole GPU keeps resident at once (cached per device and kernel).
int resident_blocks(KernelFn fn) {
  static std::mutex mu;
  static std::vector<std::pair<std::pair<int, KernelFn>, int>> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> g(mu);
  for (auto& e : cache)
    if (e.first.first == dev && e.first.second == fn) return e.second;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(fn), kBlock, 0) !=
      hipSuccess)
    return 0;
  const int blocks = std::max(1, cus * per_cu);
  cache.push_back({{dev, fn}, blocks});
  return blocks;
}

// Streams that run a forward's table groups side by side: the groups write
// disjoint output columns, and a persistent kernel's tail (its last waves)
// leaves most of the GPU idle while the next group's kernel would wait behind
// it on one stream.  One set per (device, caller stream), default priority,
// ordered against the caller's stream with events (fork before, join after), so
// the call stays asynchronous, calls on independent caller streams stay
// independent, and a caller stream under graph capture brings only its own
// side streams into the capture.  Sets are kept until the process ends; past
// kMaxStreamSets caller streams on one device, further streams run their
// groups serially on the caller's stream.
// Two streams measured best on config 3 (14 groups): 0.854 ms serial, 0.782 ms
// with 2, 0.814 ms with 4, 0.810 ms with 8.
constexpr int kGroupStreams = 2;
constexpr int kMaxStreamSets = 32;

struct GroupStreams {
  int dev = -1;
  hipStream_t caller = nullptr;
  bool ok = false;
  std::mutex mu;
  hipStream_t st[kGroupStreams] = {};
  hipEvent_t fork = nullptr;
  hipEvent_t join[kGroupStreams] = {};
};

GroupStreams* group_streams(hipStream_t caller) {
  static std::mutex mu;
  static std::vector<GroupStreams*> all;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> g(mu);
  int on_dev = 0;
  for (GroupStreams* e : all) {
    if (e->dev != dev) continue;
    if (e->caller == caller) return e->ok ? e : nullptr;
    ++on_dev;
  }
  if (on_dev >= kMaxStreamSets) return nullptr;
  GroupStreams* e = new GroupStreams();  // kept until the process ends
  e->dev = dev;
  e->caller = caller;
  bool ok = hipEventCreateWithFlags(&e->fork, hipEventDisableTiming) == hipSuccess;
  for (int i = 0; ok && i < kGroupStreams; ++i)
    ok = hipStreamCreateWithFlags(&e->st[i], hipStreamNonBlocking) == hipSuccess &&
         hipEventCreateWithFlags(&e->join[i], hipEventDisableTiming) == hipSuccess;
  e->ok = ok;
  all.push_back(e);
  return ok ? e : nullptr;
}

// Persistent launches hold what the GPU keeps resident; with at least kOverItems items per
// wave of a twice-as-large grid, the grid is doubled: waves then finish in two rounds and
// the hardware hands the second round to the CUs that finished first.  The waves of a
// persistent grid end 40 % apart (the memory side serves CUs unevenly); measured on
// configuration 2 (213 k bags, 5,120 resident waves): 121.2 -> 119.3 µs; with fewer items
// per wave the second round's set-up costs more than it saves (configuration 1: 13 bags
// per resident wave, 43.8 -> 46.2 µs with a doubled grid).
constexpr int64_t kOverItems = 20;

hipError_t launch(KernelFn fn, KParams& p, int64_t want_blocks, bool persistent, hipStream_t s) {
  int64_t blocks = want_blocks;
  if (persistent) {
    const int cap = resident_blocks(fn);
    if (cap > 0) {
      const int64_t items = static_cast<int64_t>(p.num_items);
      const int over = items >= 2 * static_cast<int64_t>(cap) * kWavesPerBlock * kOverItems ? 2 : 1;
      blocks = std::min<int64_t>(blocks, static_cast<int64_t>(cap) * over);
    }
  }
  blocks = std::max<int64_t>(1, blocks);
  void* args[] = {&p};
  return hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3(static_cast<uint32_t>(blocks)), dim3(kBlock),
                         args, 0, s);
}

}  // namespace tbe

using namespace tbe;

extern "C" {

const char* tbe_last_error(void) { return g_last_error.c_str(); }

int tbe_nbit_abi_version(void) { return TBE_NBIT_ABI_VERSION; }

int tbe_nbit_plan(const TbePlanInput* in, TbeTableDesc* descs, int32_t* table_order, TbePlanSummary* summary) {
  g_last_error.clear();
  if (!in || !descs || !table_order || !summary) return fail(TBE_ERR_INVALID_ARG, "null argument to tbe_nbit_plan");
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
    // a zero-width table would have a zero row stride (FP rows) and no column to pool
    if (D == 0) return fail(TBE_ERR_INVALID_ARG, "table %d: D must be positive (D_offsets[%d] == D_offsets[%d])", t,
                            t, t + 1);
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
    if (descs[t].num_rows * descs[t].row_stride <= static_cast<int64_t>(kNoRow)) descs[t].flags |= TBE_TABLE_OFFSET32;
    // row-stream kernel: at least 4 lanes per slot, whole lane loads
    const int vw = stream_vw_of(descs[t].weight_ty, descs[t].log2_lanes);
    if ((descs[t].flags & TBE_TABLE_OFFSET32) && (1 << descs[t].log2_lanes) >= 4 * vw &&
        descs[t].data_dwords % vw == 0)
      descs[t].flags |= TBE_TABLE_STREAM;
  }
  if (has_fp8) {
    const int eb = in->fp8_exponent_bits, bias = in->fp8_exponent_bias;
    if (eb < 1 || eb > 7 || bias < 0 || bias > 120)
      return fail(TBE_ERR_INVALID_ARG, "FP8 tables need fp8_exponent_bits in [1,7] and bias in [0,120] (got %d, %d)",
                  eb, bias);
  }
  s.has_fp8 = has_fp8;
  // group tables by kernel specialisation; table order is kept inside a group so
  // that the XCD split of a group's bags still follows table boundaries
  auto key = [&](int t) {
    const TbeTableDesc& d = descs[t];
    const bool o32 = d.flags & TBE_TABLE_OFFSET32;
    const bool st = d.flags & TBE_TABLE_STREAM;
    const int shape = d.weight_ty * 8 + d.log2_lanes;
    // tables past 32-bit byte offsets: per shape while rows fit a 32-bit index
    // (64-bit addresses in the per-bag kernel), else one generic group
    if (!o32) return d.num_rows < static_cast<int64_t>(kNoRow64) ? 1000 + shape : 100000;
    return shape * 2 + st;
  };
  std::vector<int32_t> order(T);
  for (int t = 0; t < T; ++t) order[t] = t;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return key(a) < key(b); });
  s.num_groups = 0;
  for (int i = 0; i < T;) {
    int j = i;
    int tiles = 1;
    while (j < T && key(order[j]) == key(order[i])) {
      tiles = std::max<int>(tiles, descs[order[j]].col_tiles);
      ++j;
    }
    if (s.num_groups >= TBE_MAX_GROUPS) return fail(TBE_ERR_UNSUPPORTED, "too many table groups");
    TbePlanGroup& g = s.groups[s.num_groups++];
    const TbeTableDesc& d0 = descs[order[i]];
    g.offset32 = (d0.flags & TBE_TABLE_OFFSET32) ? 1 : 0;
    const bool generic = key(order[i]) == 100000;
    g.weight_ty = generic ? -1 : d0.weight_ty;
    g.log2_lanes = generic ? -1 : d0.log2_lanes;
    g.stream = (d0.flags & TBE_TABLE_STREAM) ? 1 : 0;
    g.first = i;
    g.count = j - i;
    g.col_tiles = tiles;
    i = j;
  }
  memcpy(table_order, order.data(), sizeof(int32_t) * T);
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
  if (static_cast<int64_t>(a->T) * a->B * a->max_col_tiles > 0x7FFFFFFF)
    return fail(TBE_ERR_UNSUPPORTED, "too many bags for one call (T*B*col_tiles >= 2^31)");
  const int64_t nbags = static_cast<int64_t>(a->T) * a->B;
  if (a->pooling_mode == TBE_POOL_NONE ? a->num_indices == 0 : nbags == 0) return TBE_OK;
  if (!a->dev_weights || !a->tables || !a->offsets || !a->output || !a->plan)
    return fail(TBE_ERR_INVALID_ARG, "null pointer argument");
  if (a->num_indices > 0 && !a->indices) return fail(TBE_ERR_INVALID_ARG, "null indices");

  KParams p{};
  p.weights = a->dev_weights;
  p.tables = a->tables;
  p.order = a->table_order;
  p.indices = a->indices;
  p.offsets = a->offsets;
  p.psw = a->indice_weights;
  p.out = a->output;
  p.out_stride = a->output_stride;
  p.num_indices = a->num_indices;
  p.B = static_cast<int32_t>(a->B);
  p.T = a->T;
  p.index64 = a->index_size == 8;
  p.out_ty = a->output_dtype;
  p.mean = a->pooling_mode == TBE_POOL_MEAN;
  p.xcd = (a->flags & TBE_FLAG_NO_XCD_REMAP) ? 0 : 1;
  p.fp8 = make_fp8(a->fp8_exponent_bits, a->fp8_exponent_bias);
  p.div_B = make_fastdiv(static_cast<uint32_t>(std::max<int64_t>(a->B, 1)));
  hipStream_t s = static_cast<hipStream_t>(hip_stream);

  if (a->pooling_mode == TBE_POOL_NONE) {
    const int64_t chunks = (a->num_indices + kWave - 1) / kWave;
    if (chunks > 0x7FFFFFFF) return fail(TBE_ERR_UNSUPPORTED, "too many indices for one launch");
    p.num_items = static_cast<int32_t>(chunks);
    p.order = nullptr;
    const TbePlanSummary& plan = *a->plan;
    if (plan.num_groups < 1 || plan.num_groups > TBE_MAX_GROUPS) return fail(TBE_ERR_INVALID_ARG, "bad plan");
    // one launch per table group: each (type, lanes per row) group takes its
    // specialised kernel (32-bit offsets or 64-bit row addresses), which skips other
    // tables' segments; tables of 2^32 - 1 rows or more take the generic kernel
    // the first launch also zeroes the rows of positions outside every segment
    bool generic = false;
    p.zero_gaps = 1;
    for (int gi = 0; gi < plan.num_groups; ++gi) {
      const TbePlanGroup& g = plan.groups[gi];
      if (g.weight_ty < 0) {
        generic = true;
        continue;
      }
      const hipError_t err = launch(nobag_kernel_group(g, p.index64 != 0), p,
                                    (chunks + kWavesPerBlock - 1) / kWavesPerBlock, false, s);
      if (err != hipSuccess) return fail(TBE_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
      p.zero_gaps = 0;
    }
    if (generic) {
      const hipError_t err = launch(nobag_kernel, p, (chunks + kWavesPerBlock - 1) / kWavesPerBlock, false, s);
      if (err != hipSuccess) return fail(TBE_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
    }
    return TBE_OK;
  }

  if (!a->table_order) return fail(TBE_ERR_INVALID_ARG, "null table_order");
  const TbePlanSummary& plan = *a->plan;
  if (plan.num_groups < 1 || plan.num_groups > TBE_MAX_GROUPS) return fail(TBE_ERR_INVALID_ARG, "bad plan");
  for (int gi = 0; gi < plan.num_groups; ++gi) {
    const TbePlanGroup& g = plan.groups[gi];
    if (g.count <= 0 || g.first < 0 || g.first + g.count > a->T || g.col_tiles < 1 || g.col_tiles > 255)
      return fail(TBE_ERR_INVALID_ARG, "bad plan group %d", gi);
  }
  const bool weighted = a->indice_weights != nullptr;
  // the per-group kernels keep index positions in 32 bits
  const bool wide = a->num_indices > 0x7FFFFFFF;
  // several groups: launch them on the group streams, between a fork and a join
  GroupStreams* gs = (plan.num_groups > 1 && !(a->flags & TBE_FLAG_SERIAL_GROUPS)) ? group_streams(s) : nullptr;
  std::unique_lock<std::mutex> gs_lock;
  int used = 0;
  if (gs) {
    gs_lock = std::unique_lock<std::mutex>(gs->mu);
    if (hipEventRecord(gs->fork, s) != hipSuccess) return fail(TBE_ERR_LAUNCH, "fork event failed");
    for (int i = 0; i < std::min(kGroupStreams, plan.num_groups); ++i, ++used)
      if (hipStreamWaitEvent(gs->st[i], gs->fork, 0) != hipSuccess) break;
    if (used == 0) return fail(TBE_ERR_LAUNCH, "fork wait failed");
  }
  // Groups in decreasing estimated cost, each on the group stream with the least
  // cost so far (longest-processing-time-first), so the streams finish together.
  // Cost ~ tables x (lane words of a row + a per-bag constant); bag lengths are on
  // the device and are not read.  Groups write disjoint output columns, so the
  // assignment does not change results.
  int gorder[TBE_MAX_GROUPS];
  int gsid[TBE_MAX_GROUPS];
  {
    int64_t cost[TBE_MAX_GROUPS];
    for (int gi = 0; gi < plan.num_groups; ++gi) {
      const TbePlanGroup& g = plan.groups[gi];
      cost[gi] = static_cast<int64_t>(g.count) * ((int64_t(4) << std::max(0, std::min(g.log2_lanes, 6))) *
                                                     std::max(1, g.col_tiles) + 64);
      gorder[gi] = gi;
    }
    std::stable_sort(gorder, gorder + plan.num_groups, [&](int x, int y) { return cost[x] > cost[y]; });
    int64_t load[kGroupStreams] = {};
    for (int k = 0; k < plan.num_groups; ++k) {
      int best = 0;
      for (int i = 1; i < used; ++i)
        if (load[i] < load[best]) best = i;
      gsid[gorder[k]] = best;
      load[best] += cost[gorder[k]];
    }
  }
  hipError_t err = hipSuccess;
  for (int k = 0; k < plan.num_groups && err == hipSuccess; ++k) {
    const int gi = gorder[k];
    const hipStream_t gstream = gs ? gs->st[gsid[gi]] : s;
    const TbePlanGroup& g = plan.groups[gi];
    p.group_first = g.first;
    p.group_count = g.count;
    p.col_tiles = g.col_tiles;
    p.div_tiles = make_fastdiv(static_cast<uint32_t>(g.col_tiles));
    // row streams pay off on large groups (measured: 200 tables x 32768 bags, 25 %
    // faster); the per-bag kernel is as fast or faster below about a million bags
    const int64_t group_bags = static_cast<int64_t>(g.count) * a->B * g.col_tiles;
    const bool use_stream = g.stream && !(a->flags & TBE_FLAG_NO_STREAM) &&
                            ((a->flags & TBE_FLAG_FORCE_STREAM) || group_bags >= kStreamMinBags);
    if (!wide && use_stream) {
      // one wave per (table, range of bags, column tile), no persistence
      const KernelFn fn = stream_kernel_group(g, p.index64 != 0, weighted);
      const double rows_per_bag = static_cast<double>(a->num_indices) / static_cast<double>(std::max<int64_t>(1, a->T * a->B));
      p.bags_per_wave = stream_bags_per_wave(group_bags,
                                             static_cast<int64_t>(resident_blocks(fn)) * kWavesPerBlock, rows_per_bag);
      p.ranges = static_cast<int32_t>((a->B + p.bags_per_wave - 1) / p.bags_per_wave);
      p.div_ranges = make_fastdiv(static_cast<uint32_t>(p.ranges));
      const int64_t items = static_cast<int64_t>(g.count) * p.ranges * g.col_tiles;
      p.num_items = static_cast<int32_t>(items);
      err = launch(fn, p, (items + kWavesPerBlock - 1) / kWavesPerBlock, false, gstream);
    } else {
      const int64_t items = static_cast<int64_t>(g.count) * a->B * g.col_tiles;
      p.num_items = static_cast<int32_t>(items);
      // progress-ordered wave priority only when this group's kernel runs alone
      p.xcd = (p.xcd & 1) | (plan.num_groups == 1 ? 2 : 0);
      // two words per lane when every table of the group has an even word count
      const bool wide_words = g.stream && !(a->flags & TBE_FLAG_NARROW_WORDS);
      err = launch(pooled_kernel_for(g, p.index64 != 0, weighted, wide, wide_words), p,
                   (items + kWavesPerBlock - 1) / kWavesPerBlock, true, gstream);
    }
  }
  // join even after a failed launch, so the caller's stream still waits for the
  // groups already queued before it frees or reuses the output
  bool joined = true;
  for (int i = 0; i < used; ++i)
    if (hipEventRecord(gs->join[i], gs->st[i]) != hipSuccess || hipStreamWaitEvent(s, gs->join[i], 0) != hipSuccess)
      joined = false;
  if (err != hipSuccess) return fail(TBE_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
  if (!joined) return fail(TBE_ERR_LAUNCH, "join of the group streams failed");
  return TBE_OK;
}

}  // extern "C"
