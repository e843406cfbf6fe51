// tbe_torch.cpp — PyTorch-ROCm binding of the C ABI in include/tbe_nbit.h.
//
// Registers the HIP (dispatch key CUDA on PyTorch-ROCm) implementation of
//   fbgemm::int_nbit_split_embedding_codegen_lookup_function
// with the same argument list, checks and output allocation as the reference
// adapter (reference: src/tbe_inference/int_nbit_split_embedding_codegen_lookup_function/
// int_nbit_split_embedding_codegen_lookup_function.cpp, "A" below), which
// registers the PrivateUse1 (NPU) implementation of the same schema (A:172-176).
// The schema itself is defined by the Python loader when no fbgemm_gpu
// provides it.
//
// Table metadata (weights_offsets, weights_tys, D_offsets) is planned once on
// the host and the device copy of the plan is cached, keyed on the tensors'
// addresses and version counters (each entry keeps those tensors alive): TorchRec-style modules pass the same buffers
// every call, so after the first call no host synchronisation happens.
#include <ATen/ATen.h>
#include <ATen/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>
#include <torch/library.h>

#include <limits>
#include <list>
#include <memory>
#include <mutex>
#include <tuple>
#include <vector>

#include "tbe_nbit.h"
#include "tbe_pooled_ops.h"
#include "tbe_sparse_ops.h"

namespace tbe_torch {

using at::Tensor;

// A:37-52
at::ScalarType sparse_type_to_scalar_type(int64_t output_dtype) {
  switch (output_dtype) {
    case TBE_TY_FP32: return at::kFloat;
    case TBE_TY_FP16: return at::kHalf;
    case TBE_TY_INT8: return at::kByte;
    case TBE_TY_BF16: return at::kBFloat16;
    default:
      TORCH_CHECK(false, "Unsupported output_dtype: ", output_dtype,
                  ". Supported: 0(FP32), 1(FP16), 2(INT8), 5(BF16)");
  }
}

struct PlanKey {
  const void* wo_ptr; int64_t wo_ver;
  const void* wt_ptr; int64_t wt_ver;
  const void* do_ptr; int64_t do_ver;
  int64_t T, weights_bytes, row_alignment, fp8_bits, fp8_bias;
  int device;
  bool operator==(const PlanKey& o) const {
    return std::tie(wo_ptr, wo_ver, wt_ptr, wt_ver, do_ptr, do_ver, T, weights_bytes, row_alignment,
                    fp8_bits, fp8_bias, device) ==
           std::tie(o.wo_ptr, o.wo_ver, o.wt_ptr, o.wt_ver, o.do_ptr, o.do_ver, o.T, o.weights_bytes,
                    o.row_alignment, o.fp8_bits, o.fp8_bias, o.device);
  }
};

struct Plan {
  // one device buffer: TbeTableDesc[T] followed by the int32 table order [T]
  Tensor device_plan;
  std::shared_ptr<TbePlanSummary> summary;  // host copy, handed to every forward
  const TbeTableDesc* descs() const { return reinterpret_cast<const TbeTableDesc*>(device_plan.data_ptr<uint8_t>()); }
  const int32_t* order(int64_t T) const {
    return reinterpret_cast<const int32_t*>(device_plan.data_ptr<uint8_t>() + T * sizeof(TbeTableDesc));
  }
};

class PlanCache {
 public:
  Plan get(const PlanKey& key, const Tensor& weights_offsets, const Tensor& weights_tys,
           const Tensor& D_offsets, const at::Device& dev) {
    std::lock_guard<std::mutex> g(mu_);
    for (auto it = entries_.begin(); it != entries_.end(); ++it) {
      if (it->key == key) {
        entries_.splice(entries_.begin(), entries_, it);
        return entries_.front().plan;
      }
    }
    Plan p = build(key, weights_offsets, weights_tys, D_offsets, dev);
    entries_.push_front(Entry{key, p, weights_offsets, weights_tys, D_offsets});
    if (entries_.size() > kMaxEntries) entries_.pop_back();
    return p;
  }

 private:
  static constexpr size_t kMaxEntries = 16;

  static Plan build(const PlanKey& key, const Tensor& weights_offsets, const Tensor& weights_tys,
                    const Tensor& D_offsets, const at::Device& dev) {
    // one host round trip per distinct table layout
    Tensor wo = weights_offsets.to(at::kCPU, at::kLong).contiguous();
    Tensor wt = weights_tys.to(at::kCPU, at::kByte).contiguous();
    Tensor dof = D_offsets.to(at::kCPU, at::kInt).contiguous();
    TbePlanInput in{};
    in.T = static_cast<int32_t>(key.T);
    in.weights_offsets = wo.data_ptr<int64_t>();
    in.weights_tys = wt.data_ptr<uint8_t>();
    in.D_offsets = dof.data_ptr<int32_t>();
    in.dev_weights_bytes = key.weights_bytes;
    in.row_alignment = static_cast<int32_t>(key.row_alignment);
    in.fp8_exponent_bits = static_cast<int32_t>(key.fp8_bits);
    in.fp8_exponent_bias = static_cast<int32_t>(key.fp8_bias);
    std::vector<TbeTableDesc> descs(key.T);
    std::vector<int32_t> order(key.T);
    Plan p{};
    p.summary = std::make_shared<TbePlanSummary>();
    const int rc = tbe_nbit_plan(&in, descs.data(), order.data(), p.summary.get());
    TORCH_CHECK(rc == TBE_OK, "int_nbit_split_embedding_codegen_lookup_function: ", tbe_last_error());
    const size_t dbytes = descs.size() * sizeof(TbeTableDesc), obytes = order.size() * sizeof(int32_t);
    Tensor host = at::empty({static_cast<int64_t>(dbytes + obytes)}, at::TensorOptions().dtype(at::kByte));
    memcpy(host.data_ptr<uint8_t>(), descs.data(), dbytes);
    memcpy(host.data_ptr<uint8_t>() + dbytes, order.data(), obytes);
    p.device_plan = host.to(dev);
    return p;
  }

  // An entry holds the keyed metadata tensors, so their storage (and with it the
  // addresses in the key) cannot be freed and handed to other tensors while the
  // entry lives: an address match therefore means the same tensor, and the
  // version counter catches in-place writes to it.
  struct Entry {
    PlanKey key;
    Plan plan;
    Tensor weights_offsets, weights_tys, D_offsets;
  };
  std::mutex mu_;
  std::list<Entry> entries_;
};

PlanCache& plan_cache() {
  static PlanCache c;
  return c;
}

// Same signature as the reference adapter (A:55-78).
Tensor int_nbit_split_embedding_codegen_lookup_function_hip(
    Tensor dev_weights, Tensor uvm_weights, Tensor weights_placements, Tensor weights_offsets,
    Tensor weights_tys, Tensor D_offsets, const int64_t total_D, const int64_t max_int2_D,
    const int64_t max_int4_D, const int64_t max_int8_D, const int64_t max_float16_D,
    const int64_t max_float32_D, Tensor indices, Tensor offsets, const int64_t pooling_mode,
    std::optional<Tensor> indice_weights, const int64_t output_dtype,
    std::optional<Tensor> lxu_cache_weights, std::optional<Tensor> lxu_cache_locations,
    const std::optional<int64_t> row_alignment, const std::optional<int64_t> max_float8_D,
    const std::optional<int64_t> fp8_exponent_bits, const std::optional<int64_t> fp8_exponent_bias) {
  (void)uvm_weights;
  (void)weights_placements;
  (void)lxu_cache_weights;
  (void)lxu_cache_locations;
  const at::OptionalDeviceGuard guard(at::device_of(dev_weights));  // A:80

  const int64_t T = weights_offsets.size(0);
  const int64_t N = indices.numel();
  const int64_t row_align = row_alignment.value_or(16);        // A:86
  const int64_t fp8_bits = fp8_exponent_bits.value_or(-1);     // A:87
  const int64_t fp8_bias = fp8_exponent_bias.value_or(-1);     // A:88
  const int64_t max_D = std::max({max_int2_D, max_int4_D, max_int8_D, max_float8_D.value_or(0),
                                  max_float16_D, max_float32_D});  // A:94-102

  // A:104-107 and H:110-113
  std::optional<Tensor> psw;
  if (indice_weights && indice_weights->defined() && indice_weights->numel() > 0) {
    psw = indice_weights->to(at::kFloat).contiguous();
  }
  // A:110-113: offsets follow the indices dtype
  TORCH_CHECK(indices.scalar_type() == at::kInt || indices.scalar_type() == at::kLong,
              "indices dtype must be int32 or int64, got ", indices.scalar_type());
  Tensor off = offsets.scalar_type() == indices.scalar_type() ? offsets : offsets.to(indices.scalar_type());
  off = off.contiguous();
  Tensor idx = indices.contiguous();

  // A:116-119
  TORCH_CHECK(T > 0, "weights_offsets size must be great than 0.");
  TORCH_CHECK(N > 0, "indices can not be empty tensor.");
  TORCH_CHECK(off.size(0) > 1, "offsets dim_0 must be great than 1.");
  TORCH_CHECK(weights_tys.size(0) == T, "weights_tys size must equal weights_offsets size.");
  TORCH_CHECK(D_offsets.size(0) == T + 1, "The length of D_offsets must equal weights_offsets(", T, ") + 1.");
  TORCH_CHECK(dev_weights.is_cuda(), "dev_weights must be a HIP device tensor");
  TORCH_CHECK(dev_weights.scalar_type() == at::kByte, "dev_weights must be uint8");
  TORCH_CHECK(dev_weights.is_contiguous(), "dev_weights must be contiguous");
  TORCH_CHECK(idx.device() == dev_weights.device() && off.device() == dev_weights.device(),
              "indices and offsets must be on the weights' device");
  if (psw) {
    TORCH_CHECK(psw->numel() == N, "Len mismatch: indice_weights(", psw->numel(), ") must equal indices(", N, ").");
    TORCH_CHECK(psw->device() == dev_weights.device(), "indice_weights must be on the weights' device");
  }
  TORCH_CHECK(pooling_mode >= TBE_POOL_SUM && pooling_mode <= TBE_POOL_NONE, "Invalid pooling mode ",
              pooling_mode, ": supported modes are SUM(0), MEAN(1), NONE(2)");
  const at::ScalarType out_type = sparse_type_to_scalar_type(output_dtype);
  if (output_dtype == TBE_TY_INT8) {
    // A:125-129 first (same message), then the kernels' own rejection (P:336-338, N:295-296);
    // this path only ever raises, so its host copy costs nothing in steady state
    const bool all_int8 = weights_tys.to(at::kCPU).eq(static_cast<uint8_t>(TBE_TY_INT8)).all().item<bool>();
    TORCH_CHECK(all_int8, "int8 output_dtype requires all tables to use int8 weights.");
    TORCH_CHECK(false, "INT8 output_dtype is not supported (the reference kernel asserts on it as well)");
  }

  const PlanKey key{weights_offsets.data_ptr(), static_cast<int64_t>(weights_offsets._version()),
                    weights_tys.data_ptr(),     static_cast<int64_t>(weights_tys._version()),
                    D_offsets.data_ptr(),       static_cast<int64_t>(D_offsets._version()),
                    T, dev_weights.numel(), row_align, fp8_bits, fp8_bias,
                    static_cast<int>(dev_weights.get_device())};
  const Plan plan = plan_cache().get(key, weights_offsets, weights_tys, D_offsets, dev_weights.device());
  const TbePlanSummary& s = *plan.summary;

  TbeNbitArgs a{};
  a.dev_weights = dev_weights.data_ptr<uint8_t>();
  a.tables = plan.descs();
  a.table_order = plan.order(T);
  a.plan = plan.summary.get();
  a.T = static_cast<int32_t>(T);
  a.max_col_tiles = s.max_col_tiles;
  a.indices = idx.data_ptr();
  a.offsets = off.data_ptr();
  a.index_size = static_cast<int32_t>(idx.element_size());
  a.pooling_mode = static_cast<int32_t>(pooling_mode);
  a.num_indices = N;
  a.indice_weights = nullptr;
  a.output_dtype = static_cast<int32_t>(output_dtype);
  a.fp8_exponent_bits = static_cast<int32_t>(fp8_bits);
  a.fp8_exponent_bias = static_cast<int32_t>(fp8_bias);
  a.B = (off.size(0) - 1) / T;

  Tensor output;
  if (pooling_mode == TBE_POOL_NONE) {
    // A:132-146; every table must have D == max_D (c310/README.md:96-98)
    TORCH_CHECK(s.uniform_D && s.max_D == max_D, "nobag mode requires every table's D to equal max_D (",
                max_D, ")");
    output = at::empty({N, max_D}, dev_weights.options().dtype(out_type));
    a.output_stride = max_D;
  } else {
    // A:148-155
    TORCH_CHECK((off.size(0) - 1) % T == 0, "offset size = ", off.size(0),
                " is incorrect for feature count = ", T);
    TORCH_CHECK(s.total_D <= total_D, "D_offsets[-1] (", s.total_D, ") exceeds total_D (", total_D, ")");
    const bool full = s.covers_output && s.total_D == total_D;
    output = full ? at::empty({a.B, total_D}, dev_weights.options().dtype(out_type))
                  : at::zeros({a.B, total_D}, dev_weights.options().dtype(out_type));
    a.output_stride = total_D;
    if (psw) a.indice_weights = psw->data_ptr<float>();
  }
  a.output = output.data_ptr();
  if (output.numel() == 0) return output;
  const hipStream_t stream = c10::hip::getCurrentHIPStream(dev_weights.get_device()).stream();
  const int rc = tbe_nbit_forward(&a, stream);
  TORCH_CHECK(rc == TBE_OK, "int_nbit_split_embedding_codegen_lookup_function: ", tbe_last_error());
  return output;
}

// Reference: src/pooled_embedding_ops/permute_pooled_embs/permute_pooled_embs.cpp
// ("PA"), checks of PA:25-60 with the same messages.  inv_permute_list is not used
// (PA:69).  Unlike PA:82-98 the host never reads the lists (no synchronisation):
// every segment is copied on the device.
Tensor permute_pooled_embs_hip(const Tensor& pooled_embs, const Tensor& offset_dim_list,
                               const Tensor& permute_list, const Tensor& inv_offset_dim_list,
                               const Tensor& inv_permute_list) {
  (void)inv_permute_list;
  TORCH_CHECK(pooled_embs.dim() >= 2, "pooled_embs must be at least 2-D");
  TORCH_CHECK(offset_dim_list.scalar_type() == at::kLong, "offset_dim_list must be int64");
  TORCH_CHECK(permute_list.scalar_type() == at::kLong, "permute_list must be int64");
  TORCH_CHECK(inv_offset_dim_list.scalar_type() == at::kLong, "inv_offset_dim_list must be int64");
  const int64_t T = permute_list.numel();
  TORCH_CHECK(offset_dim_list.numel() == T + 1, "offset_dim_list must have T+1 elements");
  TORCH_CHECK(inv_offset_dim_list.numel() == T + 1, "inv_offset_dim_list must have T+1 elements");
  const auto st = pooled_embs.scalar_type();
  TORCH_CHECK(st == at::kFloat || st == at::kHalf || st == at::kBFloat16,
              "pooled_embs must be float32, float16, or bfloat16");
  const std::vector<std::pair<const Tensor*, const char*>> all = {
      {&pooled_embs, "pooled_embs"}, {&offset_dim_list, "offset_dim_list"},
      {&permute_list, "permute_list"}, {&inv_offset_dim_list, "inv_offset_dim_list"}};
  for (const auto& [x, name] : all) {
    TORCH_CHECK(x->defined(), name, " tensor must be defined");
    TORCH_CHECK(x->numel() > 0, name, " tensor must be non-empty");
    TORCH_CHECK(x->dim() > 0, name, " tensor must have non-zero dimensions");
    TORCH_CHECK(x->is_cuda() && x->get_device() == pooled_embs.get_device(), name,
                " must be on the same HIP device as pooled_embs");
  }
  at::OptionalDeviceGuard guard(at::device_of(pooled_embs));
  const Tensor in = pooled_embs.contiguous();
  const Tensor off = offset_dim_list.contiguous();
  const Tensor perm = permute_list.contiguous();
  const Tensor inv = inv_offset_dim_list.contiguous();
  Tensor output = at::empty_like(in);
  TbePermutePooledArgs a{};
  a.pooled_embs = in.data_ptr();
  a.output = output.data_ptr();
  a.B = in.size(0);
  a.total_D = in.size(1);
  a.inner = in.numel() / std::max<int64_t>(1, a.B * a.total_D);
  a.elem_size = static_cast<int32_t>(in.element_size());
  a.T = static_cast<int32_t>(T);
  a.offset_dim_list = off.data_ptr<int64_t>();
  a.permute_list = perm.data_ptr<int64_t>();
  a.inv_offset_dim_list = inv.data_ptr<int64_t>();
  const hipStream_t stream = c10::hip::getCurrentHIPStream(in.get_device()).stream();
  const int rc = tbe_permute_pooled_embs(&a, stream);
  TORCH_CHECK(rc == TBE_OK, "permute_pooled_embs: ", tbe_last_error());
  return output;
}

// Reference: src/sparse_ops/block_bucketize_sparse_features/block_bucketize_sparse_features.cpp
// ("BA"): the checks of BA:37-91 and BA:107-128 with the same messages, the
// output allocation of BA:154-204, the offsets of BA:167 and BA:172.
std::tuple<Tensor, Tensor, c10::optional<Tensor>, c10::optional<Tensor>, c10::optional<Tensor>>
block_bucketize_sparse_features_hip(const Tensor& lengths, const Tensor& indices, bool bucketize_pos, bool sequence,
                                    const Tensor& block_sizes, int64_t my_size,
                                    const c10::optional<Tensor>& weights,
                                    const c10::optional<Tensor>& batch_size_per_feature, int64_t max_B,
                                    const c10::optional<std::vector<Tensor>>& block_bucketize_pos,
                                    bool keep_orig_idx, const c10::optional<Tensor>& total_num_blocks) {
  TORCH_CHECK(my_size > 0, "my_size must be positive.");
  if (lengths.scalar_type() == at::kInt)
    TORCH_CHECK(my_size <= static_cast<int64_t>(std::numeric_limits<uint32_t>::max()),
                "my_size must fit into uint32 for int32 tensors.");
  TORCH_CHECK(lengths.dim() == 1, "lengths must be 1D.");
  TORCH_CHECK(indices.dim() == 1, "indices must be 1D.");
  TORCH_CHECK(block_sizes.dim() == 1, "block_sizes must be 1D.");
  TORCH_CHECK(block_sizes.numel() > 0, "block_sizes must be non-empty.");
  TORCH_CHECK(block_sizes.scalar_type() == indices.scalar_type(), "block_sizes dtype must match indices.");
  TORCH_CHECK(lengths.scalar_type() == at::kInt || lengths.scalar_type() == at::kLong,
              "lengths must be int32 or int64.");
  TORCH_CHECK(indices.scalar_type() == at::kInt || indices.scalar_type() == at::kLong,
              "indices must be int32 or int64.");
  if (weights.has_value()) {
    TORCH_CHECK(weights->dim() == 1, "weights must be 1D.");
    TORCH_CHECK(weights->numel() == indices.numel(), "weights must match indices length.");
    TORCH_CHECK(weights->scalar_type() == at::kFloat, "weights dtype must be float32.");
  }
  if (batch_size_per_feature.has_value()) {
    TORCH_CHECK(batch_size_per_feature->dim() == 1, "batch_size_per_feature must be 1D.");
    TORCH_CHECK(batch_size_per_feature->scalar_type() == lengths.scalar_type(),
                "batch_size_per_feature dtype must match lengths.");
    TORCH_CHECK(batch_size_per_feature->numel() == block_sizes.numel(),
                "batch_size_per_feature length must match block_sizes length.");
    TORCH_CHECK(max_B > 0, "max_B must be positive when batch_size_per_feature is provided.");
  } else {
    TORCH_CHECK(lengths.numel() % block_sizes.numel() == 0,
                "lengths.size(0) must be divisible by block_sizes.size(0) when batch_size_per_feature is absent.");
  }
  if (total_num_blocks.has_value()) {
    TORCH_CHECK(total_num_blocks->dim() == 1, "total_num_blocks must be 1D.");
    TORCH_CHECK(total_num_blocks->scalar_type() == indices.scalar_type(),
                "total_num_blocks dtype must match indices.");
    TORCH_CHECK(total_num_blocks->numel() == block_sizes.numel(), "total_num_blocks must match block_sizes length.");
  }
  const int dev = lengths.get_device();
  std::vector<std::pair<const Tensor*, const char*>> all = {
      {&lengths, "lengths"}, {&indices, "indices"}, {&block_sizes, "block_sizes"}};
  if (weights.has_value()) all.push_back({&*weights, "weights"});
  if (batch_size_per_feature.has_value()) all.push_back({&*batch_size_per_feature, "batch_size_per_feature"});
  if (total_num_blocks.has_value()) all.push_back({&*total_num_blocks, "total_num_blocks"});
  for (const auto& [x, name] : all)
    TORCH_CHECK(x->is_cuda() && x->get_device() == dev, name, " must be on the same HIP device as lengths");

  at::OptionalDeviceGuard guard(at::device_of(lengths));
  const Tensor len_c = lengths.contiguous();
  const Tensor idx_c = indices.contiguous();
  const Tensor bs_c = block_sizes.contiguous();
  const int64_t L = len_c.numel();
  const int64_t N = idx_c.numel();
  const int64_t F = bs_c.numel();
  const auto lopt = len_c.options();
  const auto iopt = idx_c.options();
  Tensor new_lengths = at::empty({my_size * L}, lopt);
  Tensor new_offsets = at::empty({my_size * L + 1}, lopt);
  Tensor new_indices = at::empty({N}, iopt);
  Tensor bso;
  if (batch_size_per_feature.has_value())  // BA:172: complete cumsum
    bso = at::cat({at::zeros({1}, lopt), at::cumsum(batch_size_per_feature->contiguous(), 0, len_c.scalar_type())}).contiguous();
  Tensor w_c, new_w, new_pos, unb, tnb_c, pos_ptrs, pos_lens;
  std::vector<Tensor> pos_keep;
  if (weights.has_value()) {
    w_c = weights->contiguous();
    new_w = at::empty({N}, w_c.options());
  }
  if (bucketize_pos) new_pos = at::empty({N}, iopt);
  if (sequence) unb = at::empty({N}, iopt);
  if (total_num_blocks.has_value()) tnb_c = total_num_blocks->contiguous();
  if (block_bucketize_pos.has_value()) {
    TORCH_CHECK(static_cast<int64_t>(block_bucketize_pos->size()) == F,
                "block_bucketize_pos must hold one tensor per feature");
    std::vector<int64_t> ptrs(F), lens(F);
    for (int64_t f = 0; f < F; ++f) {
      const Tensor& t = (*block_bucketize_pos)[f];
      TORCH_CHECK(t.scalar_type() == idx_c.scalar_type(), "block_bucketize_pos dtype must match indices.");
      TORCH_CHECK(t.is_cuda() && t.get_device() == dev, "block_bucketize_pos must be on the same HIP device");
      pos_keep.push_back(t.contiguous());
      ptrs[f] = reinterpret_cast<int64_t>(pos_keep.back().data_ptr());
      lens[f] = t.dim() == 1 ? t.numel() : 0;
    }
    auto cpu64 = at::TensorOptions().dtype(at::kLong);
    pos_ptrs = at::tensor(ptrs, cpu64).to(len_c.device());
    pos_lens = at::tensor(lens, cpu64).to(len_c.device());
  }
  const int64_t ws_bytes = tbe_block_bucketize_workspace_bytes(my_size, L, static_cast<int32_t>(len_c.element_size()));
  TORCH_CHECK(ws_bytes > 0, "block_bucketize_sparse_features: bad sizes");
  Tensor ws = at::empty({ws_bytes}, lopt.dtype(at::kByte));

  TbeBlockBucketizeArgs a{};
  a.indices = idx_c.data_ptr();
  a.num_indices = N;
  a.offsets = nullptr;  // formed from the lengths by the library (BA:167)
  a.lengths = len_c.data_ptr();
  a.lengths_size = L;
  a.index_size = static_cast<int32_t>(idx_c.element_size());
  a.offset_size = static_cast<int32_t>(len_c.element_size());
  a.block_sizes = bs_c.data_ptr();
  a.num_features = static_cast<int32_t>(F);
  a.keep_orig_idx = keep_orig_idx ? 1 : 0;
  a.my_size = my_size;
  a.weights = w_c.defined() ? w_c.data_ptr<float>() : nullptr;
  a.batch_size_offsets = bso.defined() ? bso.data_ptr() : nullptr;
  a.total_num_blocks = tnb_c.defined() ? tnb_c.data_ptr() : nullptr;
  a.bucketize_pos = pos_ptrs.defined() ? reinterpret_cast<const void* const*>(pos_ptrs.data_ptr()) : nullptr;
  a.bucketize_pos_len = pos_lens.defined() ? pos_lens.data_ptr<int64_t>() : nullptr;
  a.new_lengths = new_lengths.data_ptr();
  a.new_offsets = new_offsets.data_ptr();
  a.new_indices = new_indices.data_ptr();
  a.new_weights = new_w.defined() ? new_w.data_ptr<float>() : nullptr;
  a.new_pos = new_pos.defined() ? new_pos.data_ptr() : nullptr;
  a.unbucketize_permute = unb.defined() ? unb.data_ptr() : nullptr;
  a.workspace = ws.data_ptr();
  a.workspace_bytes = ws_bytes;
  const hipStream_t stream = c10::hip::getCurrentHIPStream(dev).stream();
  const int rc = tbe_block_bucketize_sparse_features(&a, stream);
  TORCH_CHECK(rc == TBE_OK, "block_bucketize_sparse_features: ", tbe_last_error());
  auto opt = [](const Tensor& t) { return t.defined() ? c10::optional<Tensor>(t) : c10::nullopt; };
  return {new_lengths, new_indices, opt(new_w), opt(new_pos), opt(unb)};
}

// The module's forward without the dispatcher: the operator's arguments that do not
// change between calls (the module's buffers and sizes) are bound once, and a call
// passes only indices, offsets and per-sample weights.  Same function, checks and
// plan cache as the operator; what it saves is the Python-side packing of 23
// arguments into the dispatcher's boxed form (most of the host time of a call on a
// small batch).
struct BoundLookup {
  Tensor dev_weights, uvm_weights, weights_placements, weights_offsets, weights_tys, D_offsets;
  int64_t total_D, max_int2_D, max_int4_D, max_int8_D, max_float16_D, max_float32_D, pooling_mode, output_dtype;
  std::optional<int64_t> row_alignment, max_float8_D, fp8_exponent_bits, fp8_exponent_bias;

  Tensor operator()(const Tensor& indices, const Tensor& offsets, const std::optional<Tensor>& indice_weights) const {
    // the dispatcher would pick a backend from the tensors' devices: with none on a
    // HIP device there is no implementation (no CPU fallback), as through the op
    TORCH_CHECK_NOT_IMPLEMENTED(
        dev_weights.is_cuda() || indices.is_cuda() || offsets.is_cuda() ||
            (indice_weights && indice_weights->is_cuda()),
        "Could not run 'fbgemm::int_nbit_split_embedding_codegen_lookup_function' with arguments from the '",
        indices.device().type(), "' backend: this package implements it for HIP tensors only");
    return int_nbit_split_embedding_codegen_lookup_function_hip(
        dev_weights, uvm_weights, weights_placements, weights_offsets, weights_tys, D_offsets, total_D,
        max_int2_D, max_int4_D, max_int8_D, max_float16_D, max_float32_D, indices, offsets, pooling_mode,
        indice_weights, output_dtype, std::nullopt, std::nullopt, row_alignment, max_float8_D, fp8_exponent_bits,
        fp8_exponent_bias);
  }
};

}  // namespace tbe_torch

PYBIND11_MODULE(_tbe_torch, m) {
  namespace py = pybind11;
  using at::Tensor;
  py::class_<tbe_torch::BoundLookup>(m, "BoundLookup")
      .def(py::init([](Tensor dev_weights, Tensor uvm_weights, Tensor weights_placements, Tensor weights_offsets,
                       Tensor weights_tys, Tensor D_offsets, int64_t total_D, int64_t max_int2_D,
                       int64_t max_int4_D, int64_t max_int8_D, int64_t max_float16_D, int64_t max_float32_D,
                       int64_t pooling_mode, int64_t output_dtype, std::optional<int64_t> row_alignment,
                       std::optional<int64_t> max_float8_D, std::optional<int64_t> fp8_exponent_bits,
                       std::optional<int64_t> fp8_exponent_bias) {
             return tbe_torch::BoundLookup{dev_weights, uvm_weights, weights_placements, weights_offsets,
                                           weights_tys, D_offsets, total_D, max_int2_D, max_int4_D,
                                           max_int8_D, max_float16_D, max_float32_D, pooling_mode,
                                           output_dtype, row_alignment, max_float8_D, fp8_exponent_bits,
                                           fp8_exponent_bias};
           }))
      .def("__call__", &tbe_torch::BoundLookup::operator(), py::arg("indices"), py::arg("offsets"),
           py::arg("indice_weights") = py::none());
}

// PyTorch-ROCm routes HIP tensors through the CUDA dispatch key.
TORCH_LIBRARY_IMPL(fbgemm, CUDA, m) {
  m.impl("int_nbit_split_embedding_codegen_lookup_function",
         TORCH_FN(tbe_torch::int_nbit_split_embedding_codegen_lookup_function_hip));
  m.impl("permute_pooled_embs", TORCH_FN(tbe_torch::permute_pooled_embs_hip));  // PA:119-121
  m.impl("block_bucketize_sparse_features", TORCH_FN(tbe_torch::block_bucketize_sparse_features_hip));  // BA:262-266
}

// PA:107-117: the reference also exposes the op as mxrec::permute_pooled_embs.
TORCH_LIBRARY_IMPL(mxrec, CUDA, m) {
  m.impl("permute_pooled_embs", TORCH_FN(tbe_torch::permute_pooled_embs_hip));
  m.impl("block_bucketize_sparse_features", TORCH_FN(tbe_torch::block_bucketize_sparse_features_hip));  // BA:256-260
}
