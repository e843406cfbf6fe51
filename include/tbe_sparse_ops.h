/*
 * tbe_sparse_ops.h — C ABI of the MI355X (gfx950) block bucketisation of sparse
 * features: the step before the TBE forward that splits each feature's indices
 * over my_size shards (row-wise sharded embedding tables).
 *
 * Same conventions as tbe_nbit.h (TBE_OK / negative TbeStatus, tbe_last_error(),
 * asynchronous launches on hip_stream, plain device pointers).
 *
 * Reference interface (paths relative to the reference repository root):
 *   tbe_block_bucketize_sparse_features <- block_bucketize_sparse_features_npu
 *     (src/sparse_ops/block_bucketize_sparse_features/block_bucketize_sparse_features.cpp:93-246)
 *     and its two kernels, ComputeNewLengths and ScatterNewIndices
 *     (.../c310/op_kernel/block_bucketize_sparse_features_kernel_full.h:106-219).
 */
#ifndef TBE_SPARSE_OPS_H
#define TBE_SPARSE_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Row r in [0, lengths_size) holds indices [offsets[r-1], offsets[r]) (offsets is
 * the inclusive cumsum of lengths; offsets[-1] = 0) and belongs to feature
 * r / (lengths_size / num_features), or, with batch_size_offsets (the complete
 * cumsum of batch_size_per_feature, num_features+1 entries), to the last f with
 * batch_size_offsets[f] <= r.  Each index is mapped to a bucket (the shard) and a
 * new index by the rule of kernel_full.h:387-455 and 560-603 (block sizes,
 * optional total_num_blocks, optional per-feature block_bucketize_pos boundaries,
 * keep_orig_idx), and written to segment (bucket, r) of the outputs, which starts at
 * new_offsets[bucket * lengths_size + r].  Inside a segment indices keep their order
 * in the row (the reference keeps it only for sequence = 1).
 *
 * Outputs: new_lengths [my_size * lengths_size], new_offsets [my_size *
 * lengths_size + 1] (complete cumsum of new_lengths), new_indices [num_indices], and
 * when requested new_weights (weights given), new_pos (bucketize_pos: position of
 * the index inside its row) and unbucketize_permute (sequence: output position of
 * every input index).
 *
 * Widths: index_size (indices, block_sizes, total_num_blocks, pos lists, new_indices,
 * new_pos, unbucketize_permute) and offset_size (lengths, offsets, batch_size_offsets,
 * new_lengths, new_offsets), each 4 or 8.  Rows of a feature with a negative block
 * size, and indices whose bucket would fall outside [0, my_size) (only possible
 * with a total_num_blocks that is not a multiple of my_size), are left out; the
 * reference writes those out of bounds.  Positions of new_indices, new_weights and
 * new_pos past sum(new_lengths), and unbucketize_permute entries of left-out
 * indices, are then not written.
 *
 * `workspace` is device scratch of tbe_block_bucketize_workspace_bytes() bytes.
 */
typedef struct TbeBlockBucketizeArgs {
  const void* indices;                 /* device [num_indices]                        */
  int64_t num_indices;
  const void* offsets;                 /* device [lengths_size], inclusive cumsum,
                                          or NULL with `lengths` given (see below)    */
  int64_t lengths_size;
  int32_t index_size;                  /* 4 or 8                                      */
  int32_t offset_size;                 /* 4 or 8                                      */
  const void* block_sizes;             /* device [num_features]                       */
  int32_t num_features;
  int32_t keep_orig_idx;               /* 0 / 1                                       */
  int64_t my_size;                     /* >= 1                                        */
  const float* weights;                /* device [num_indices] or NULL                */
  const void* batch_size_offsets;      /* device [num_features + 1] or NULL           */
  const void* total_num_blocks;        /* device [num_features] or NULL               */
  const void* const* bucketize_pos;    /* device [num_features] pointers, or NULL     */
  const int64_t* bucketize_pos_len;    /* device [num_features]                       */
  void* new_lengths;                   /* device [my_size * lengths_size]             */
  void* new_offsets;                   /* device [my_size * lengths_size + 1]         */
  void* new_indices;                   /* device [num_indices]                        */
  float* new_weights;                  /* device [num_indices] or NULL                */
  void* new_pos;                       /* device [num_indices] or NULL                */
  void* unbucketize_permute;           /* device [num_indices] or NULL                */
  void* workspace;
  int64_t workspace_bytes;
  /* device [lengths_size] or NULL.  With offsets NULL the library forms the offsets
   * from these lengths itself (the complete cumsum of BA:167) in its scratch, on the
   * call's stream; with offsets given it is not read. */
  const void* lengths;
} TbeBlockBucketizeArgs;

int64_t tbe_block_bucketize_workspace_bytes(int64_t my_size, int64_t lengths_size, int32_t offset_size);

int tbe_block_bucketize_sparse_features(const TbeBlockBucketizeArgs* args, void* hip_stream);

/*
 * Same operation and results as tbe_block_bucketize_sparse_features, without any
 * allocation: no hipMalloc / hipFree / allocating library call, and no workspace
 * argument (args->workspace and args->workspace_bytes are ignored).  It has no
 * counterpart in the reference; it is for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid it).  The
 * caller still passes every input and output.
 *
 * Scratch (the per-segment write cursors when my_size > 64, one flag byte per
 * row otherwise, and the scan's tile sums) lives in a static device array of
 * TBE_BLOCK_BUCKETIZE_NOALLOC_SCRATCH_BYTES bytes that each GPU the library runs
 * on holds until the process ends; it is cleared or fully written by the call's own
 * kernels where it must start at a known value.  A call needs
 *   roundup(my_size > 64 ? 4 * my_size * lengths_size : lengths_size, 256)
 *   + roundup(offset_size * (lengths_size + 1), 256)
 *   + offset_size * max(1, ceil(my_size * lengths_size / 1024))
 * bytes of it; larger calls are rejected with TBE_ERR_UNSUPPORTED and a message.
 * Every call on one GPU shares that GPU's array, so calls on one GPU are made
 * to run one after another: each call (from any stream or host thread) first
 * makes its stream wait for an event recorded after the previous call on that
 * GPU, then records it after its own kernels; calls on different streams are
 * therefore serialised on the GPU rather than overlapped.  The first call on a GPU
 * looks up the array's address and creates that event.  A call made while its
 * stream is being captured into a HIP graph neither waits nor records (an event
 * from outside the capture cannot be waited on inside it): the graph orders the
 * captured call, and a replay must not run at the same time as another call on
 * the same GPU.
 */
#define TBE_BLOCK_BUCKETIZE_NOALLOC_SCRATCH_BYTES (32LL << 20)
int tbe_block_bucketize_sparse_features_noalloc(const TbeBlockBucketizeArgs* args, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* TBE_SPARSE_OPS_H */
