/*
 * tbe_pooled_ops.h — C ABI of the MI355X (gfx950) operators on either side of
 * the TBE inference forward: the column permutation of its pooled output and
 * the bucketisation of its sparse input.
 *
 * Same conventions as tbe_nbit.h: plain pointers and sizes, every entry point
 * returns TBE_OK (0) or a negative TbeStatus and tbe_last_error() names the
 * failed check; launches are asynchronous on the given hip_stream.
 *
 * Reference interfaces (paths relative to the reference repository root):
 *   tbe_permute_pooled_embs <- permute_pooled_embs_impl_npu and its kernel
 *     (src/pooled_embedding_ops/permute_pooled_embs/permute_pooled_embs.cpp:62-105,
 *      .../v220/op_kernel/permute_pooled_embs_kernel.h:173-211)
 */
#ifndef TBE_POOLED_OPS_H
#define TBE_POOLED_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * output[:, inv_offset_dim_list[i] : inv_offset_dim_list[i+1]] =
 *     pooled_embs[:, offset_dim_list[p] : offset_dim_list[p] + that width], p = permute_list[i]
 * for i in [0, T).  Both tensors are row-major [B, total_D, inner] (inner = 1
 * for the usual 2-D case: a column is `inner` consecutive elements) with
 * elements of elem_size bytes (2: fp16/bf16, 4: fp32); the copy is bit-exact.
 * The three lists are device arrays of int64.  A destination segment whose p is
 * outside [0, T), or whose source columns leave [0, total_D), is written as
 * zeros; one whose own columns leave [0, total_D) is not written.
 */
typedef struct TbePermutePooledArgs {
  const void* pooled_embs;             /* device [B, total_D, inner]     */
  void* output;                        /* device [B, total_D, inner]     */
  int64_t B;
  int64_t total_D;
  int64_t inner;                       /* >= 1                           */
  int32_t elem_size;                   /* 2 or 4                         */
  int32_t T;
  const int64_t* offset_dim_list;      /* device [T+1]                   */
  const int64_t* permute_list;         /* device [T]                     */
  const int64_t* inv_offset_dim_list;  /* device [T+1]                   */
} TbePermutePooledArgs;

int tbe_permute_pooled_embs(const TbePermutePooledArgs* args, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* TBE_POOLED_OPS_H */
