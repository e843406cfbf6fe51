/*
 * tbe_nbit.h — C ABI of the MI355X (gfx950) quantized table-batched-embedding
 * inference forward: the drop-in device path behind
 * torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function.
 *
 * Only plain pointers and sizes cross this boundary (no torch types).  The
 * torch extension in fbgemm-ascend_amd/csrc/tbe_torch.cpp is one caller; any
 * FFI (ctypes, cgo, JNI) can bind the same symbols.
 *
 * Reference interfaces this ABI replaces (paths relative to the reference
 * repository root; A = src/tbe_inference/int_nbit_split_embedding_codegen_lookup_function/
 * int_nbit_split_embedding_codegen_lookup_function.cpp, H/HT = its c310/op_host
 * files, E = c310/op_kernel/int_nbit_split_embedding_codegen_lookup_function.cpp):
 *   - tbe_nbit_plan     <- TilingFunc / ShapeTilingFunc (H:88-276) and the
 *                          tiling struct (HT:20-45): host-side shape checks and
 *                          the per-table work description.
 *   - tbe_nbit_forward  <- EXEC_NPU_CMD(aclnnIntNbitSplitEmbeddingCodegenLookupFunction, ...)
 *                          (A:140-144, A:161-165) and the device entry
 *                          int_nbit_split_embedding_codegen_lookup_function (E:58-89).
 *   - tbe_last_error    <- the OPS_LOG_E / TORCH_CHECK messages of H:110-204 and A:116-151.
 */
#ifndef TBE_NBIT_H
#define TBE_NBIT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight / output type codes: SparseType, A:24-33 and c310/op_kernel/common.h:58-67. */
enum TbeSparseType {
  TBE_TY_FP32 = 0,
  TBE_TY_FP16 = 1,
  TBE_TY_INT8 = 2,
  TBE_TY_INT4 = 3,
  TBE_TY_INT2 = 4,
  TBE_TY_BF16 = 5,
  TBE_TY_FP8 = 6
};

/* Pooling modes: PoolingMode, A:18-22. */
enum TbePoolingMode { TBE_POOL_SUM = 0, TBE_POOL_MEAN = 1, TBE_POOL_NONE = 2 };

/* Status codes returned by every entry point. */
enum TbeStatus {
  TBE_OK = 0,
  TBE_ERR_INVALID_ARG = -1,   /* shape / dtype / attribute check failed   */
  TBE_ERR_UNSUPPORTED = -2,   /* valid in the schema but not implemented  */
  TBE_ERR_LAUNCH = -3         /* the HIP runtime rejected a launch        */
};

/*
 * Per-table work description, produced on the host by tbe_nbit_plan and read
 * by the device kernels (the caller copies the array to device memory once
 * and may reuse it for every call with the same table metadata).
 * Row r of table t occupies dev_weights[weights_offset + r*row_stride, +row_stride);
 * its payload starts data_offset bytes in (after the fp16 scale/bias header of
 * INT8/INT4/INT2 rows).
 */
typedef struct TbeTableDesc {
  int64_t weights_offset; /* byte offset of row 0 inside dev_weights              */
  int64_t num_rows;       /* rows that fit before the next table / buffer end     */
  int32_t D;              /* embedding dim                                        */
  int32_t D_offset;       /* first output column of this table                    */
  int32_t row_stride;     /* bytes, roundup(unpadded row bytes, row_alignment)    */
  int32_t data_offset;    /* 4 for INT8/INT4/INT2 (fp16 scale, fp16 bias), else 0 */
  int32_t data_dwords;    /* payload size in 4-byte words = D*bits/32             */
  uint8_t weight_ty;      /* TbeSparseType                                        */
  uint8_t log2_lanes;     /* lanes of a 64-wide wavefront that share one row     */
  uint8_t col_tiles;      /* 256-byte column tiles per row (>1 only for wide rows)*/
  uint8_t flags;          /* TBE_TABLE_* bits, set by the planner                 */
} TbeTableDesc;

/* TbeTableDesc.flags: the table's rows span at most 0xFFFE0000 bytes (4 GiB less
 * 128 KiB), so the kernels address them with 32-bit offsets from the table base
 * (buffer loads with range checking). */
#define TBE_TABLE_OFFSET32 0x1
/* TbeTableDesc.flags: OFFSET32 and a payload of at least 8 words in an even
 * number of words, so the table may be gathered by the row-stream kernel (8-byte
 * lanes, one contiguous index run per slot of lanes) and, for INT4 rows of 17-32
 * words, by the per-bag kernel with 8-byte lanes. */
#define TBE_TABLE_STREAM 0x2

/* Host-side table metadata handed to the planner (all host pointers). */
typedef struct TbePlanInput {
  int32_t T;                       /* number of tables                          */
  const int64_t* weights_offsets;  /* [T]   byte offsets into dev_weights       */
  const uint8_t* weights_tys;      /* [T]   TbeSparseType                       */
  const int32_t* D_offsets;        /* [T+1] prefix sum of embedding dims        */
  int64_t dev_weights_bytes;       /* size of dev_weights                       */
  int32_t row_alignment;           /* bytes, reference default 16 (A:86)        */
  int32_t fp8_exponent_bits;       /* -1 when no FP8 table                      */
  int32_t fp8_exponent_bias;       /* -1 when no FP8 table                      */
} TbePlanInput;

/*
 * Tables that share one kernel specialisation: same weight type, same lanes per
 * row, same addressing mode.  Their ids are table_order[first .. first+count).
 */
typedef struct TbePlanGroup {
  int32_t weight_ty;      /* TbeSparseType; -1: the generic 64-bit group (tables of */
                          /* 2^32 - 1 rows or more, any type and width)            */
  int32_t log2_lanes;     /* as in TbeTableDesc; -1 for the generic group          */
  int32_t offset32;       /* 1: all rows addressed with 32-bit offsets; 0: 64-bit  */
                          /* row addresses (the per-bag kernel's A64 form, or the  */
                          /* generic kernel when weight_ty is -1)                  */
  int32_t first;          /* position in table_order                               */
  int32_t count;          /* tables in the group                                   */
  int32_t col_tiles;      /* max col_tiles over the group's tables                 */
  int32_t stream;         /* 1: every table has TBE_TABLE_STREAM                   */
} TbePlanGroup;

#define TBE_MAX_GROUPS 64

/* Summary of a plan: what the launcher needs beyond the per-table array. */
typedef struct TbePlanSummary {
  int32_t max_col_tiles;  /* max over tables of col_tiles                          */
  int32_t max_D;          /* max over tables of D                                  */
  int32_t total_D;        /* D_offsets[T]                                          */
  int32_t uniform_D;      /* 1 if every table has the same D (nobag requirement)   */
  int32_t covers_output;  /* 1 if D_offsets[0]==0 and tables tile [0,total_D)     */
  int32_t has_fp8;        /* 1 if any table is FP8                                 */
  int32_t num_groups;     /* entries of groups[]                                   */
  TbePlanGroup groups[TBE_MAX_GROUPS];
} TbePlanSummary;

/*
 * Arguments of one forward call.  All pointers are device pointers except
 * `tables`, which is a device copy of the array tbe_nbit_plan filled.
 * Layout contract (A:155, A:135): bag mode writes output[B, output_stride]
 * (output_stride = total_D) in the output dtype; nobag writes
 * output[num_indices, output_stride] (output_stride = max_D).
 * Every output element inside a table's column range is written, including
 * the zeros of empty bags, so the caller need not pre-clear the output when
 * TbePlanSummary.covers_output is 1.  Nobag writes every one of the
 * num_indices output rows: rows of positions outside [offsets[0], offsets[T*B])
 * are zero.
 */
typedef struct TbeNbitArgs {
  const uint8_t* dev_weights;      /* packed rows of all tables                 */
  const TbeTableDesc* tables;      /* device [T]                                */
  const int32_t* table_order;      /* device [T], from tbe_nbit_plan            */
  const TbePlanSummary* plan;      /* HOST pointer, from tbe_nbit_plan          */
  int32_t T;
  int32_t max_col_tiles;           /* from TbePlanSummary                       */
  int64_t B;                       /* bags per table = (len(offsets)-1)/T       */
  const void* indices;             /* device [num_indices], int32 or int64      */
  const void* offsets;             /* device [T*B+1], same dtype as indices     */
  int32_t index_size;              /* 4 or 8                                    */
  int32_t pooling_mode;            /* TbePoolingMode                            */
  int64_t num_indices;
  const float* indice_weights;     /* device [num_indices] or NULL (bag modes)  */
  int32_t output_dtype;            /* TBE_TY_FP32, TBE_TY_FP16 or TBE_TY_BF16   */
  int32_t fp8_exponent_bits;
  int32_t fp8_exponent_bias;
  int32_t flags;                   /* TBE_FLAG_* tuning switches, 0 = default   */
  void* output;
  int64_t output_stride;           /* elements per output row                   */
} TbeNbitArgs;

/* Tuning switches for TbeNbitArgs.flags (results are identical either way). */
#define TBE_FLAG_NO_XCD_REMAP 0x1  /* keep the hardware's round-robin block order */
#define TBE_FLAG_NO_STREAM 0x2     /* never use the row-stream kernel (per-bag kernel for every group) */
#define TBE_FLAG_FORCE_STREAM 0x4  /* row-stream kernel for every eligible group, whatever its size */
#define TBE_FLAG_SERIAL_GROUPS 0x8 /* launch every table group on the caller's stream (no fork/join) */
#define TBE_FLAG_NARROW_WORDS 0x10 /* per-bag kernel: one 4-byte word per lane, also for rows of 16+ words */

/*
 * Validate the table metadata and fill descs[T], table_order[T] (host memory)
 * and *summary (which lists the table groups the forward launches one kernel
 * for).  Mirrors the shape checks of H:95-204 and A:116-151, and rejects what the
 * kernels cannot address: a known weight type per table, D_offsets increasing
 * (every table at least one column), rows of whole 4-byte words, 4-byte aligned
 * table offsets inside dev_weights, row_alignment a positive multiple of 4, and
 * FP8 exponent bits / bias in range when an FP8 table is present.  Returns TBE_OK
 * or a negative TbeStatus; tbe_last_error() then names the failed check.
 */
int tbe_nbit_plan(const TbePlanInput* in, TbeTableDesc* descs, int32_t* table_order,
                  TbePlanSummary* summary);

/*
 * Enqueue the forward on `hip_stream` (a hipStream_t; NULL = default stream).
 * Asynchronous: returns after the launch, without a host synchronisation.
 * Returns TBE_OK or a negative TbeStatus.
 */
int tbe_nbit_forward(const TbeNbitArgs* args, void* hip_stream);

/* Message of the last failure on the calling thread ("" if none). */
const char* tbe_last_error(void);

/* ABI version of this header; bumped on any layout change of the structs above. */
int tbe_nbit_abi_version(void);
#define TBE_NBIT_ABI_VERSION 3

#ifdef __cplusplus
}
#endif

#endif /* TBE_NBIT_H */
