"""ctypes/numpy front end of the CPU oracle (oracle/tbe_oracle.c).

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, as the checker; the product path never
does.  Semantics and citations are in the header of tbe_oracle.c; the Python
signature mirrors torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function
(reference A:55-78) with host numpy arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libtbe_oracle.so")
_lib = None

FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6
_BITS = {FP32: 32, FP16: 16, BF16: 16, INT8: 8, FP8: 8, INT4: 4, INT2: 2}


def build() -> str:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        path = os.environ.get("TBE_ORACLE_LIB")  # e.g. the sanitizer build (make asan)
        if not path:
            path = _LIB_PATH
            if not os.path.exists(path):
                build()
        L = ctypes.CDLL(path)
        P, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.oracle_tbe_forward.restype = ctypes.c_int
        L.oracle_tbe_forward.argtypes = [P, ctypes.c_int, P, P, P, P, P, P, ctypes.c_int, i64, i64,
                                         ctypes.c_int, P, ctypes.c_int, i64, ctypes.c_int,
                                         ctypes.c_int, P, P, i64, ctypes.c_int]
        L.oracle_fp8_to_float.restype = ctypes.c_float
        L.oracle_fp8_to_float.argtypes = [ctypes.c_uint8, ctypes.c_int, ctypes.c_int]
        L.oracle_decode_fp8_table.argtypes = [ctypes.c_int, ctypes.c_int, P]
        for name in ("oracle_half_to_float_n", "oracle_float_to_half_n", "oracle_float_to_bf16_n"):
            getattr(L, name).argtypes = [P, P, i64]
        L.oracle_row_stride.restype = i64
        L.oracle_row_stride.argtypes = [ctypes.c_int, i64, i64]
        L.oracle_block_bucketize.restype = ctypes.c_int
        L.oracle_block_bucketize.argtypes = [P, i64, ctypes.c_int, P, ctypes.c_int, i64, P, ctypes.c_int, i64, P, P, P,
                                             P, P, ctypes.c_int, P, P, P, P, P, P]
        L.oracle_permute_pooled_embs.restype = None
        L.oracle_permute_pooled_embs.argtypes = [P, P, i64, i64, i64, ctypes.c_int, ctypes.c_int, P, P, P]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def row_stride(ty: int, D: int, row_alignment: int = 16) -> int:
    return int(lib().oracle_row_stride(ty, D, row_alignment))


def table_rows(weights_offsets, weights_tys, D_offsets, weights_bytes, row_alignment=16):
    """Rows of each table that lie before the next table's first byte (or the buffer end)."""
    wo = np.asarray(weights_offsets, dtype=np.int64)
    starts = np.unique(wo)
    rows = np.zeros(len(wo), dtype=np.int64)
    for t in range(len(wo)):
        nxt = starts[starts > wo[t]]
        end = int(nxt[0]) if len(nxt) else int(weights_bytes)
        stride = row_stride(int(weights_tys[t]), int(D_offsets[t + 1] - D_offsets[t]), row_alignment)
        rows[t] = max(0, (end - int(wo[t])) // stride)
    return rows


def fp8_table(exp_bits: int, exp_bias: int) -> np.ndarray:
    out = np.zeros(256, dtype=np.float32)
    lib().oracle_decode_fp8_table(exp_bits, exp_bias, _ptr(out))
    return out


def half_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_half_to_float_n(_ptr(h), _ptr(out), h.size)
    return out


def float_to_half_bits(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().oracle_float_to_half_n(_ptr(f), _ptr(out), f.size)
    return out


def float_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().oracle_float_to_bf16_n(_ptr(f), _ptr(out), f.size)
    return out


def forward(dev_weights, weights_offsets, weights_tys, D_offsets, indices, offsets,
            pooling_mode: int, indice_weights=None, output_dtype: int = FP32,
            row_alignment: int = 16, fp8_exponent_bits: int = -1, fp8_exponent_bias: int = -1,
            rows=None, num_threads: int | None = None):
    """Run the oracle.  Returns (out, out_f32): `out` holds the output dtype's bits
    (float32 array, or uint16 array of fp16/bf16 bit patterns) and `out_f32` the fp32
    value of every element before the final cast."""
    w = np.ascontiguousarray(dev_weights, dtype=np.uint8)
    wo = np.ascontiguousarray(weights_offsets, dtype=np.int64)
    wt = np.ascontiguousarray(weights_tys, dtype=np.uint8)
    do = np.ascontiguousarray(D_offsets, dtype=np.int32)
    idx = np.ascontiguousarray(indices)
    if idx.dtype not in (np.int32, np.int64):
        raise TypeError("indices must be int32 or int64")
    off = np.ascontiguousarray(offsets, dtype=idx.dtype)
    T = len(wo)
    B = (len(off) - 1) // T
    if rows is None:
        rows = table_rows(wo, wt, do, w.size, row_alignment)
    rows = np.ascontiguousarray(rows, dtype=np.int64)
    psw = None if indice_weights is None else np.ascontiguousarray(indice_weights, dtype=np.float32)
    if pooling_mode == 2:
        max_D = int(np.max(do[1:] - do[:-1]))
        shape = (idx.size, max_D)
    else:
        shape = (B, int(do[-1]))
    out_f32 = np.zeros(shape, dtype=np.float32)
    out = np.zeros(shape, dtype=np.float32 if output_dtype == FP32 else np.uint16)
    nt = num_threads or os.cpu_count() or 1
    rc = lib().oracle_tbe_forward(_ptr(w), T, _ptr(wo), _ptr(wt), _ptr(do), _ptr(rows), _ptr(idx),
                                  _ptr(off), idx.itemsize, idx.size, B, pooling_mode, _ptr(psw),
                                  output_dtype, row_alignment, fp8_exponent_bits, fp8_exponent_bias,
                                  _ptr(out), _ptr(out_f32), shape[1], nt)
    if rc != 0:
        raise ValueError("oracle_tbe_forward rejected its arguments")
    return out, out_f32


def permute_pooled_embs(pooled_embs: np.ndarray, offset_dim_list, permute_list, inv_offset_dim_list,
                        out: np.ndarray | None = None) -> np.ndarray:
    """CPU restatement of permute_pooled_embs (oracle_permute_pooled_embs in tbe_oracle.c).
    `pooled_embs` is any [B, total_D, ...] array of 2- or 4-byte elements; the result
    has the same dtype and bits.  Columns no segment writes are taken from `out`
    (zeros by default)."""
    x = np.ascontiguousarray(pooled_embs)
    if x.itemsize not in (2, 4) or x.ndim < 2:
        raise TypeError("pooled_embs must be at least 2-D with 2- or 4-byte elements")
    off = np.ascontiguousarray(offset_dim_list, dtype=np.int64)
    perm = np.ascontiguousarray(permute_list, dtype=np.int64)
    inv = np.ascontiguousarray(inv_offset_dim_list, dtype=np.int64)
    res = np.zeros_like(x) if out is None else np.ascontiguousarray(out, dtype=x.dtype).copy()
    B, D = x.shape[0], x.shape[1]
    inner = x.size // max(1, B * D)
    lib().oracle_permute_pooled_embs(_ptr(x), _ptr(res), B, D, inner, x.itemsize, len(perm),
                                     _ptr(off), _ptr(perm), _ptr(inv))
    return res


def block_bucketize_sparse_features(lengths, indices, bucketize_pos: bool, sequence: bool, block_sizes,
                                    my_size: int, weights=None, batch_size_per_feature=None,
                                    block_bucketize_pos=None, keep_orig_idx: bool = False,
                                    total_num_blocks=None):
    """CPU restatement of block_bucketize_sparse_features (oracle_block_bucketize in
    tbe_oracle.c) with the op's argument list; numpy arrays in, a tuple (new_lengths,
    new_indices, new_weights, new_pos, unbucketize_permute) out, optional entries None
    when not requested.  Within a (bucket, row) segment indices keep their row order."""
    L_ = np.ascontiguousarray(lengths)
    idx = np.ascontiguousarray(indices)
    bs = np.ascontiguousarray(block_sizes, dtype=idx.dtype)
    if L_.dtype not in (np.int32, np.int64) or idx.dtype not in (np.int32, np.int64):
        raise TypeError("lengths and indices must be int32 or int64")
    os_, is_ = L_.itemsize, idx.itemsize
    L = L_.size
    F = bs.size
    offsets = np.cumsum(L_, dtype=L_.dtype) if L else np.zeros(0, L_.dtype)
    bso = None
    if batch_size_per_feature is not None:
        bso = np.concatenate([[0], np.cumsum(np.asarray(batch_size_per_feature, dtype=np.int64))]).astype(L_.dtype)
    tnb = None if total_num_blocks is None else np.ascontiguousarray(total_num_blocks, dtype=idx.dtype)
    pos_arrays = None
    pos_ptrs = pos_lens = None
    if block_bucketize_pos is not None:
        pos_arrays = [np.ascontiguousarray(p, dtype=idx.dtype) for p in block_bucketize_pos]
        pos_ptrs = (ctypes.c_void_p * F)(*[p.ctypes.data for p in pos_arrays])
        pos_lens = np.array([p.size for p in pos_arrays], dtype=np.int64)
    w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
    new_lengths = np.zeros(my_size * L, dtype=L_.dtype)
    f = lib().oracle_block_bucketize
    args_common = [_ptr(idx), idx.size, is_, _ptr(offsets), os_, L, _ptr(bs), F, int(my_size), _ptr(w), _ptr(bso), _ptr(tnb),
                   pos_ptrs, _ptr(pos_lens), int(bool(keep_orig_idx))]
    if f(*args_common, _ptr(new_lengths), None, None, None, None, None) != 0:
        raise MemoryError("oracle_block_bucketize")
    new_offsets = np.concatenate([[0], np.cumsum(new_lengths.astype(np.int64))]).astype(L_.dtype)
    n = idx.size
    new_indices = np.zeros(n, dtype=idx.dtype)
    new_weights = np.zeros(n, dtype=np.float32) if w is not None else None
    new_pos = np.zeros(n, dtype=idx.dtype) if bucketize_pos else None
    unb = np.zeros(n, dtype=idx.dtype) if sequence else None
    if f(*args_common, _ptr(new_lengths), _ptr(new_offsets), _ptr(new_indices), _ptr(new_weights), _ptr(new_pos),
         _ptr(unb)) != 0:
        raise MemoryError("oracle_block_bucketize")
    return new_lengths, new_indices, new_weights, new_pos, unb
