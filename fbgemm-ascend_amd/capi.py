"""ctypes binding of the C ABIs declared in include/tbe_nbit.h,
include/tbe_pooled_ops.h and include/tbe_sparse_ops.h (libtbe_hip.so).

This is the same boundary a cgo/JNI/N-API binding would use; the GPU parity
tests call the kernels through it directly, without the torch dispatcher.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import HIP_LIB

ABI_VERSION = 3
EXPORTS = ("tbe_nbit_plan", "tbe_nbit_forward", "tbe_last_error", "tbe_nbit_abi_version",
           "tbe_permute_pooled_embs", "tbe_block_bucketize_workspace_bytes",
           "tbe_block_bucketize_sparse_features", "tbe_block_bucketize_sparse_features_noalloc")
# TBE_BLOCK_BUCKETIZE_NOALLOC_SCRATCH_BYTES of include/tbe_sparse_ops.h
NOALLOC_SCRATCH_BYTES = 32 << 20

TBE_OK, TBE_ERR_INVALID_ARG, TBE_ERR_UNSUPPORTED, TBE_ERR_LAUNCH = 0, -1, -2, -3
TBE_FLAG_NO_XCD_REMAP = 0x1
TBE_FLAG_NO_STREAM = 0x2
TBE_FLAG_FORCE_STREAM = 0x4
TBE_FLAG_SERIAL_GROUPS = 0x8
TBE_FLAG_NARROW_WORDS = 0x10
TBE_TABLE_OFFSET32 = 0x1
TBE_TABLE_STREAM = 0x2


class TbeTableDesc(ctypes.Structure):
    _fields_ = [("weights_offset", ctypes.c_int64), ("num_rows", ctypes.c_int64),
                ("D", ctypes.c_int32), ("D_offset", ctypes.c_int32),
                ("row_stride", ctypes.c_int32), ("data_offset", ctypes.c_int32),
                ("data_dwords", ctypes.c_int32), ("weight_ty", ctypes.c_uint8),
                ("log2_lanes", ctypes.c_uint8), ("col_tiles", ctypes.c_uint8),
                ("flags", ctypes.c_uint8)]


class TbePlanInput(ctypes.Structure):
    _fields_ = [("T", ctypes.c_int32), ("weights_offsets", ctypes.c_void_p),
                ("weights_tys", ctypes.c_void_p), ("D_offsets", ctypes.c_void_p),
                ("dev_weights_bytes", ctypes.c_int64), ("row_alignment", ctypes.c_int32),
                ("fp8_exponent_bits", ctypes.c_int32), ("fp8_exponent_bias", ctypes.c_int32)]


class TbePlanGroup(ctypes.Structure):
    _fields_ = [("weight_ty", ctypes.c_int32), ("log2_lanes", ctypes.c_int32),
                ("offset32", ctypes.c_int32), ("first", ctypes.c_int32), ("count", ctypes.c_int32),
                ("col_tiles", ctypes.c_int32), ("stream", ctypes.c_int32)]


TBE_MAX_GROUPS = 64


class TbePlanSummary(ctypes.Structure):
    _fields_ = [("max_col_tiles", ctypes.c_int32), ("max_D", ctypes.c_int32),
                ("total_D", ctypes.c_int32), ("uniform_D", ctypes.c_int32),
                ("covers_output", ctypes.c_int32), ("has_fp8", ctypes.c_int32),
                ("num_groups", ctypes.c_int32), ("groups", TbePlanGroup * TBE_MAX_GROUPS)]


class TbeNbitArgs(ctypes.Structure):
    _fields_ = [("dev_weights", ctypes.c_void_p), ("tables", ctypes.c_void_p),
                ("table_order", ctypes.c_void_p), ("plan", ctypes.POINTER(TbePlanSummary)),
                ("T", ctypes.c_int32), ("max_col_tiles", ctypes.c_int32), ("B", ctypes.c_int64),
                ("indices", ctypes.c_void_p), ("offsets", ctypes.c_void_p),
                ("index_size", ctypes.c_int32), ("pooling_mode", ctypes.c_int32),
                ("num_indices", ctypes.c_int64), ("indice_weights", ctypes.c_void_p),
                ("output_dtype", ctypes.c_int32), ("fp8_exponent_bits", ctypes.c_int32),
                ("fp8_exponent_bias", ctypes.c_int32), ("flags", ctypes.c_int32),
                ("output", ctypes.c_void_p), ("output_stride", ctypes.c_int64)]


class TbePermutePooledArgs(ctypes.Structure):
    _fields_ = [("pooled_embs", ctypes.c_void_p), ("output", ctypes.c_void_p),
                ("B", ctypes.c_int64), ("total_D", ctypes.c_int64), ("inner", ctypes.c_int64),
                ("elem_size", ctypes.c_int32), ("T", ctypes.c_int32),
                ("offset_dim_list", ctypes.c_void_p), ("permute_list", ctypes.c_void_p),
                ("inv_offset_dim_list", ctypes.c_void_p)]


class TbeBlockBucketizeArgs(ctypes.Structure):
    _fields_ = [("indices", ctypes.c_void_p), ("num_indices", ctypes.c_int64),
                ("offsets", ctypes.c_void_p), ("lengths_size", ctypes.c_int64),
                ("index_size", ctypes.c_int32), ("offset_size", ctypes.c_int32),
                ("block_sizes", ctypes.c_void_p), ("num_features", ctypes.c_int32),
                ("keep_orig_idx", ctypes.c_int32), ("my_size", ctypes.c_int64),
                ("weights", ctypes.c_void_p), ("batch_size_offsets", ctypes.c_void_p),
                ("total_num_blocks", ctypes.c_void_p), ("bucketize_pos", ctypes.c_void_p),
                ("bucketize_pos_len", ctypes.c_void_p), ("new_lengths", ctypes.c_void_p),
                ("new_offsets", ctypes.c_void_p), ("new_indices", ctypes.c_void_p),
                ("new_weights", ctypes.c_void_p), ("new_pos", ctypes.c_void_p),
                ("unbucketize_permute", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
                ("workspace_bytes", ctypes.c_int64), ("lengths", ctypes.c_void_p)]


_lib = None


def lib_path() -> str:
    """The libtbe_hip.so this binding loads: the package's own, or the build named by
    TBE_HIP_LIB (e.g. the host-sanitizer build of build.py --sanitize)."""
    return os.environ.get("TBE_HIP_LIB") or HIP_LIB


def lib():
    """Load libtbe_hip.so (loading needs no GPU; launching does)."""
    global _lib
    if _lib is None:
        path = lib_path()
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built")
        L = ctypes.CDLL(path)
        L.tbe_nbit_plan.restype = ctypes.c_int
        L.tbe_nbit_plan.argtypes = [ctypes.POINTER(TbePlanInput), ctypes.POINTER(TbeTableDesc),
                                    ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(TbePlanSummary)]
        L.tbe_nbit_forward.restype = ctypes.c_int
        L.tbe_nbit_forward.argtypes = [ctypes.POINTER(TbeNbitArgs), ctypes.c_void_p]
        L.tbe_last_error.restype = ctypes.c_char_p
        L.tbe_last_error.argtypes = []
        L.tbe_nbit_abi_version.restype = ctypes.c_int
        L.tbe_nbit_abi_version.argtypes = []
        L.tbe_permute_pooled_embs.restype = ctypes.c_int
        L.tbe_permute_pooled_embs.argtypes = [ctypes.POINTER(TbePermutePooledArgs), ctypes.c_void_p]
        L.tbe_block_bucketize_workspace_bytes.restype = ctypes.c_int64
        L.tbe_block_bucketize_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int32]
        L.tbe_block_bucketize_sparse_features.restype = ctypes.c_int
        L.tbe_block_bucketize_sparse_features.argtypes = [ctypes.POINTER(TbeBlockBucketizeArgs), ctypes.c_void_p]
        L.tbe_block_bucketize_sparse_features_noalloc.restype = ctypes.c_int
        L.tbe_block_bucketize_sparse_features_noalloc.argtypes = [ctypes.POINTER(TbeBlockBucketizeArgs),
                                                                  ctypes.c_void_p]
        _lib = L
    return _lib


class TbeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def last_error() -> str:
    return lib().tbe_last_error().decode()


def plan(weights_offsets, weights_tys, D_offsets, dev_weights_bytes: int, row_alignment: int = 16,
         fp8_exponent_bits: int = -1, fp8_exponent_bias: int = -1):
    """Host planner.  Returns (descs: ctypes array of TbeTableDesc, order: int32 numpy
    array, summary: TbePlanSummary)."""
    wo = np.ascontiguousarray(weights_offsets, dtype=np.int64)
    wt = np.ascontiguousarray(weights_tys, dtype=np.uint8)
    do = np.ascontiguousarray(D_offsets, dtype=np.int32)
    T = int(wo.size)
    inp = TbePlanInput(T, wo.ctypes.data, wt.ctypes.data, do.ctypes.data, int(dev_weights_bytes),
                       int(row_alignment), int(fp8_exponent_bits), int(fp8_exponent_bias))
    descs = (TbeTableDesc * max(T, 1))()
    order = np.zeros(max(T, 1), dtype=np.int32)
    summary = TbePlanSummary()
    rc = lib().tbe_nbit_plan(ctypes.byref(inp), descs,
                             order.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), ctypes.byref(summary))
    if rc != TBE_OK:
        raise TbeError(rc, last_error())
    return descs, order[:T], summary


def descs_to_bytes(descs) -> bytes:
    return ctypes.string_at(ctypes.addressof(descs), ctypes.sizeof(descs))


def forward(args: TbeNbitArgs, stream: int = 0) -> None:
    rc = lib().tbe_nbit_forward(ctypes.byref(args), ctypes.c_void_p(stream))
    if rc != TBE_OK:
        raise TbeError(rc, last_error())


def forward_tensors(dev_weights, weights_offsets, weights_tys, D_offsets, indices, offsets,
                    pooling_mode: int, indice_weights=None, output_dtype: int = 0,
                    row_alignment: int = 16, fp8_exponent_bits: int = -1,
                    fp8_exponent_bias: int = -1, flags: int = 0, out=None):
    """Run the op through the C ABI on torch device tensors (plan + upload + launch).

    Allocates the output with torch (zero-filled) unless `out` is given."""
    return prepare_forward(dev_weights, weights_offsets, weights_tys, D_offsets, indices, offsets, pooling_mode,
                           indice_weights, output_dtype, row_alignment, fp8_exponent_bits, fp8_exponent_bias,
                           flags, out)()


def prepare_forward(dev_weights, weights_offsets, weights_tys, D_offsets, indices, offsets,
                    pooling_mode: int, indice_weights=None, output_dtype: int = 0,
                    row_alignment: int = 16, fp8_exponent_bits: int = -1,
                    fp8_exponent_bias: int = -1, flags: int = 0, out=None):
    """Plan, upload the plan and allocate the output once; returns a callable that
    launches the forward through the C ABI on the current stream and returns the
    output tensor (the same tensor on every call)."""
    import torch

    wo = weights_offsets.detach().cpu().numpy()
    wt = weights_tys.detach().cpu().numpy()
    do = D_offsets.detach().cpu().numpy()
    descs, order, s = plan(wo, wt, do, dev_weights.numel(), row_alignment, fp8_exponent_bits,
                           fp8_exponent_bias)
    dev = dev_weights.device
    tables = torch.from_numpy(np.frombuffer(descs_to_bytes(descs), dtype=np.uint8).copy()).to(dev)
    order_d = torch.from_numpy(order.copy()).to(dev)
    T = int(wo.size)
    B = (offsets.numel() - 1) // T
    out_dt = {0: torch.float32, 1: torch.float16, 5: torch.bfloat16}.get(int(output_dtype), torch.uint8)
    if out is None:
        shape = (indices.numel(), s.max_D) if pooling_mode == 2 else (B, s.total_D)
        out = torch.zeros(shape, dtype=out_dt, device=dev)
    a = TbeNbitArgs()
    a.dev_weights = dev_weights.data_ptr()
    a.tables = tables.data_ptr()
    a.table_order = order_d.data_ptr()
    a.plan = ctypes.pointer(s)
    a.T = T
    a.max_col_tiles = s.max_col_tiles
    a.B = B
    a.indices = indices.data_ptr()
    a.offsets = offsets.data_ptr()
    a.index_size = indices.element_size()
    a.pooling_mode = int(pooling_mode)
    a.num_indices = indices.numel()
    a.indice_weights = indice_weights.data_ptr() if indice_weights is not None else None
    a.output_dtype = int(output_dtype)
    a.fp8_exponent_bits = int(fp8_exponent_bits)
    a.fp8_exponent_bias = int(fp8_exponent_bias)
    a.flags = int(flags)
    a.output = out.data_ptr()
    a.output_stride = out.shape[1]
    out._tbe_keepalive = (tables, order_d)  # the plan arrays must outlive the async launches

    def launch():
        forward(a, torch.cuda.current_stream(dev).cuda_stream)
        return out
    return launch


def permute_pooled_embs(pooled_embs, offset_dim_list, permute_list, inv_offset_dim_list, out=None):
    """tbe_permute_pooled_embs on torch device tensors (the lists: int64 device tensors)."""
    import torch

    x = pooled_embs.contiguous()
    if out is None:
        out = torch.empty_like(x)
    a = TbePermutePooledArgs()
    a.pooled_embs = x.data_ptr()
    a.output = out.data_ptr()
    a.B = x.shape[0]
    a.total_D = x.shape[1]
    a.inner = x.numel() // max(1, x.shape[0] * x.shape[1])
    a.elem_size = x.element_size()
    a.T = permute_list.numel()
    a.offset_dim_list = offset_dim_list.data_ptr()
    a.permute_list = permute_list.data_ptr()
    a.inv_offset_dim_list = inv_offset_dim_list.data_ptr()
    stream = torch.cuda.current_stream(x.device).cuda_stream if x.is_cuda else 0
    rc = lib().tbe_permute_pooled_embs(ctypes.byref(a), ctypes.c_void_p(stream))
    if rc != TBE_OK:
        raise TbeError(rc, last_error())
    return out


def block_bucketize_sparse_features(lengths, indices, bucketize_pos, sequence, block_sizes, my_size,
                                    weights=None, batch_size_per_feature=None, block_bucketize_pos=None,
                                    keep_orig_idx=False, total_num_blocks=None, noalloc=False, sync=True,
                                    pass_offsets=True):
    """tbe_block_bucketize_sparse_features on torch device tensors; returns the op's
    five outputs (None where not requested) plus new_offsets.  noalloc=True calls
    tbe_block_bucketize_sparse_features_noalloc instead (no workspace passed).
    sync=False returns without waiting for the launches (the temporaries the call
    reads are kept alive by new_offsets until it is freed).  pass_offsets=False hands
    the lengths to the library instead of their cumsum (the torch op's way)."""
    import torch

    dev = indices.device
    L, N, F = lengths.numel(), indices.numel(), block_sizes.numel()
    lopt = dict(dtype=lengths.dtype, device=dev)
    lengths = lengths.contiguous()
    offsets = torch.cumsum(lengths, 0, dtype=lengths.dtype).contiguous() if pass_offsets else None
    bso = None
    if batch_size_per_feature is not None:
        bso = torch.cat([torch.zeros(1, **lopt),
                         torch.cumsum(batch_size_per_feature, 0, dtype=lengths.dtype)]).contiguous()
    new_lengths = torch.empty(my_size * L, **lopt)
    new_offsets = torch.empty(my_size * L + 1, **lopt)
    new_indices = torch.empty(N, dtype=indices.dtype, device=dev)
    new_w = torch.empty(N, dtype=torch.float32, device=dev) if weights is not None else None
    new_pos = torch.empty_like(new_indices) if bucketize_pos else None
    unb = torch.empty_like(new_indices) if sequence else None
    keep = [offsets, bso, lengths]
    pos_ptrs = pos_lens = None
    if block_bucketize_pos is not None:
        ps = [p.contiguous() for p in block_bucketize_pos]
        keep += ps
        pos_ptrs = torch.tensor([p.data_ptr() for p in ps], dtype=torch.int64, device=dev)
        pos_lens = torch.tensor([p.numel() for p in ps], dtype=torch.int64, device=dev)
    wsb = 0 if noalloc else lib().tbe_block_bucketize_workspace_bytes(my_size, L, lengths.element_size())
    ws = None if noalloc else torch.empty(max(1, wsb), dtype=torch.uint8, device=dev)
    a = TbeBlockBucketizeArgs()
    ptr = lambda x: x.data_ptr() if x is not None else None  # noqa: E731
    a.indices, a.num_indices, a.offsets, a.lengths_size = ptr(indices), N, ptr(offsets), L
    a.index_size, a.offset_size = indices.element_size(), lengths.element_size()
    a.block_sizes, a.num_features, a.keep_orig_idx, a.my_size = ptr(block_sizes), F, int(keep_orig_idx), my_size
    a.weights, a.batch_size_offsets = ptr(weights), ptr(bso)
    a.total_num_blocks, a.bucketize_pos, a.bucketize_pos_len = ptr(total_num_blocks), ptr(pos_ptrs), ptr(pos_lens)
    a.new_lengths, a.new_offsets, a.new_indices = ptr(new_lengths), ptr(new_offsets), ptr(new_indices)
    a.new_weights, a.new_pos, a.unbucketize_permute = ptr(new_w), ptr(new_pos), ptr(unb)
    a.workspace, a.workspace_bytes = ptr(ws), wsb
    a.lengths = ptr(lengths)
    stream = torch.cuda.current_stream(dev).cuda_stream if indices.is_cuda else 0
    fn = lib().tbe_block_bucketize_sparse_features_noalloc if noalloc else lib().tbe_block_bucketize_sparse_features
    rc = fn(ctypes.byref(a), ctypes.c_void_p(stream))
    if rc != TBE_OK:
        raise TbeError(rc, last_error())
    # the temporaries above must outlive the launches; under graph capture they stay
    # in the graph's memory pool, reused only by work captured after these launches
    if not sync:
        new_offsets._tbe_keep = (keep, ws, pos_ptrs, pos_lens)
    elif not (indices.is_cuda and torch.cuda.is_current_stream_capturing()):
        torch.cuda.synchronize(dev)
    del keep, ws, pos_ptrs, pos_lens
    return (new_lengths, new_indices, new_w, new_pos, unb), new_offsets
