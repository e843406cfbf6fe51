"""ctypes binding of the C ABIs declared in include/tbe_nbit.h and
include/tbe_pooled_ops.h (libtbe_hip.so).

This is the same boundary a cgo/JNI/N-API binding would use; the GPU parity
tests call the kernels through it directly, without the torch dispatcher.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import HIP_LIB

ABI_VERSION = 2
EXPORTS = ("tbe_nbit_plan", "tbe_nbit_forward", "tbe_last_error", "tbe_nbit_abi_version",
           "tbe_permute_pooled_embs")

TBE_OK, TBE_ERR_INVALID_ARG, TBE_ERR_UNSUPPORTED, TBE_ERR_LAUNCH = 0, -1, -2, -3
TBE_FLAG_NO_XCD_REMAP = 0x1
TBE_TABLE_OFFSET32 = 0x1


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
                ("col_tiles", ctypes.c_int32)]


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


_lib = None


def lib():
    """Load libtbe_hip.so (loading needs no GPU; launching does)."""
    global _lib
    if _lib is None:
        if not os.path.exists(HIP_LIB):
            raise FileNotFoundError(f"{HIP_LIB} is not built")
        L = ctypes.CDLL(HIP_LIB)
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
    stream = torch.cuda.current_stream(dev).cuda_stream
    forward(a, stream)
    out._tbe_keepalive = (tables, order_d)  # the plan arrays must outlive the async launch
    return out


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
