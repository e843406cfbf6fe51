"""fbgemm-ascend_amd: MI355X-native quantized TBE inference forward.

Importing the package makes torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function
run on HIP tensors, like `import fbgemm_ascend` does for NPU tensors (reference
fbgemm_ascend/__init__.py:9 and :189-231).  The reference relies on fbgemm_gpu
to define the op schema; when fbgemm_gpu is absent this package defines the
identical schema itself.

The directory name contains a hyphen, so load it with `load_package()` below
(or importlib) under the module name `fbgemm_ascend_amd`.
"""
from __future__ import annotations

import importlib.machinery
import importlib.util
import os

import torch

__version__ = "0.1.0"

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(PKG_DIR, "libtbe_hip.so")
TORCH_LIB = os.path.join(PKG_DIR, "_tbe_torch.so")

OP_NAME = "int_nbit_split_embedding_codegen_lookup_function"
# Same schema as fbgemm_gpu's (reference call site T:94-118, adapter A:55-78).
OP_SCHEMA = (
    "int_nbit_split_embedding_codegen_lookup_function("
    "Tensor dev_weights, Tensor uvm_weights, Tensor weights_placements, Tensor weights_offsets, "
    "Tensor weights_tys, Tensor D_offsets, int total_D, int max_int2_D, int max_int4_D, "
    "int max_int8_D, int max_float16_D, int max_float32_D, Tensor indices, Tensor offsets, "
    "int pooling_mode, Tensor? indice_weights, int output_dtype, Tensor? lxu_cache_weights, "
    "Tensor? lxu_cache_locations, int? row_alignment, int? max_float8_D, "
    "int? fp8_exponent_bits, int? fp8_exponent_bias) -> Tensor"
)

# Reference: src/pooled_embedding_ops/permute_pooled_embs/permute_pooled_embs.cpp:107-121
# (fbgemm_gpu's schema, also exposed in the mxrec namespace).
PERMUTE_POOLED_EMBS_SCHEMA = (
    "permute_pooled_embs(Tensor pooled_embs, Tensor offset_dim_list, Tensor permute_list, "
    "Tensor inv_offset_dim_list, Tensor inv_permute_list) -> Tensor"
)

# Reference: src/sparse_ops/block_bucketize_sparse_features/block_bucketize_sparse_features.cpp:248-254
BLOCK_BUCKETIZE_SCHEMA = (
    "block_bucketize_sparse_features(Tensor lengths, Tensor indices, bool bucketize_pos, bool sequence, "
    "Tensor block_sizes, SymInt my_size, Tensor? weights=None, Tensor? batch_size_per_feature=None, "
    "SymInt max_B= -1, Tensor[]? block_bucketize_pos=None, bool keep_orig_idx=False, "
    "Tensor? total_num_blocks=None) -> (Tensor, Tensor, Tensor?, Tensor?, Tensor?)"
)

# (namespace, op name, schema) of every op this package implements for HIP tensors
SCHEMAS = [
    ("fbgemm", OP_NAME, OP_SCHEMA),
    ("fbgemm", "permute_pooled_embs", PERMUTE_POOLED_EMBS_SCHEMA),
    ("mxrec", "permute_pooled_embs", PERMUTE_POOLED_EMBS_SCHEMA),
    ("fbgemm", "block_bucketize_sparse_features", BLOCK_BUCKETIZE_SCHEMA),
    ("mxrec", "block_bucketize_sparse_features", BLOCK_BUCKETIZE_SCHEMA),
]

_schema_libs = []
_loaded = False
_ext = None  # _tbe_torch.so imported as a Python extension module (BoundLookup)


def _op_defined(qualname: str) -> bool:
    try:
        torch._C._dispatch_find_schema_or_throw(qualname, "")
        return True
    except RuntimeError:
        return False


def _define_schema() -> None:
    """Define each schema that no other library (e.g. fbgemm_gpu) has defined."""
    libs = {}
    for ns, name, schema in SCHEMAS:
        if _op_defined(f"{ns}::{name}"):
            continue
        if ns not in libs:
            libs[ns] = torch.library.Library(ns, "FRAGMENT")
            _schema_libs.append(libs[ns])
        libs[ns].define(schema)


def load_library() -> None:
    """Define the schema (if needed) and register the HIP implementation.

    Raises if the built extension is missing: there is no CPU fallback."""
    global _loaded
    if _loaded:
        return
    if not os.path.exists(TORCH_LIB) or not os.path.exists(HIP_LIB):
        raise FileNotFoundError(
            f"fbgemm_ascend_amd: built extension not found ({TORCH_LIB}); "
            "run fbgemm-ascend_amd/build.py (or __graft_entry__.build()) first")
    _define_schema()
    torch.ops.load_library(TORCH_LIB)
    global _ext
    name = f"{__name__}._tbe_torch"
    loader = importlib.machinery.ExtensionFileLoader(name, TORCH_LIB)
    spec = importlib.util.spec_from_file_location(name, TORCH_LIB, loader=loader)
    _ext = importlib.util.module_from_spec(spec)
    loader.exec_module(_ext)
    _loaded = True


load_library()

from . import capi  # noqa: E402,F401
from .sparse_types import PoolingMode, SparseType  # noqa: E402,F401
from .tbe_module import IntNBitTableBatchedEmbeddingBagsCodegen, fp8_code_values, fp8_quantize  # noqa: E402,F401
from .permute_pooled_embedding_modules import PermutePooledEmbeddings  # noqa: E402,F401


def int_nbit_split_embedding_codegen_lookup_function(**kwargs):
    """Keyword passthrough to the registered torch op."""
    return torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(**kwargs)
