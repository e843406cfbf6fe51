"""Type and pooling codes of the TBE op (reference A:18-33, c310/op_kernel/common.h:44-67)
plus the row-layout rules of each weight type (fbgemm_gpu's layout, which the
reference test uses through IntNBitTableBatchedEmbeddingBagsCodegen, T:121-141)."""
from __future__ import annotations

import enum


class SparseType(enum.IntEnum):
    FP32 = 0
    FP16 = 1
    INT8 = 2
    INT4 = 3
    INT2 = 4
    BF16 = 5
    FP8 = 6

    def as_int(self) -> int:
        return int(self)

    def bit_rate(self) -> int:
        return {0: 32, 1: 16, 2: 8, 3: 4, 4: 2, 5: 16, 6: 8}[int(self)]

    def align_size(self) -> int:
        """Smallest D granularity for which a row fills whole 4-byte words."""
        return {0: 1, 1: 2, 2: 4, 3: 8, 4: 16, 5: 2, 6: 4}[int(self)]

    def has_scale_bias(self) -> bool:
        return self in (SparseType.INT8, SparseType.INT4, SparseType.INT2)


class PoolingMode(enum.IntEnum):
    SUM = 0
    MEAN = 1
    NONE = 2


def unpadded_row_bytes(ty: SparseType, D: int) -> int:
    ty = SparseType(ty)
    return (D * ty.bit_rate() + 7) // 8 + (4 if ty.has_scale_bias() else 0)


def row_stride(ty: SparseType, D: int, row_alignment: int = 16) -> int:
    u = unpadded_row_bytes(ty, D)
    return (u + row_alignment - 1) // row_alignment * row_alignment
