"""Module-level packer: the on-device weight format callers build.

`IntNBitTableBatchedEmbeddingBagsCodegen` mirrors the fbgemm_gpu module of the
same name as the reference test uses it (T:121-156, T:88-118): it lays out all
tables' rows back to back in one uint8 buffer and exposes the tensors the op
takes (weights_dev, weights_offsets, weights_tys, D_offsets, total_D,
max_*_D, row_alignment, fp8 parameters).

Row formats (fbgemm_gpu layout; the reference kernel reads FP8 rows only, P:235-278):
  INT8/INT4/INT2: [fp16 scale][fp16 bias][codes, low bits first], value = scale*q + bias
  FP8:            D one-byte codes (exponent_bits / exponent_bias), no header (P:241)
  FP16/BF16/FP32: D plain values
Each row is padded to a multiple of row_alignment bytes (default 16, A:86).
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from .sparse_types import PoolingMode, SparseType, row_stride


def fp8_code_values(exponent_bits: int, exponent_bias: int) -> torch.Tensor:
    """fp32 values of the 128 non-negative FP8 codes 0x00..0x7F, increasing.

    Format of c310/op_kernel/common.h:120-167: a code is [sign][exponent_bits
    exponent bits E][m = 7 - exponent_bits mantissa bits M]; E > 0 is the normal
    value 2^(E - bias) * (1 + M / 2^m), E = 0 the subnormal 2^(1 - bias) * M / 2^m.
    No Inf / NaN codes.
    """
    if not (1 <= exponent_bits <= 7 and 0 <= exponent_bias <= 120):
        raise ValueError(f"bad FP8 parameters ({exponent_bits}, {exponent_bias})")
    m = 7 - exponent_bits
    code = torch.arange(128, dtype=torch.float64)
    E = torch.div(code, 1 << m, rounding_mode="floor")
    M = code - E * (1 << m)
    normal = torch.exp2(E - exponent_bias) * (1 + M / (1 << m))
    sub = 2.0 ** (1 - exponent_bias) * M / (1 << m)
    return torch.where(E > 0, normal, sub).to(torch.float32)


def fp8_quantize(w: torch.Tensor, exponent_bits: int, exponent_bias: int) -> torch.Tensor:
    """Nearest FP8 code of every element (uint8, same shape).  Ties go to the even
    code (even mantissa); magnitudes above the largest code saturate to it; the
    sign bit follows the sign of w (-0.0 keeps it)."""
    vals = fp8_code_values(exponent_bits, exponent_bias).to(w.device, torch.float64)
    x = w.to(torch.float64)
    a = x.abs()
    hi = torch.searchsorted(vals, a).clamp(1, 127)  # vals[hi-1] < a <= vals[hi] inside the range
    lo = hi - 1
    dlo = a - vals[lo]
    dhi = vals[hi] - a
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = torch.where(pick_hi, hi, lo)
    code = torch.where(a >= vals[127], torch.full_like(code, 127), code)
    code = torch.where(a <= vals[0], torch.zeros_like(code), code)
    sign = torch.signbit(x).to(torch.int64) << 7
    return (code | sign).to(torch.uint8)


def _spec_fields(spec) -> Tuple[int, int, SparseType]:
    # accepts (E, D, ty) or fbgemm's (name, E, D, ty, location)
    if len(spec) == 3:
        E, D, ty = spec
    else:
        _, E, D, ty = spec[:4]
    return int(E), int(D), SparseType(int(ty))


# Attributes bound into the module's BoundLookup: setting one drops the binding.
_BOUND_FIELDS = frozenset((
    "weights_dev", "weights_uvm", "weights_placements", "weights_offsets", "weights_tys", "D_offsets",
    "total_D", "max_int2_D", "max_int4_D", "max_int8_D", "max_float16_D", "max_float32_D", "max_float8_D",
    "pooling_mode", "output_dtype", "row_alignment", "fp8_exponent_bits", "fp8_exponent_bias"))


class IntNBitTableBatchedEmbeddingBagsCodegen(torch.nn.Module):
    def __init__(self, embedding_specs: Sequence, device="cuda", pooling_mode=PoolingMode.SUM,
                 output_dtype=SparseType.FP16, indices_dtype=torch.int32, row_alignment: int = 16,
                 fp8_exponent_bits: Optional[int] = None, fp8_exponent_bias: Optional[int] = None):
        super().__init__()
        self.specs = [_spec_fields(s) for s in embedding_specs]
        if not self.specs:
            raise ValueError("at least one table is required")
        self.device_ = torch.device(device)
        self.pooling_mode = PoolingMode(int(pooling_mode))
        self.output_dtype = int(output_dtype)
        self.indices_dtype = indices_dtype
        self.row_alignment = int(row_alignment)
        for E, D, ty in self.specs:
            if D % ty.align_size():
                raise ValueError(f"D={D} is not a multiple of {ty.align_size()} for {ty.name}")
        has_fp8 = any(ty == SparseType.FP8 for _, _, ty in self.specs)
        if has_fp8:
            self.fp8_exponent_bits = 4 if fp8_exponent_bits is None else int(fp8_exponent_bits)
            self.fp8_exponent_bias = ((1 << (self.fp8_exponent_bits - 1)) - 1
                                      if fp8_exponent_bias is None else int(fp8_exponent_bias))
        else:
            self.fp8_exponent_bits = -1
            self.fp8_exponent_bias = -1

        strides, offs, dofs, acc = [], [], [0], 0
        for E, D, ty in self.specs:
            st = row_stride(ty, D, self.row_alignment)
            strides.append(st)
            offs.append(acc)
            acc += E * st
            dofs.append(dofs[-1] + D)
        self.row_strides = strides
        self.total_D = dofs[-1]

        def max_d(*tys):
            ds = [D for _, D, ty in self.specs if ty in tys]
            return max(ds) if ds else 0

        self.max_int2_D = max_d(SparseType.INT2)
        self.max_int4_D = max_d(SparseType.INT4)
        self.max_int8_D = max_d(SparseType.INT8)
        self.max_float8_D = max_d(SparseType.FP8)
        self.max_float16_D = max_d(SparseType.FP16, SparseType.BF16)
        self.max_float32_D = max_d(SparseType.FP32)

        dev = self.device_
        self.register_buffer("weights_dev", torch.zeros(acc, dtype=torch.uint8, device=dev))
        self.register_buffer("weights_uvm", torch.empty(0, dtype=torch.uint8, device=dev))
        self.register_buffer("weights_placements",
                             torch.zeros(len(self.specs), dtype=torch.int32, device=dev))
        self.register_buffer("weights_offsets", torch.tensor(offs, dtype=torch.int64, device=dev))
        self.register_buffer("weights_tys", torch.tensor([int(t) for _, _, t in self.specs],
                                                         dtype=torch.uint8, device=dev))
        self.register_buffer("D_offsets", torch.tensor(dofs, dtype=torch.int32, device=dev))
        self._offs = offs

    # ------------------------------------------------------------------ layout views
    def table_rows(self, t: int) -> torch.Tensor:
        """uint8 [E, row_stride] view of table t's rows."""
        E, _, _ = self.specs[t]
        st = self.row_strides[t]
        return self.weights_dev[self._offs[t]: self._offs[t] + E * st].view(E, st)

    def split_embedding_weights(self) -> List[Tuple[torch.Tensor, Optional[torch.Tensor]]]:
        """Per table (payload view [E, payload bytes], scale/bias view [E, 4] or None)."""
        out = []
        for t, (E, D, ty) in enumerate(self.specs):
            rows = self.table_rows(t)
            hdr = 4 if ty.has_scale_bias() else 0
            payload = (D * ty.bit_rate() + 7) // 8
            out.append((rows[:, hdr:hdr + payload], rows[:, :4] if hdr else None))
        return out

    # ------------------------------------------------------------------ weight fill
    @torch.no_grad()
    def fill_random_weights(self, seed: int = 0) -> None:
        """Codes uniform over their range; fp16 scale U(0.001, 0.01), fp16 bias U(-1, 1);
        float rows U(-1, 1); FP8 codes uniform over all 256 patterns."""
        g = torch.Generator(device=self.device_)
        g.manual_seed(seed)
        for t, (E, D, ty) in enumerate(self.specs):
            payload, sb = self.split_embedding_weights()[t]
            if ty in (SparseType.INT8, SparseType.INT4, SparseType.INT2, SparseType.FP8):
                payload.copy_(torch.randint(0, 256, payload.shape, dtype=torch.uint8,
                                            device=self.device_, generator=g))
            else:
                fdt = {SparseType.FP16: torch.float16, SparseType.BF16: torch.bfloat16,
                       SparseType.FP32: torch.float32}[ty]
                vals = torch.rand((E, D), device=self.device_, generator=g) * 2 - 1
                payload.copy_(vals.to(fdt).view(torch.uint8).view(E, -1))
            if sb is not None:
                scale = torch.rand(E, device=self.device_, generator=g) * 0.009 + 0.001
                bias = torch.rand(E, device=self.device_, generator=g) * 2 - 1
                hb = torch.stack([scale, bias], dim=1).to(torch.float16).contiguous()
                sb.copy_(hb.view(torch.uint8).view(E, 4))

    @torch.no_grad()
    def load_float_weights(self, t: int, weight: torch.Tensor) -> None:
        """Quantize a float [E, D] table into table t (row-wise min/max for INT types:
        scale = (max-min)/(2^bits-1), bias = min, q = round((w-bias)/scale), with scale
        and bias stored as fp16; FP8: the nearest code under the module's
        (fp8_exponent_bits, fp8_exponent_bias), see fp8_quantize; FP16/BF16/FP32: a
        cast)."""
        E, D, ty = self.specs[t]
        w = weight.to(self.device_, torch.float32)
        if tuple(w.shape) != (E, D):
            raise ValueError(f"table {t} expects [{E}, {D}], got {tuple(w.shape)}")
        payload, sb = self.split_embedding_weights()[t]
        if ty in (SparseType.FP16, SparseType.BF16, SparseType.FP32):
            fdt = {SparseType.FP16: torch.float16, SparseType.BF16: torch.bfloat16,
                   SparseType.FP32: torch.float32}[ty]
            payload.copy_(w.to(fdt).view(torch.uint8).view(E, -1))
            return
        if ty == SparseType.FP8:
            codes = fp8_quantize(w, self.fp8_exponent_bits, self.fp8_exponent_bias)
            payload.copy_(codes)
            return
        bits = ty.bit_rate()
        lo = w.min(dim=1).values
        hi = w.max(dim=1).values
        scale = ((hi - lo) / ((1 << bits) - 1)).to(torch.float16)
        bias = lo.to(torch.float16)
        s32 = scale.float().clamp_min(1e-8)
        q = torch.round((w - bias.float()[:, None]) / s32[:, None]).clamp(0, (1 << bits) - 1)
        q = q.to(torch.int32)
        per = 8 // bits
        q = q.view(E, D // per, per)
        packed = torch.zeros(E, D // per, dtype=torch.int32, device=self.device_)
        for j in range(per):
            packed |= q[:, :, j] << (bits * j)
        payload.copy_(packed.to(torch.uint8))
        sb.copy_(torch.stack([scale, bias], 1).contiguous().view(torch.uint8).view(E, 4))

    # ------------------------------------------------------------------ forward
    def _bind(self):
        """The op's arguments that do not change between calls, bound once in C++
        (`BoundLookup`): a forward then passes three arguments instead of packing
        23 into the dispatcher's boxed form, which costs more host time than the
        launch itself on small batches.  Same function, checks and plan cache as
        torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function."""
        from . import _ext
        b = _ext.BoundLookup(self.weights_dev, self.weights_uvm, self.weights_placements, self.weights_offsets,
                             self.weights_tys, self.D_offsets, self.total_D, self.max_int2_D, self.max_int4_D,
                             self.max_int8_D, self.max_float16_D, self.max_float32_D, int(self.pooling_mode),
                             self.output_dtype, self.row_alignment, self.max_float8_D, self.fp8_exponent_bits,
                             self.fp8_exponent_bias)
        self.__dict__["_bound"] = b
        return b

    def __setattr__(self, name, value):
        if name in _BOUND_FIELDS:
            self.__dict__["_bound"] = None
        super().__setattr__(name, value)

    def register_buffer(self, name, tensor, persistent=True):
        if name in _BOUND_FIELDS:
            self.__dict__["_bound"] = None
        super().register_buffer(name, tensor, persistent)

    def _apply(self, fn, *args, **kwargs):
        # .to() / .cuda() / .half() may replace the buffers
        self.__dict__["_bound"] = None
        return super()._apply(fn, *args, **kwargs)

    def __getstate__(self):
        state = self.__dict__.copy()
        state["_bound"] = None  # a C++ object: rebuilt at the first forward
        return state

    def forward(self, indices: torch.Tensor, offsets: torch.Tensor,
                per_sample_weights: Optional[torch.Tensor] = None) -> torch.Tensor:
        b = self.__dict__.get("_bound")
        if b is None:
            b = self._bind()
        return b(indices, offsets, per_sample_weights)
