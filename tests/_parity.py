"""Parity helpers shared by the GPU tests: carve the oracle-sized sub-problem out of
a device-resident workload and compare the GPU output with the oracle's.

Tolerance (stated per BASELINE north star, with the atol that cancellation needs):
    |gpu - ref| <= atol_k + rtol * |ref|,   atol_k = rtol * sum_{i in bag k} |w_i| * max|row_i|
(times 1/L for MEAN), rtol = 1e-5 for fp32 output, 1e-3 for fp16, 2^-7 for bf16
(the reference test's bf16 tolerance, T:358-366).  `ref` is the oracle's fp32 value
before the output cast, so the cast's own rounding is inside rtol.
"""
from __future__ import annotations

import numpy as np
import torch

RTOL = {0: 1e-5, 1: 1e-3, 5: 2.0 ** -7}
FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6


def compact_problem(module, indices, offsets, psw, b_sel=None):
    """Sub-problem holding only the samples b_sel (all if None) and only the rows they
    reference.  Returns a dict of host arrays for the oracle plus the device b_sel."""
    dev = indices.device
    T = len(module.specs)
    B = (offsets.numel() - 1) // T
    if b_sel is None:
        b_sel = torch.arange(B, device=dev)
    b_sel = b_sel.to(dev, torch.int64)
    Bs = b_sel.numel()
    k = (torch.arange(T, device=dev)[:, None] * B + b_sel[None, :]).reshape(-1)
    off64 = offsets.to(torch.int64)
    starts, ends = off64[k], off64[k + 1]
    lens = ends - starts
    new_off = torch.zeros(k.numel() + 1, dtype=torch.int64, device=dev)
    torch.cumsum(lens, 0, out=new_off[1:])
    total = int(new_off[-1])
    bag_of = torch.repeat_interleave(torch.arange(k.numel(), device=dev), lens)
    pos = starts[bag_of] + (torch.arange(total, device=dev) - new_off[bag_of])
    idx = indices[pos].to(torch.int64)
    w = psw[pos].float() if psw is not None else None
    new_idx = torch.full_like(idx, -1)
    blocks, woffs, acc = [], [], 0
    rowmax = []
    for t, (E, D, ty) in enumerate(module.specs):
        lo, hi = int(new_off[t * Bs]), int(new_off[(t + 1) * Bs])
        it = idx[lo:hi]
        valid = (it >= 0) & (it < E)
        uniq, inv = torch.unique(it[valid], return_inverse=True)
        sub = torch.full_like(it, -1)
        sub[valid] = inv
        new_idx[lo:hi] = sub
        rows = module.table_rows(t)[uniq].cpu().numpy()
        blocks.append(rows.reshape(-1))
        woffs.append(acc)
        acc += rows.size
        rowmax.append(_row_magnitude(rows, D, ty, module))
    return dict(
        weights=np.concatenate(blocks) if blocks else np.zeros(0, np.uint8),
        weights_offsets=np.array(woffs, np.int64),
        weights_tys=module.weights_tys.cpu().numpy(),
        D_offsets=module.D_offsets.cpu().numpy(),
        indices=new_idx.cpu().numpy(),
        offsets=new_off.cpu().numpy(),
        psw=None if w is None else w.cpu().numpy(),
        rowmax=rowmax, B=Bs, b_sel=b_sel, lengths=lens.cpu().numpy(),
        fp8=(module.fp8_exponent_bits, module.fp8_exponent_bias),
    )


def _row_magnitude(rows: np.ndarray, D: int, ty: int, module) -> np.ndarray:
    """Upper bound of max_d |value| of each row."""
    n = rows.shape[0]
    if n == 0:
        return np.zeros(0, np.float64)
    if ty in (INT8, INT4, INT2):
        bits = {INT8: 8, INT4: 4, INT2: 2}[ty]
        sc = rows[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
        bi = rows[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
        return np.abs(sc) * ((1 << bits) - 1) + np.abs(bi)
    if ty == FP16:
        v = rows[:, :2 * D].copy().view(np.float16).astype(np.float64)
    elif ty == BF16:
        v = (rows[:, :2 * D].copy().view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    elif ty == FP32:
        v = rows[:, :4 * D].copy().view(np.float32).astype(np.float64)
    else:  # FP8: |value| <= 2^(2^e - 1 - bias) * 2
        e, bias = module.fp8_exponent_bits, module.fp8_exponent_bias
        return np.full(n, 2.0 ** ((1 << e) - 1 - bias) * 2.0)
    return np.abs(v).max(axis=1)


def run_oracle(oracle, prob, pooling_mode, output_dtype, row_alignment=16):
    bits, bias = prob["fp8"]
    return oracle.forward(prob["weights"], prob["weights_offsets"], prob["weights_tys"], prob["D_offsets"],
                          prob["indices"], prob["offsets"], pooling_mode, prob["psw"], output_dtype,
                          row_alignment=row_alignment, fp8_exponent_bits=bits, fp8_exponent_bias=bias)


F16_MAX = 65504.0         # largest finite half
F16_INF_FROM = 65520.0    # half-way to the next power of two: RNE rounds here and above to inf


def bag_tolerance(prob, pooling_mode, output_dtype):
    """atol per output element [B', total_D]."""
    rtol = RTOL[output_dtype]
    T = len(prob["weights_tys"])
    B = prob["B"]
    dofs = prob["D_offsets"]
    idx, off = prob["indices"], prob["offsets"]
    w = np.abs(prob["psw"]) if prob["psw"] is not None else np.ones(idx.size)
    atol = np.zeros((B, int(dofs[-1])), np.float64)
    for t in range(T):
        lo, hi = int(off[t * B]), int(off[(t + 1) * B])
        it = idx[lo:hi]
        rm = np.where(it >= 0, prob["rowmax"][t][np.maximum(it, 0)] if len(prob["rowmax"][t]) else 0.0, 0.0)
        contrib = rm * w[lo:hi]
        csum = np.concatenate([[0.0], np.cumsum(contrib)])
        bag_off = off[t * B:(t + 1) * B + 1] - lo
        m = csum[bag_off[1:]] - csum[bag_off[:-1]]
        if pooling_mode == 1:
            L = np.maximum(bag_off[1:] - bag_off[:-1], 1)
            m = m / L
        atol[:, dofs[t]:dofs[t + 1]] = (rtol * m)[:, None]
    return atol + 1e-30


def to_f32(out: torch.Tensor) -> np.ndarray:
    return out.float().cpu().numpy()


def assert_bag_parity(gpu_out, prob, ref32, pooling_mode, output_dtype, label=""):
    got = to_f32(gpu_out)
    if pooling_mode == 2:
        rtol = RTOL[output_dtype]
        atol = rtol * np.abs(ref32).max(initial=0.0) * 1e-3 + 1e-30
    else:
        atol = bag_tolerance(prob, pooling_mode, output_dtype)
        rtol = RTOL[output_dtype]
    r64 = ref32.astype(np.float64)
    err = np.abs(got.astype(np.float64) - r64)
    lim = atol + rtol * np.abs(r64)
    bad = err > lim
    if output_dtype == 1:
        # fp16 out: the round-to-nearest-even cast (P:330) takes sums from 65520 up to
        # +-inf and sums from 65504 to 65520 to +-65504; near those bounds the fp32
        # summation order may land on either side
        a = np.abs(r64)
        same_sign = np.sign(got) == np.sign(r64)
        must_inf = a >= F16_INF_FROM * (1 + rtol)
        near = a >= F16_MAX * (1 - rtol)
        edge_ok = near & ~must_inf & same_sign & (np.isinf(got) | (np.abs(got) >= F16_MAX * (1 - rtol)))
        inf_ok = must_inf & same_sign & np.isinf(got)
        bad = (bad & ~edge_ok & ~inf_ok) | (must_inf & ~inf_ok)
        err = np.where(edge_ok | inf_ok, 0.0, err)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{label}: {int(bad.sum())}/{bad.size} elements out of tolerance; first at {tuple(i)}: "
            f"gpu={got[tuple(i)]!r} ref={ref32[tuple(i)]!r} lim={lim[tuple(i)]:.3e}")
    return float((err / np.maximum(lim, 1e-30)).max(initial=0.0))


def ulp_stats(gpu_out: torch.Tensor, ref_out: np.ndarray, output_dtype: int):
    """Distance between the GPU output and the oracle's output in units in the last place
    of the output dtype (bit patterns mapped to a monotonic integer scale): returns
    (max distance, fraction of elements bit-identical)."""
    if output_dtype == 0:  # fp32
        a = gpu_out.float().cpu().numpy().view(np.int32).astype(np.int64)
        b = np.ascontiguousarray(ref_out, dtype=np.float32).view(np.int32).astype(np.int64)
        sign = np.int64(1) << 31
    else:                  # fp16 / bf16 bit patterns
        a = gpu_out.cpu().view(torch.int16).numpy().astype(np.int64) & 0xFFFF
        b = np.ascontiguousarray(ref_out).astype(np.int64) & 0xFFFF
        a = np.where(a >= 0x8000, a - 0x10000, a)
        b = np.where(b >= 0x8000, b - 0x10000, b)
        sign = np.int64(1) << 15
    # sign-magnitude -> ordered integers (+0 and -0 both map to 0)
    ka = np.where(a < 0, -(a + sign), a)
    kb = np.where(b < 0, -(b + sign), b)
    d = np.abs(ka - kb)
    return int(d.max(initial=0)), float((d == 0).mean()) if d.size else 1.0
