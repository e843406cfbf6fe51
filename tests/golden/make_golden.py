"""Writes tests/golden/library_vectors.npz: input/output vectors of the TBE op's
arithmetic produced by LIBRARY routines that are independent of this repo's
oracle and kernels:

  * torch.ops.quantized.embedding_bag_{byte,4bit,2bit}_rowwise_offsets (FBGEMM's
    CPU kernels shipped with torch) for INT8/INT4/INT2 rows, after repacking the
    TBE row layout ([fp16 scale][fp16 bias][codes]) to the scale/bias-last layout
    those kernels read;
    (MEAN cases: the library's sum times float(1)/float(L), since those kernels
    return the sum for mode=1);
  * torch.nn.functional.embedding_bag for FP32/FP16/BF16 rows;
  * torch.float8_e4m3fn / torch.float8_e5m2 for the FP8 decode with exponent
    bits/bias (4,7) and (5,15).

The reference repository holds no golden files for this op (its test builds every
input at run time against fbgemm_gpu, which is not installed here), so these
vectors are the committed fixtures.  Regenerate with
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "library_vectors.npz")

FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6
BITS = {INT8: 8, INT4: 4, INT2: 2}


def stride_of(ty, D, align=16):
    hdr = 4 if ty in BITS else 0
    bits = {FP32: 32, FP16: 16, BF16: 16, FP8: 8, **BITS}[ty]
    u = D * bits // 8 + hdr
    return (u + align - 1) // align * align


def make_case(rs: np.random.RandomState, tables, B, mode, weighted):
    """Multi-table TBE problem; expected output from the library routines."""
    T = len(tables)
    blocks, woffs, dofs = [], [], [0]
    pos = 0
    for (E, D, ty) in tables:
        st = stride_of(ty, D)
        buf = np.zeros((E, st), dtype=np.uint8)
        if ty in BITS:
            bits = BITS[ty]
            q = rs.randint(0, 1 << bits, size=(E, D)).astype(np.uint8)
            per = 8 // bits
            packed = np.zeros((E, D // per), dtype=np.uint8)
            for j in range(per):
                packed |= (q[:, j::per] << (bits * j)).astype(np.uint8)
            scale = rs.uniform(0.001, 0.01, size=E).astype(np.float16)
            bias = rs.uniform(-1, 1, size=E).astype(np.float16)
            buf[:, 0:2] = scale.view(np.uint8).reshape(E, 2)
            buf[:, 2:4] = bias.view(np.uint8).reshape(E, 2)
            buf[:, 4:4 + packed.shape[1]] = packed
        else:
            vals = rs.uniform(-1, 1, size=(E, D)).astype(np.float32)
            if ty == FP16:
                buf[:, :2 * D] = vals.astype(np.float16).view(np.uint8).reshape(E, -1)
            elif ty == BF16:
                b16 = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy()
                buf[:, :2 * D] = b16.view(np.uint8).reshape(E, -1)
            else:
                buf[:, :4 * D] = vals.view(np.uint8).reshape(E, -1)
        blocks.append(buf.reshape(-1))
        woffs.append(pos)
        pos += buf.size
        dofs.append(dofs[-1] + D)
    weights = np.concatenate(blocks)
    lengths = rs.randint(0, 9, size=T * B)
    lengths[rs.randint(0, T * B)] = 0  # at least one empty bag
    offsets = np.zeros(T * B + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(lengths)
    idx_parts = []
    for t, (E, D, ty) in enumerate(tables):
        idx_parts.append(rs.randint(0, E, size=int(lengths[t * B:(t + 1) * B].sum())))
    indices = np.concatenate(idx_parts).astype(np.int64)
    psw = rs.uniform(0, 1, size=indices.size).astype(np.float32) if weighted else None

    out = np.zeros((B, dofs[-1]), dtype=np.float32)
    for t, (E, D, ty) in enumerate(tables):
        st = stride_of(ty, D)
        rows = weights[woffs[t]:woffs[t] + E * st].reshape(E, st)
        lo, hi = offsets[t * B], offsets[(t + 1) * B]
        idx_t = torch.from_numpy(indices[lo:hi].copy())
        off_t = torch.from_numpy(offsets[t * B:(t + 1) * B + 1] - lo)
        psw_t = torch.from_numpy(psw[lo:hi].copy()) if weighted else None
        if ty in BITS:
            bits = BITS[ty]
            payload = rows[:, 4:4 + D * bits // 8]
            if ty == INT8:
                sb = np.stack([rows[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0],
                               rows[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]], 1)
                w = np.concatenate([payload, sb.astype(np.float32).view(np.uint8).reshape(E, 8)], 1)
                fn = torch.ops.quantized.embedding_bag_byte_rowwise_offsets
            else:
                w = np.concatenate([payload, rows[:, 0:4]], 1)
                fn = (torch.ops.quantized.embedding_bag_4bit_rowwise_offsets if ty == INT4
                      else torch.ops.quantized.embedding_bag_2bit_rowwise_offsets)
            # these kernels ignore mode=1 (they return the sum), so MEAN is the library's
            # sum times float(1)/float(L), the reference's mean rule (P:355)
            res = fn(torch.from_numpy(np.ascontiguousarray(w)), idx_t, off_t, False, 0, False,
                     psw_t, None, True)
            if mode == 1:
                L = (off_t[1:] - off_t[:-1]).numpy()
                inv = np.array([np.float32(1) / np.float32(x) if x else np.float32(1) for x in L],
                               dtype=np.float32)
                res = res * torch.from_numpy(inv)[:, None]
        else:
            if ty == FP16:
                wf = torch.from_numpy(rows[:, :2 * D].copy().view(np.float16)).float()
            elif ty == BF16:
                wf = torch.from_numpy(rows[:, :2 * D].copy().view(np.int16)).view(torch.bfloat16).float()
            else:
                wf = torch.from_numpy(rows[:, :4 * D].copy().view(np.float32))
            res = F.embedding_bag(idx_t, wf, off_t, mode="sum" if mode == 0 else "mean",
                                  per_sample_weights=psw_t, include_last_offset=True)
        out[:, dofs[t]:dofs[t + 1]] = res.numpy()
    return dict(weights=weights, weights_offsets=np.array(woffs, dtype=np.int64),
                weights_tys=np.array([ty for _, _, ty in tables], dtype=np.uint8),
                D_offsets=np.array(dofs, dtype=np.int32), indices=indices, offsets=offsets,
                psw=psw if weighted else np.zeros(0, dtype=np.float32),
                pooling_mode=np.int64(mode), expected=out)


def main():
    rs = np.random.RandomState(20251201)
    arrays = {}
    cases = [
        ("int8_sum", [(40, 16, INT8), (30, 32, INT8)], 0, False),
        ("int8_mean", [(40, 16, INT8), (30, 32, INT8)], 1, False),
        ("int8_wsum", [(40, 16, INT8), (30, 32, INT8)], 0, True),
        ("int4_sum", [(50, 16, INT4), (20, 64, INT4)], 0, False),
        ("int4_mean", [(50, 16, INT4), (20, 64, INT4)], 1, False),
        ("int4_wsum", [(50, 16, INT4), (20, 64, INT4)], 0, True),
        ("int2_sum", [(60, 16, INT2), (25, 32, INT2)], 0, False),
        ("int2_mean", [(60, 16, INT2), (25, 32, INT2)], 1, False),
        ("int2_wsum", [(60, 16, INT2), (25, 32, INT2)], 0, True),
        ("mixed_sum", [(40, 16, INT8), (50, 32, INT4), (60, 64, INT2)], 0, False),
        ("fp32_sum", [(30, 8, FP32), (20, 12, FP32)], 0, False),
        ("fp16_mean", [(30, 8, FP16), (20, 16, FP16)], 1, False),
        ("fp16_wsum", [(30, 8, FP16), (20, 16, FP16)], 0, True),
        ("bf16_sum", [(30, 8, BF16), (20, 16, BF16)], 0, False),
    ]
    names = []
    for name, tables, mode, weighted in cases:
        case = make_case(rs, tables, B=7, mode=mode, weighted=weighted)
        for k, v in case.items():
            arrays[f"{name}/{k}"] = v
        names.append(name)
    arrays["case_names"] = np.array(names)
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    arrays["fp8_e4m3fn"] = codes.view(torch.float8_e4m3fn).float().numpy()
    arrays["fp8_e5m2"] = codes.view(torch.float8_e5m2).float().numpy()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}: {len(names)} bag cases + 2 fp8 tables")


if __name__ == "__main__":
    main()
