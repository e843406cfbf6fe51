"""Pins of the CPU oracle (CPU only).

Each check compares the oracle against something it was not derived from: a
library routine (torch float8 dtypes, torch's fp16/bf16 casts, FBGEMM's quantized
embedding_bag kernels, F.embedding_bag), the committed golden vectors made by
those routines, the closed form of a number format, or brute force over tiny
integer-exact inputs.
"""
import math

import numpy as np
import pytest
import torch

FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6


# ----------------------------------------------------------------- FP8 decode (C:120-167)

def _fp8_closed_form(code: int, e: int, bias: int) -> float:
    """(-1)^s * 2^(E-bias) * (1 + M/2^m), subnormal 2^(1-bias) * M/2^m when E == 0."""
    m = 7 - e
    s = -1.0 if code & 0x80 else 1.0
    E = (code & 0x7F) >> m
    M = code & ((1 << m) - 1)
    if E == 0:
        return s * math.ldexp(M / (1 << m), 1 - bias)
    return s * math.ldexp(1.0 + M / (1 << m), E - bias)


@pytest.mark.parametrize("e,bias", [(4, 7), (5, 15), (4, 8), (3, 3), (2, 1), (5, 16), (6, 31), (1, 0), (7, 63)])
def test_fp8_exhaustive_closed_form(oracle, e, bias):
    got = oracle.fp8_table(e, bias)
    for c in range(256):
        want = _fp8_closed_form(c, e, bias)
        assert got[c] == np.float32(want), (c, got[c], want)
        assert math.copysign(1.0, float(got[c])) == math.copysign(1.0, want)  # -0 kept


def test_fp8_e4m3_matches_torch(oracle, golden):
    got = oracle.fp8_table(4, 7)
    lib = golden["fp8_e4m3fn"]
    live = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(lib, live)  # fixture still matches the library
    ok = ~np.isnan(lib)  # e4m3fn spends 0x7F/0xFF on NaN; the TBE decode gives +-480 there
    np.testing.assert_array_equal(got[ok], lib[ok])
    assert got[0x7F] == 480.0 and got[0xFF] == -480.0


def test_fp8_e5m2_matches_torch(oracle, golden):
    got = oracle.fp8_table(5, 15)
    lib = golden["fp8_e5m2"]
    finite = np.isfinite(lib)  # E=31 codes are inf/nan in e5m2, plain numbers in the TBE decode
    np.testing.assert_array_equal(got[finite], lib[finite])


# ----------------------------------------------------------------- fp16 / bf16 casts

def test_half_decode_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.half_to_float(bits)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.float16).float().numpy()
    both_nan = np.isnan(got) & np.isnan(want)
    np.testing.assert_array_equal(got[~both_nan], want[~both_nan])
    assert both_nan.sum() == np.isnan(want).sum()


def _cast_inputs():
    rs = np.random.RandomState(1)
    x = np.concatenate([
        rs.standard_normal(200000).astype(np.float32) * 10,
        rs.uniform(-7e4, 7e4, 20000).astype(np.float32),
        (rs.uniform(-1, 1, 20000) * 1e-5).astype(np.float32),      # fp16 subnormal range
        (rs.uniform(-1, 1, 20000) * 1e-8).astype(np.float32),      # underflow
        # exact fp16 ties: midpoints between neighbouring halves
        ((np.arange(0, 65504, 7, dtype=np.float32) + 0.5)),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, -65520, 1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14], dtype=np.float32),
    ])
    # random bit patterns cover every exponent (NaNs excluded: payload conventions differ)
    r = rs.randint(0, 2 ** 32, size=200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate([x, r[~np.isnan(r)]])


def test_half_encode_matches_torch(oracle):
    x = _cast_inputs()
    got = oracle.float_to_half_bits(x)
    want = torch.from_numpy(x).half().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)


def test_bf16_encode_matches_torch(oracle):
    x = _cast_inputs()
    got = oracle.float_to_bf16_bits(x)
    want = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)


# ----------------------------------------------------------------- INT row decode, exhaustive codes

@pytest.mark.parametrize("ty,bits", [(INT8, 8), (INT4, 4), (INT2, 2)])
def test_int_codes_exhaustive(oracle, ty, bits):
    """Nobag output of a table whose rows enumerate every code equals scale*q + bias
    (the float64 value is exact, so rounding it to fp32 is the fused multiply-add)."""
    ncode = 1 << bits
    D = max(ncode, 16)
    rs = np.random.RandomState(bits)
    scales = np.array([1.0, 0.5, 0.0078125, 0.001, 0.01, 3.5], dtype=np.float16)
    biases = np.array([0.0, -1.0, 0.5, -0.999, 0.3333, 7.0], dtype=np.float16)
    E = len(scales)
    per = 8 // bits
    stride = (4 + D // per + 15) // 16 * 16
    w = np.zeros((E, stride), dtype=np.uint8)
    q = np.tile(np.arange(D) % ncode, (E, 1))
    q = np.array([rs.permutation(row) for row in q])
    for r in range(E):
        w[r, 0:2] = scales[r:r + 1].view(np.uint8)
        w[r, 2:4] = biases[r:r + 1].view(np.uint8)
        for j in range(D // per):
            byte = 0
            for k in range(per):
                byte |= int(q[r, j * per + k]) << (bits * k)
            w[r, 4 + j] = byte
    indices = np.arange(E, dtype=np.int32)
    out, out32 = oracle.forward(w.reshape(-1), [0], [ty], [0, D], indices, np.array([0, E], np.int32),
                                pooling_mode=2, output_dtype=FP32)
    want = (scales.astype(np.float64)[:, None] * q + biases.astype(np.float64)[:, None]).astype(np.float32)
    np.testing.assert_array_equal(out, want)


# ----------------------------------------------------------------- golden library vectors

def _run_case(oracle, golden, name, out_ty=FP32):
    g = {k: golden[f"{name}/{k}"] for k in ("weights", "weights_offsets", "weights_tys", "D_offsets",
                                             "indices", "offsets", "psw", "pooling_mode", "expected")}
    psw = g["psw"] if g["psw"].size else None
    out, out32 = oracle.forward(g["weights"], g["weights_offsets"], g["weights_tys"], g["D_offsets"],
                                g["indices"], g["offsets"], int(g["pooling_mode"]), psw, out_ty)
    return out, out32, g


def test_golden_library_vectors(oracle, golden):
    names = [str(n) for n in golden["case_names"]]
    assert len(names) >= 10
    for name in names:
        out, out32, g = _run_case(oracle, golden, name)
        exp = g["expected"]
        # FBGEMM/ATen accumulate in a different order (and may fuse differently): fp32 rounding only
        np.testing.assert_allclose(out32, exp, rtol=1e-5, atol=1e-5, err_msg=name)


def test_golden_int32_indices_same_result(oracle, golden):
    for name in ("int4_sum", "int2_mean", "fp16_wsum"):
        _, a, g = _run_case(oracle, golden, name)
        psw = g["psw"] if g["psw"].size else None
        _, b = oracle.forward(g["weights"], g["weights_offsets"], g["weights_tys"], g["D_offsets"],
                              g["indices"].astype(np.int32), g["offsets"].astype(np.int32),
                              int(g["pooling_mode"]), psw, FP32)
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("out_ty,tdt", [(FP16, torch.float16), (BF16, torch.bfloat16)])
def test_golden_output_cast(oracle, golden, out_ty, tdt):
    out, out32, g = _run_case(oracle, golden, "mixed_sum", out_ty)
    want = torch.from_numpy(out32).to(tdt).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(out, want)


# ----------------------------------------------------------------- integer-exact known answers

def _kat_problem(rs, tables, B, idx_dtype, Lmax=70):
    """Tables whose dequantized values are small integers, so every pooled sum is exact in fp32."""
    blocks, woffs, dofs, pos = [], [], [0], 0
    vals = []
    for t, (E, D, ty) in enumerate(tables):
        bits = {INT8: 8, INT4: 4, INT2: 2, FP16: 16, FP32: 32, BF16: 16, FP8: 8}[ty]
        hdr = 4 if ty in (INT8, INT4, INT2) else 0
        st = (hdr + D * bits // 8 + 15) // 16 * 16
        buf = np.zeros((E, st), dtype=np.uint8)
        if ty in (INT8, INT4, INT2):
            q = (np.arange(E)[:, None] * 7 + np.arange(D)[None, :] * 3 + t) % (1 << bits)
            per = 8 // bits
            packed = np.zeros((E, D // per), dtype=np.uint8)
            for k in range(per):
                packed |= (q[:, k::per] << (bits * k)).astype(np.uint8)
            buf[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
            buf[:, 2:4] = np.array([-(t % 3)], np.float16).view(np.uint8)
            buf[:, 4:4 + packed.shape[1]] = packed
            v = q.astype(np.float64) - (t % 3)
        elif ty == FP8:
            # codes whose (4,7) value is an integer 1..15: E field 7..10 with zero mantissa low bits
            ints = np.array([0x38, 0x40, 0x44, 0x48, 0x4A, 0x4C, 0x4E, 0x50, 0x51, 0x52, 0x53, 0x54,
                             0x55, 0x56, 0x57], dtype=np.uint8)  # 1,2,3,4,5,6,7,8,9,...,15
            sel = (np.arange(E)[:, None] + np.arange(D)[None, :] + t) % len(ints)
            buf[:, :D] = ints[sel]
            v = (sel + 1).astype(np.float64)
        else:
            v = ((np.arange(E)[:, None] * 5 + np.arange(D)[None, :] + t) % 17 - 8).astype(np.float64)
            if ty == FP16:
                buf[:, :2 * D] = v.astype(np.float16).view(np.uint8).reshape(E, -1)
            elif ty == BF16:
                buf[:, :2 * D] = (v.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(E, -1)
            else:
                buf[:, :4 * D] = v.astype(np.float32).view(np.uint8).reshape(E, -1)
        blocks.append(buf.reshape(-1))
        woffs.append(pos)
        pos += buf.size
        dofs.append(dofs[-1] + D)
        vals.append(v)
    lengths = rs.randint(0, Lmax, size=len(tables) * B)
    offsets = np.zeros(len(lengths) + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(lengths)
    indices = np.concatenate([rs.randint(0, E, size=int(lengths[t * B:(t + 1) * B].sum()))
                              for t, (E, _, _) in enumerate(tables)]).astype(idx_dtype)
    return (np.concatenate(blocks), np.array(woffs, np.int64), np.array([ty for *_, ty in tables], np.uint8),
            np.array(dofs, np.int32), indices, offsets.astype(idx_dtype), vals, lengths)


def kat_expected(vals, dofs, indices, offsets, B, lengths, pooling_mode, weights=None):
    """Brute force: gather each bag's rows and sum them (float64, exact for these inputs)."""
    T = len(vals)
    out = np.zeros((B, int(dofs[-1])), dtype=np.float64)
    for t in range(T):
        for b in range(B):
            k = t * B + b
            sl = slice(int(offsets[k]), int(offsets[k + 1]))
            rows = vals[t][indices[sl].astype(np.int64)]
            if weights is not None:
                rows = rows * weights[sl, None]
            s = rows.sum(axis=0)
            if pooling_mode == 1 and lengths[k] > 0:
                s = s * np.float64(np.float32(1.0) / np.float32(lengths[k]))
            out[b, dofs[t]:dofs[t + 1]] = s
    return out


@pytest.mark.parametrize("idx_dtype", [np.int32, np.int64])
def test_kat_bit_exact_indexing(oracle, idx_dtype):
    rs = np.random.RandomState(7)
    tables = [(37, 16, INT8), (53, 32, INT4), (29, 64, INT2), (41, 8, FP16), (23, 12, FP32),
              (31, 20, FP8), (19, 6, BF16)]
    B = 11
    w, wo, wt, do, idx, off, vals, lengths = _kat_problem(rs, tables, B, idx_dtype)
    out, _ = oracle.forward(w, wo, wt, do, idx, off, 0, None, FP32, fp8_exponent_bits=4,
                            fp8_exponent_bias=7)
    exp = kat_expected(vals, do, idx, off, B, lengths, 0)
    np.testing.assert_array_equal(out, exp.astype(np.float32))
    # nobag: row i of the output is the row of indices[i] (tables of one D only)
    tables_nb = [(37, 32, INT8), (53, 32, INT4), (29, 32, FP16)]
    w, wo, wt, do, idx, off, vals, lengths = _kat_problem(rs, tables_nb, 5, idx_dtype)
    out, _ = oracle.forward(w, wo, wt, do, idx, off, 2, None, FP32)
    T = len(tables_nb)
    want = np.concatenate([vals[t][idx[int(off[t * 5]):int(off[(t + 1) * 5])].astype(np.int64)]
                           for t in range(T)])
    np.testing.assert_array_equal(out, want.astype(np.float32))


def test_out_of_range_rows_are_skipped(oracle):
    rs = np.random.RandomState(3)
    tables = [(20, 16, INT8), (30, 16, INT4)]
    w, wo, wt, do, idx, off, vals, lengths = _kat_problem(rs, tables, 4, np.int64, Lmax=10)
    bad = idx.copy()
    bad[::3] = -1
    bad[1::7] = 10 ** 6
    out, _ = oracle.forward(w, wo, wt, do, bad, off, 0, None, FP32)
    keep = (bad >= 0) & (bad < 10 ** 5)
    keep_t = np.zeros_like(keep)
    for t, (E, _, _) in enumerate(tables):
        lo, hi = off[t * 4], off[(t + 1) * 4]
        keep_t[lo:hi] = (bad[lo:hi] >= 0) & (bad[lo:hi] < E)
    wts = keep_t.astype(np.float64)
    exp = kat_expected(vals, do, np.where(keep_t, bad, 0), off, 4, lengths, 0, weights=wts)
    np.testing.assert_array_equal(out, exp.astype(np.float32))


def test_mean_uses_reciprocal_of_length(oracle):
    """MEAN multiplies the fp32 sum by float(1)/float(L) (P:355), not a division by L."""
    rs = np.random.RandomState(11)
    tables = [(40, 16, FP32)]
    w, wo, wt, do, idx, off, vals, lengths = _kat_problem(rs, tables, 50, np.int32, Lmax=40)
    out, _ = oracle.forward(w, wo, wt, do, idx, off, 1, None, FP32)
    sums = kat_expected(vals, do, idx, off, 50, lengths, 0).astype(np.float32)
    inv = np.array([np.float32(1) / np.float32(L) if L else np.float32(1) for L in lengths], np.float32)
    np.testing.assert_array_equal(out, sums * inv[:, None])
