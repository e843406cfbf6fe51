"""Host-side checks that need no GPU: the C ABI library loads and exports what
include/tbe_nbit.h declares, the planner's layout rules and validation errors,
the op schema registration, and the module-level packer's layout."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6


def _header_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(tbe_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_abi_exports_every_declared_symbol(pkg):
    names = _header_functions()
    assert {"tbe_nbit_plan", "tbe_nbit_forward", "tbe_last_error", "tbe_nbit_abi_version"} <= set(names)
    lib = ctypes.CDLL(pkg.HIP_LIB)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
    assert set(names) == set(pkg.capi.EXPORTS)


def test_abi_version_and_struct_layout(pkg, tmp_path):
    """The ctypes mirror has the C compiler's sizes and field offsets for every struct."""
    import subprocess
    c = pkg.capi
    assert c.lib().tbe_nbit_abi_version() == c.ABI_VERSION == 3
    structs = [c.TbeTableDesc, c.TbePlanInput, c.TbePlanGroup, c.TbePlanSummary, c.TbeNbitArgs,
               c.TbePermutePooledArgs, c.TbeBlockBucketizeArgs]
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "tbe_nbit.h"', '#include "tbe_pooled_ops.h"',
             '#include "tbe_sparse_ops.h"', "int main(void){"]
    for st in structs:
        lines.append(f'printf("%zu\\n", sizeof({st.__name__}));')
        for f, _ in st._fields_:
            lines.append(f'printf("%zu\\n", offsetof({st.__name__}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", f"-I{ROOT}/include", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()]
    want = []
    for st in structs:
        want.append(ctypes.sizeof(st))
        want += [getattr(st, f).offset for f, _ in st._fields_]
    assert got == want


def test_forward_rejects_bad_args_without_gpu(pkg):
    c = pkg.capi
    a = c.TbeNbitArgs()
    a.T, a.B, a.index_size, a.max_col_tiles, a.output_dtype = 1, 1, 3, 1, 0
    with pytest.raises(c.TbeError, match="int32 or int64"):
        c.forward(a)
    a.index_size, a.pooling_mode = 4, 7
    with pytest.raises(c.TbeError, match="pooling mode"):
        c.forward(a)
    a.pooling_mode, a.output_dtype = 0, 2
    with pytest.raises(c.TbeError, match="INT8 output"):
        c.forward(a)
    a.output_dtype = 9
    with pytest.raises(c.TbeError, match="output_dtype"):
        c.forward(a)
    a.output_dtype, a.B = 0, 0
    c.forward(a)  # nothing to do: returns before touching the device


@pytest.mark.parametrize("ty,D,stride,lanes,tiles", [
    (INT8, 128, 144, 32, 1), (INT4, 128, 80, 16, 1), (INT2, 128, 48, 8, 1), (FP16, 128, 256, 64, 1),
    (FP32, 128, 512, 64, 2), (FP8, 128, 128, 32, 1), (BF16, 64, 128, 32, 1), (INT4, 32, 32, 4, 1),
    (FP8, 4096, 4096, 64, 16), (INT2, 16, 16, 1, 1), (FP8, 12, 16, 4, 1)])
def test_plan_layout(pkg, ty, D, stride, lanes, tiles):
    descs, order, s = pkg.capi.plan([0], [ty], [0, D], 1000 * stride, 16, 4, 7)
    d = descs[0]
    assert (d.row_stride, 1 << d.log2_lanes, d.col_tiles, d.D) == (stride, lanes, tiles, D)
    assert d.data_offset == (4 if ty in (INT8, INT4, INT2) else 0)
    assert d.num_rows == 1000
    assert s.max_col_tiles == tiles and s.total_D == D and s.covers_output == 1


def test_plan_num_rows_follow_table_extents(pkg):
    # tables laid out out of order; rows end where the next table starts
    descs, order, s = pkg.capi.plan([800, 0, 400], [INT4, INT8, INT4], [0, 128, 256, 384], 1600)
    assert [descs[i].num_rows for i in range(3)] == [10, 400 // 144, 5]
    assert s.uniform_D == 1 and s.max_D == 128


def test_plan_groups_tables_by_kernel_shape(pkg):
    """Tables are grouped by (weight type, lanes per row), keeping table order in a group."""
    tys = [INT4, INT8, INT4, FP16, INT4, INT8]
    Ds = [128, 128, 64, 128, 128, 128]
    dofs = np.concatenate([[0], np.cumsum(Ds)])
    woffs = np.arange(6) * 100000
    descs, order, s = pkg.capi.plan(woffs, tys, dofs, 600000)
    groups = [(g.weight_ty, g.log2_lanes, g.offset32, g.first, g.count) for g in s.groups[:s.num_groups]]
    assert sum(g[4] for g in groups) == 6 and len(groups) == 4
    members = {(g[0], g[1]): list(order[g[3]:g[3] + g[4]]) for g in groups}
    assert members[(INT4, 4)] == [0, 4] and members[(INT8, 5)] == [1, 5]
    assert members[(INT4, 3)] == [2] and members[(FP16, 6)] == [3]
    assert sorted(order.tolist()) == list(range(6))


def test_plan_groups_64bit_tables_by_shape(pkg):
    """Tables past 32-bit byte offsets keep per-shape groups (the per-bag kernel with
    64-bit addresses) while their rows fit a 32-bit index; only tables of 2^32 - 1
    rows or more share the generic group (weight_ty -1)."""
    big = 0xFFFE0000 + 80 * 16
    woffs = [0, big, 2 * big, 2 * big + 2 ** 34]
    tys, Ds = [INT4, INT4, INT8, FP32], [128, 128, 128, 1]
    dofs = np.concatenate([[0], np.cumsum(Ds)])
    descs, order, s = pkg.capi.plan(woffs, tys, dofs, woffs[3] + 2 ** 32 * 4, row_alignment=4)
    groups = sorted((g.weight_ty, g.offset32, sorted(order[g.first:g.first + g.count].tolist()))
                    for g in s.groups[:s.num_groups])
    assert groups == [(-1, 0, [3]), (INT8, 0, [2]), (INT4, 0, [0, 1])]


def test_plan_offset32_covers_tables_below_4gib(pkg):
    """32-bit table addressing (and with it the per-bag and row-stream kernels) holds
    up to 0xFFFE0000 bytes of rows; beyond that the 64-bit kernel takes the table."""
    limit = 0xFFFE0000
    for nbytes in (2 ** 31 + 4096, limit, limit + 80 * 2000):
        descs, order, s = pkg.capi.plan([0], [INT4], [0, 128], nbytes)
        rows = nbytes // 80
        o32 = bool(descs[0].flags & pkg.capi.TBE_TABLE_OFFSET32)
        assert descs[0].num_rows == rows
        assert o32 == (rows * 80 <= limit), nbytes
        assert s.groups[0].offset32 == int(o32)


@pytest.mark.parametrize("kw,match", [
    (dict(tys=[9]), "unsupported weight type"),
    (dict(tys=[INT4], dofs=[0, 12]), "4-byte words"),
    (dict(dofs=[0, -4]), "non-decreasing"),
    (dict(tys=[FP8], bits=-1, bias=-1), "fp8_exponent_bits"),
    (dict(woffs=[10 ** 9]), "outside dev_weights"),
    (dict(align=6), "row_alignment"),
])
def test_plan_rejects(pkg, kw, match):
    c = pkg.capi
    with pytest.raises(c.TbeError, match=match):
        c.plan(kw.get("woffs", [0]), kw.get("tys", [INT8]), kw.get("dofs", [0, 16]), 4096,
               kw.get("align", 16), kw.get("bits", 4), kw.get("bias", 7))


def test_plan_rejects_empty(pkg):
    with pytest.raises(pkg.capi.TbeError, match="greater than 0"):
        pkg.capi.plan(np.zeros(0, np.int64), np.zeros(0, np.uint8), [0], 16)


def test_schema_registered(pkg):
    schema = torch._C._dispatch_find_schema_or_throw(
        "fbgemm::int_nbit_split_embedding_codegen_lookup_function", "")
    assert schema is not None
    s = str(torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function.default._schema)
    for arg in ("Tensor dev_weights", "Tensor? indice_weights", "int output_dtype", "int? row_alignment",
                "int? max_float8_D", "int? fp8_exponent_bits", "int? fp8_exponent_bias"):
        assert arg in s


def test_cpu_tensors_have_no_fallback(pkg):
    from fbgemm_ascend_amd.workloads import make_workload
    wl = make_workload(0, device="cpu", scale_rows=0.01, batch=4)
    with pytest.raises(NotImplementedError):
        wl.run()


def test_module_layout_matches_oracle_rules(pkg, oracle):
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    specs = [("a", 10, 128, SparseType.INT4, 0), ("b", 7, 64, SparseType.INT8, 0),
             ("c", 5, 32, SparseType.FP16, 0), ("d", 3, 16, SparseType.INT2, 0),
             ("e", 4, 12, SparseType.FP8, 0)]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device="cpu")
    strides = [oracle.row_stride(int(ty), D) for _, _, D, ty, _ in specs]
    assert m.row_strides == strides
    assert m.weights_offsets.tolist() == list(np.cumsum([0] + [E * s for (_, E, *_), s in zip(specs, strides)])[:-1])
    assert m.D_offsets.tolist() == [0, 128, 192, 224, 240, 252]
    assert (m.max_int4_D, m.max_int8_D, m.max_float16_D, m.max_int2_D, m.max_float8_D) == (128, 64, 32, 16, 12)
    assert (m.fp8_exponent_bits, m.fp8_exponent_bias) == (4, 7)
    m.fill_random_weights(0)
    pay, sb = m.split_embedding_weights()[0]
    assert pay.shape == (10, 64) and sb.shape == (10, 4)
    sc = sb.contiguous().view(torch.float16)[:, 0].float()
    assert bool(((sc >= 0.00099) & (sc <= 0.0101)).all())


def test_module_quantize_roundtrip(pkg, oracle):
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    w = torch.randn(6, 32)
    for ty, bits in ((SparseType.INT8, 8), (SparseType.INT4, 4), (SparseType.INT2, 2)):
        m = IntNBitTableBatchedEmbeddingBagsCodegen([(6, 32, ty)], device="cpu")
        m.load_float_weights(0, w)
        out, _ = oracle.forward(m.weights_dev.numpy(), m.weights_offsets.numpy(), m.weights_tys.numpy(),
                                m.D_offsets.numpy(), np.arange(6, dtype=np.int32),
                                np.array([0, 6], np.int32), 2, None, 0)
        step = (w.max(1).values - w.min(1).values) / ((1 << bits) - 1)
        err = (torch.from_numpy(out) - w).abs().max(1).values
        assert bool((err <= step * 0.5 + 2e-3 * w.abs().max()).all()), ty


def test_workload_specs():
    import __graft_entry__ as g
    g.load_package()
    from fbgemm_ascend_amd.workloads import config_spec, make_workload
    s3 = config_spec(3)
    assert len(s3.tables) == 64 and s3.weighted and int(s3.pooling) == 1
    assert all(100_000 <= E <= 5_000_000 and D in (32, 64, 128, 256) for E, D, _ in s3.tables)
    wl = make_workload(1, device="cpu", scale_rows=0.001, batch=64)
    L = wl.lengths
    assert int(L.min()) >= 1 and int(L.max()) <= 100 and abs(float(L.float().mean()) - 30) < 2
    assert wl.offsets.dtype == torch.int32 and int(wl.offsets[-1]) == wl.num_indices
    wl3 = make_workload(3, device="cpu", scale_rows=0.001, batch=32)
    assert int(wl3.lengths.min()) == 0 and wl3.per_sample_weights is not None


FP8_PARAMS = [(4, 7), (5, 15), (3, 3), (4, 8), (2, 1), (6, 31), (1, 0), (7, 60)]


@pytest.mark.parametrize("eb,bias", FP8_PARAMS)
def test_fp8_quantize_exact_codes_and_midpoints(pkg, oracle, eb, bias):
    """Every code value quantises to itself (sign included); a point strictly between
    two neighbouring codes goes to the nearer one, an exact midpoint to the even code;
    magnitudes past the largest code saturate.  Code values come from the oracle's
    decoder (pinned exhaustively against the closed form in test_oracle.py)."""
    from fbgemm_ascend_amd import fp8_code_values, fp8_quantize
    table = oracle.fp8_table(eb, bias).astype(np.float64)  # 256 codes
    vals = fp8_code_values(eb, bias).double()
    np.testing.assert_array_equal(vals.numpy(), table[:128])
    codes = torch.arange(256)
    x = torch.from_numpy(table)
    got = fp8_quantize(x, eb, bias).to(torch.int64)
    # +0 / -0 keep their sign bit; every other code round-trips
    assert torch.equal(got, codes)
    lo, hi = vals[:-1], vals[1:]
    mid = (lo + hi) / 2
    q = fp8_quantize(mid, eb, bias).to(torch.int64)
    even = torch.where(torch.arange(1, 128) % 2 == 0, torch.arange(1, 128), torch.arange(0, 127))
    assert torch.equal(q, even)
    near_lo = lo + (hi - lo) * 0.25
    near_hi = lo + (hi - lo) * 0.75
    assert torch.equal(fp8_quantize(near_lo, eb, bias).to(torch.int64), torch.arange(0, 127))
    assert torch.equal(fp8_quantize(near_hi, eb, bias).to(torch.int64), torch.arange(1, 128))
    assert torch.equal(fp8_quantize(-near_hi, eb, bias).to(torch.int64), torch.arange(1, 128) | 0x80)
    big = torch.tensor([float(vals[127]) * 1.5, -float(vals[127]) * 4])
    assert fp8_quantize(big, eb, bias).tolist() == [0x7F, 0xFF]


@pytest.mark.parametrize("eb,bias,tdt,maxfin", [(4, 7, torch.float8_e4m3fn, 448.0), (5, 15, torch.float8_e5m2, 57344.0)])
def test_fp8_quantize_matches_torch_float8_casts(pkg, eb, bias, tdt, maxfin):
    """Inside the finite range of torch's float8 formats (same exponent width and bias,
    round to nearest even) the quantiser picks the same bit pattern as torch's cast."""
    from fbgemm_ascend_amd import fp8_quantize
    g = torch.Generator().manual_seed(eb)
    x = (torch.rand(200000, generator=g, dtype=torch.float64) * 2 - 1) * maxfin
    x = x * torch.exp2(-torch.randint(0, 20, x.shape, generator=g).double())
    x = x.float()
    want = x.to(tdt).view(torch.uint8)
    got = fp8_quantize(x, eb, bias)
    assert torch.equal(got, want)


@pytest.mark.parametrize("eb,bias", FP8_PARAMS[:4])
def test_module_fp8_quantize_roundtrip(pkg, oracle, eb, bias):
    """load_float_weights on an FP8 table: decoded rows (oracle nobag) are within half
    a code step of the float table."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType, fp8_code_values
    vals = fp8_code_values(eb, bias).double()
    w = (torch.rand(8, 64, dtype=torch.float64) * 2 - 1) * float(vals[127]) * 0.9
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(8, 64, SparseType.FP8)], device="cpu",
                                                fp8_exponent_bits=eb, fp8_exponent_bias=bias)
    m.load_float_weights(0, w.float())
    out, _ = oracle.forward(m.weights_dev.numpy(), m.weights_offsets.numpy(), m.weights_tys.numpy(),
                            m.D_offsets.numpy(), np.arange(8, dtype=np.int32), np.array([0, 8], np.int32),
                            2, None, 0, fp8_exponent_bits=eb, fp8_exponent_bias=bias)
    a = w.float().double().abs()
    k = torch.searchsorted(vals, a).clamp(1, 127)
    half_step = (vals[k] - vals[k - 1]) / 2
    assert bool(((torch.from_numpy(out).double() - w.float().double()).abs() <= half_step).all())


def test_gather_floor_row_addresses(pkg):
    """bench.row_addresses (the gather floor's input): every lookup's address is the
    table base + index * row stride of the lookup's table, including empty bags and
    tables of different strides."""
    import sys
    sys.path.insert(0, ROOT)
    import bench
    from fbgemm_ascend_amd.workloads import make_workload
    wl = make_workload(3, device="cpu", scale_rows=1e-4, batch=6, table_limit=7)
    m = wl.module
    for i in range(len(wl.batches)):
        bt = wl.batches[i]
        got = bench.row_addresses(wl, i).tolist()
        off = bt.offsets.tolist()
        B = wl.spec.B
        want = []
        for t in range(len(m.specs)):
            for j in range(off[t * B], off[(t + 1) * B]):
                want.append(m.weights_dev.data_ptr() + int(m.weights_offsets[t]) +
                            int(bt.indices[j]) * int(m.row_strides[t]))
        assert got == want


def test_plan_fuzz_accepts_or_rejects_cleanly(pkg):
    """Random table metadata, valid layouts with one field broken half of the time
    (unknown type, a width that does not fill 4-byte words, zero or decreasing
    D_offsets, an offset outside the buffer or unaligned, an odd row alignment, FP8
    parameters out of range): the planner either rejects with a message or returns a plan
    whose every table lies inside dev_weights and whose groups list each table exactly
    once.  (Run also under ASan and UBSan by test_sanitizers.py.)"""
    import random
    c = pkg.capi
    rnd = random.Random(1234)
    word_D = {FP32: 1, FP16: 2, BF16: 2, FP8: 4, INT8: 4, INT4: 8, INT2: 16}
    accepted = rejected = a64_groups = generic_groups = 0
    for _ in range(600):
        T = rnd.choice([1, 2, 3, 7, 26, 64])
        tys = [rnd.choice([FP32, FP16, INT8, INT4, INT2, BF16, FP8]) for _ in range(T)]
        Ds = [word_D[ty] * rnd.choice([1, 2, 3, 8, 16, 32, 64, 65, 128, 300]) for ty in tys]
        align = rnd.choice([4, 8, 16, 16, 32, 64])
        # mostly small tables, some past 4 GiB of rows, some of 2^32 rows or more
        # (the planner only does arithmetic on the sizes: nothing is allocated)
        rows = [rnd.choice([1, 2, 10, 1000, 1000, 1000, 60_000_000, 2 ** 32 + 5]) for _ in range(T)]
        woffs, pos = [], 0
        for ty, D, E in zip(tys, Ds, rows):
            woffs.append(pos)
            pos += E * _stride(ty, D, align)
        nbytes = pos + rnd.choice([0, 0, 4, 1000])
        bits, bias = rnd.choice([(4, 7), (5, 15), (1, 0), (7, 120)])
        dofs = [0] + np.cumsum(Ds).tolist()
        if rnd.random() < 0.5:  # break one thing
            k = rnd.randrange(T)
            what = rnd.randrange(9)
            if what == 0:
                tys[k] = rnd.choice([7, 9, 255])
            elif what == 1:
                dofs[k + 1] = dofs[k] + rnd.choice([1, 3, 5])  # a width that does not fill words (or 0-width)
                dofs[k + 2:] = [d - Ds[k] + dofs[k + 1] - dofs[k] for d in dofs[k + 2:]]
            elif what == 2:
                dofs[k + 1] = dofs[k]  # zero-width table
            elif what == 3:
                dofs[k + 1] = dofs[k] - 4  # decreasing
            elif what == 4:
                woffs[k] = rnd.choice([-16, nbytes + 16, 2 ** 62])
            elif what == 5:
                woffs[k] += 2  # unaligned
            elif what == 6:
                align = rnd.choice([0, -16, 6, 1, 1 << 20])
            elif what == 7:
                bits, bias = rnd.choice([(-1, -1), (0, 0), (8, 1), (3, -200), (7, 1000)])
            else:
                nbytes = rnd.choice([0, 16])
        try:
            descs, order, s = c.plan(woffs, tys, dofs, nbytes, align, bits, bias)
        except c.TbeError as e:
            assert str(e).strip(), "rejection without a message"
            rejected += 1
            continue
        accepted += 1
        seen = []
        for gi in range(s.num_groups):
            g = s.groups[gi]
            members = list(order[g.first:g.first + g.count])
            seen += members
            a64_groups += int(g.weight_ty >= 0 and not g.offset32)
            generic_groups += int(g.weight_ty < 0)
            # a group is one kernel shape: its tables share type, lanes per row and
            # addressing form (only the generic group, weight_ty -1, mixes them)
            for t in members:
                d = descs[t]
                assert bool(d.flags & c.TBE_TABLE_OFFSET32) == bool(g.offset32)
                if g.weight_ty >= 0:
                    assert (d.weight_ty, d.log2_lanes) == (g.weight_ty, g.log2_lanes)
                    assert bool(d.flags & c.TBE_TABLE_STREAM) == bool(g.stream)
                else:
                    assert d.num_rows >= 2 ** 32 - 1 and not g.offset32
        assert sorted(seen) == list(range(T))
        for t in range(T):
            d = descs[t]
            assert d.row_stride > 0 and d.num_rows >= 0
            assert 0 <= d.weights_offset and d.weights_offset + d.num_rows * d.row_stride <= nbytes
    assert accepted > 100 and rejected > 100, (accepted, rejected)
    assert a64_groups > 20 and generic_groups > 20, (a64_groups, generic_groups)


def _stride(ty, D, align):
    bits = {FP32: 32, FP16: 16, BF16: 16, FP8: 8, INT8: 8, INT4: 4, INT2: 2}[ty]
    u = D * bits // 8 + (4 if ty in (INT8, INT4, INT2) else 0)
    return (u + align - 1) // align * align


def test_module_copies_drop_the_bound_call(pkg):
    """deepcopy / pickle of the module work (the bound C++ call is not copied) and the
    copy still refuses CPU tensors like the op."""
    import copy
    import pickle
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(10, 16, SparseType.INT8)], device="cpu")
    idx, off = torch.tensor([1, 2], dtype=torch.int32), torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        m(idx, off)
    for c in (copy.deepcopy(m), pickle.loads(pickle.dumps(m))):
        assert c.__dict__.get("_bound") is None
        assert torch.equal(c.weights_offsets, m.weights_offsets)
        with pytest.raises(NotImplementedError):
            c(idx, off)


def test_parity_fp16_overflow_rule():
    """The fp16 comparison accepts +-inf exactly where the RNE cast of the fp32 sum
    overflows, and nowhere else."""
    import numpy as np
    from _parity import assert_bag_parity
    prob = {"weights_tys": np.array([1], np.uint8), "B": 1, "D_offsets": np.array([0, 4]),
            "indices": np.array([0]), "offsets": np.array([0, 1]), "psw": None,
            "rowmax": [np.array([1.0])]}
    ref = np.array([[70000.0, -80000.0, 65510.0, 100.0]], np.float32)
    ok = torch.tensor([[float("inf"), float("-inf"), 65504.0, 100.0]], dtype=torch.float16)
    assert_bag_parity(ok, prob, ref, 0, 1)
    for bad in ([65504.0, float("-inf"), 65504.0, 100.0], [float("-inf"), float("-inf"), 65504.0, 100.0],
                [float("inf"), float("-inf"), 65504.0, float("inf")]):
        with pytest.raises(AssertionError):
            assert_bag_parity(torch.tensor([bad], dtype=torch.float16), prob, ref, 0, 1)
