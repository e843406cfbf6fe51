"""GPU parity of the paths the random matrices do not reach:

* tables whose rows span more than 4 GiB (the 64-bit-address forms of the per-bag
  and nobag kernels), a table of more than 2^32 rows and calls with more than 2^31
  indices (the generic kernels);
* FP8 rows under exponent-bit / bias pairs other than (4, 7), so both FP8 decodes
  run (fp16 placement for exponent_bits <= 4, shift-and-multiply above);
* the plan cache under freed and reallocated table metadata;
* nobag output rows outside every table's segment;
* the module packer: float tables -> load_float_weights -> the HIP op, against the
  dequantised table (oracle) and against the float table within the quantisation
  bound.

Reference: c310/op_kernel/common.h:120-167 (FP8), int_nbit_split_embedding_pooling_kernel.h:235-278
(row addressing), test_int_nbit_split_embedding_codegen_lookup_function.py:121-156 (packer use).
"""
import sys

import numpy as np
import pytest
import torch

from _parity import assert_bag_parity, compact_problem, run_oracle
from test_gpu_parity import OUT_TORCH, _check_module, _random_case

pytestmark = pytest.mark.gpu

FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _free_gib():
    free, _ = torch.cuda.mem_get_info()
    return free / 2 ** 30


# ----------------------------------------------------------------- tables beyond 32-bit addressing

BIG_ROWS = 60_000_000  # INT4 D=128: 80-byte rows, 4.8 GB, past the 0xFFFE0000-byte limit


@pytest.fixture(scope="module")
def big_tables(gpu):
    """One 4.8 GB INT4 table next to a small INT8 table (same D, so nobag applies)."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    if _free_gib() < 16:
        pytest.skip("needs ~6 GiB of free HBM")
    specs = [(BIG_ROWS, 128, SparseType.INT4), (1000, 128, SparseType.INT8)]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu)
    m.fill_random_weights(60)
    yield m
    del m
    torch.cuda.empty_cache()


def _big_inputs(gpu, idx_dtype, B=96, L=40, seed=5):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    lens = torch.randint(0, 2 * L, (2 * B,), device=gpu, generator=g)
    lens[::11] = 0
    off = torch.zeros(2 * B + 1, dtype=torch.int64, device=gpu)
    torch.cumsum(lens, 0, out=off[1:])
    n0, N = int(off[B]), int(off[-1])
    big = torch.randint(BIG_ROWS - 50000, BIG_ROWS + 2, (n0,), device=gpu, generator=g)  # last rows + 2 past the end
    big[::5] = torch.randint(0, BIG_ROWS, (big[::5].numel(),), device=gpu, generator=g)
    small = torch.randint(0, 1000, (N - n0,), device=gpu, generator=g)
    idx = torch.cat([big, small]).to(idx_dtype)
    psw = torch.rand(N, device=gpu, generator=g)
    return idx, off.to(idx_dtype), psw


def test_big_table_plan_is_64bit(pkg, big_tables):
    m = big_tables
    plan = pkg.capi.plan(m.weights_offsets.cpu().numpy(), m.weights_tys.cpu().numpy(), m.D_offsets.cpu().numpy(),
                         m.weights_dev.numel())
    descs = plan[0]
    assert not (descs[0].flags & pkg.capi.TBE_TABLE_OFFSET32)
    assert descs[1].flags & pkg.capi.TBE_TABLE_OFFSET32
    s = plan[2]
    groups = {(g.weight_ty, g.offset32) for g in s.groups[:s.num_groups]}
    assert groups == {(INT4, 0), (INT8, 1)}  # the big table keeps its own (A64) group


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("pm,weighted,out_ty", [(0, False, FP16), (1, True, FP32), (0, True, BF16)])
def test_big_table_pooled(pkg, oracle, gpu, big_tables, idx_dtype, pm, weighted, out_ty):
    """The per-bag kernel with 64-bit row addresses on a 4.8 GB table (its last rows,
    two indices past the end, which read the zero row)."""
    m = big_tables
    m.pooling_mode = pkg.PoolingMode(pm)
    m.output_dtype = out_ty
    idx, off, psw = _big_inputs(gpu, idx_dtype)
    _check_module(oracle, m, idx, off, psw if weighted else None,
                  f"4.8 GB table pm={pm} w={weighted} {idx_dtype} out={out_ty}")


@pytest.mark.parametrize("out_ty", [FP16, FP32])
def test_big_table_nobag(pkg, oracle, gpu, big_tables, out_ty):
    """The nobag kernel with 64-bit row addresses (big table) next to the 32-bit one
    (small table)."""
    m = big_tables
    m.pooling_mode = pkg.PoolingMode(2)
    m.output_dtype = out_ty
    idx, off, _ = _big_inputs(gpu, torch.int32)
    _check_module(oracle, m, idx, off, None, f"4.8 GB table nobag out={out_ty}")


@pytest.mark.parametrize("ty,D", [(FP32, 64), (FP16, 256), (BF16, 128), (FP8, 128), (INT8, 256), (INT2, 64)])
def test_every_row_type_past_4gib(pkg, oracle, gpu, ty, D):
    """One table of each row type just past 32-bit byte offsets (64-bit row addresses;
    FP16 D=256 spans two column tiles): SUM, weighted MEAN and NONE, int32 indices at
    the end of the table and past it."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    from fbgemm_ascend_amd.sparse_types import row_stride
    if _free_gib() < 16:
        pytest.skip("needs ~6 GiB of free HBM")
    st = row_stride(SparseType(ty), D, 16)
    E = 0xFFFE0000 // st + 4096
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(E, D, SparseType(ty))], device=gpu)
    try:
        m.fill_random_weights(ty + 1)
        plan = pkg.capi.plan(m.weights_offsets.cpu().numpy(), m.weights_tys.cpu().numpy(),
                             m.D_offsets.cpu().numpy(), m.weights_dev.numel(), 16, m.fp8_exponent_bits,
                             m.fp8_exponent_bias)
        assert not (plan[0][0].flags & pkg.capi.TBE_TABLE_OFFSET32)
        g = torch.Generator(device=gpu)
        g.manual_seed(400 + ty)
        B = 48
        lens = torch.randint(0, 70, (B,), device=gpu, generator=g)
        off = torch.zeros(B + 1, dtype=torch.int64, device=gpu)
        torch.cumsum(lens, 0, out=off[1:])
        N = int(off[-1])
        idx = torch.randint(E - 8192, E + 2, (N,), device=gpu, generator=g)  # the rows past 4 GiB, 2 past the end
        idx[::3] = torch.randint(0, E, (idx[::3].numel(),), device=gpu, generator=g)
        idx, off = idx.to(torch.int32), off.to(torch.int32)
        psw = torch.rand(N, device=gpu, generator=g)
        for pm, w, out_ty in ((0, False, FP16), (1, True, FP32), (2, False, BF16)):
            m.pooling_mode = pkg.PoolingMode(pm)
            m.output_dtype = out_ty
            _check_module(oracle, m, idx, off, psw if w else None, f"type {ty} D={D} past 4 GiB pm={pm}")
    finally:
        del m
        torch.cuda.empty_cache()


@pytest.mark.parametrize("pm,weighted", [(0, False), (1, True), (2, False)])
def test_table_past_2pow32_rows(pkg, oracle, gpu, pm, weighted):
    """A table of 2^32 + 8 rows (FP32 D=1 at row_alignment 4: 16 GiB), past 32-bit
    row indices: the generic pooled and nobag kernels, next to a small table that
    keeps its specialised kernel; int64 indices at both ends of the big table and
    past it."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    if _free_gib() < 48:
        pytest.skip("needs ~40 GiB of free HBM")
    E = 2 ** 32 + 8
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(E, 1, SparseType.FP32), (1000, 1, SparseType.FP32)], device=gpu,
                                                pooling_mode=pm, output_dtype=FP32, indices_dtype=torch.int64,
                                                row_alignment=4)
    try:
        w = m.weights_dev
        g = torch.Generator(device=gpu)
        g.manual_seed(32 + pm)
        rows_f = w.view(torch.float32)  # one float per row
        for lo in range(0, rows_f.numel(), 1 << 30):  # U(-1, 1) in slices
            n = min(1 << 30, rows_f.numel() - lo)
            rows_f[lo:lo + n] = torch.rand(n, device=gpu, generator=g) * 2 - 1
        plan = pkg.capi.plan(m.weights_offsets.cpu().numpy(), m.weights_tys.cpu().numpy(),
                             m.D_offsets.cpu().numpy(), w.numel(), row_alignment=4)
        s = plan[2]
        assert sorted(gr.weight_ty for gr in s.groups[:s.num_groups]) == [-1, FP32]
        B = 64
        lens = torch.randint(0, 30, (2 * B,), device=gpu, generator=g)
        off = torch.zeros(2 * B + 1, dtype=torch.int64, device=gpu)
        torch.cumsum(lens, 0, out=off[1:])
        n0, N = int(off[B]), int(off[-1])
        big = torch.randint(E - 3000, E + 2, (n0,), device=gpu, generator=g)  # its last rows, 2 past the end
        big[::4] = torch.randint(0, 3000, (big[::4].numel(),), device=gpu, generator=g)
        big[1::4] = torch.randint(0, E, (big[1::4].numel(),), device=gpu, generator=g)
        idx = torch.cat([big, torch.randint(0, 1000, (N - n0,), device=gpu, generator=g)])
        psw = torch.rand(N, device=gpu, generator=g) if weighted else None
        _check_module(oracle, m, idx, off, psw, f"2^32+8 rows pm={pm} w={weighted}")
    finally:
        del m
        torch.cuda.empty_cache()


def test_more_than_2pow31_indices(pkg, gpu):
    """A call with 2^31 + 4096 indices (positions past 32 bits take the generic
    kernel).  Exact known answer: an FP32 D=4 table whose element c of row r is
    bit c of r, so every bag sum is an integer count below 2^24 (exact in fp32 in
    any order); counts are taken with torch.bincount per bag."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    if _free_gib() < 40:
        pytest.skip("needs ~30 GiB of free HBM")
    E, D, B = 1000, 4, 2048
    N = (1 << 31) + 4096
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(E, D, SparseType.FP32)], device=gpu, output_dtype=FP32)
    r = torch.arange(E, device=gpu)
    table = torch.stack([((r >> c) & 1).float() for c in range(D)], 1)
    m.load_float_weights(0, table)
    g = torch.Generator(device=gpu)
    g.manual_seed(31)
    idx = torch.randint(0, E, (N,), device=gpu, generator=g, dtype=torch.int32)
    cuts = torch.sort(torch.randint(0, N + 1, (B - 1,), device=gpu, generator=g)).values
    off = torch.cat([torch.zeros(1, dtype=torch.int64, device=gpu), cuts,
                     torch.full((1,), N, dtype=torch.int64, device=gpu)]).to(torch.int32)
    _say(f"[gpu] 2^31+ indices: N={N} B={B}")
    for pm in (0, 1):
        m.pooling_mode = pkg.PoolingMode(pm)
        out = m(idx, off, None)
        torch.cuda.synchronize()
        offs = off.to(torch.int64).cpu().tolist()
        want = torch.zeros(B, D, dtype=torch.float64)
        for b in range(B):
            cnt = torch.bincount(idx[offs[b]:offs[b + 1]].to(torch.int64), minlength=E).double().cpu()
            want[b] = cnt @ table.double().cpu()
        if pm == 1:
            L = torch.tensor([offs[b + 1] - offs[b] for b in range(B)], dtype=torch.float32)
            want = (want.float() * (1.0 / torch.clamp(L, min=1.0))[:, None]).double()  # float(1)/float(L), P:355
        assert torch.equal(out.cpu().double(), want), f"pm={pm}"
    del idx, off, m
    torch.cuda.empty_cache()


# ----------------------------------------------------------------- FP8 exponent widths and biases

FP8_PARAMS = [(5, 15), (3, 3), (4, 8), (2, 1), (6, 31), (1, 0), (7, 60)]


def _fp8_case(pkg, gpu, seed, T, eb, bias, pm, weighted, idx_dtype, out_ty):
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    rs = np.random.RandomState(seed)
    D = 4 * int(rs.randint(1, 300))
    tables = [(int(rs.randint(1, 5000)), D if pm == 2 else 4 * int(rs.randint(1, 300))) for _ in range(T)]
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(E, d, SparseType.FP8) for E, d in tables], device=gpu,
                                                pooling_mode=pm, output_dtype=out_ty, indices_dtype=idx_dtype,
                                                fp8_exponent_bits=eb, fp8_exponent_bias=bias)
    m.fill_random_weights(seed)
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    B = 37
    lens = torch.randint(0, 90, (T * B,), device=gpu, generator=g)
    off = torch.zeros(T * B + 1, dtype=torch.int64, device=gpu)
    torch.cumsum(lens, 0, out=off[1:])
    offs = off.cpu()
    idx = torch.cat([torch.randint(0, E, (int(offs[(t + 1) * B] - offs[t * B]),), device=gpu, generator=g)
                     for t, (E, _) in enumerate(tables)]).to(idx_dtype)
    psw = torch.rand(idx.numel(), device=gpu, generator=g) if weighted else None
    return m, idx, off.to(idx_dtype), psw


def _fp8_params():
    out = []
    for eb, bias in FP8_PARAMS:
        # fp16 out with wide exponents: sums past 65504 become +-inf, as the RNE cast gives
        outs = (FP32, FP16, BF16)
        for pm, weighted in ((0, False), (1, True), (2, False)):
            for idx_dtype in (torch.int32, torch.int64):
                for out_ty in outs:
                    if pm == 2 and idx_dtype != torch.int32:
                        continue
                    out.append((eb, bias, pm, weighted, idx_dtype, out_ty))
    return out


# (nobag has one kernel per group: no forced row-stream run of pooling NONE)
_FP8_CASES = [(k,) + c for k in ("default", "stream") for c in _fp8_params() if not (k == "stream" and c[2] == 2)]


@pytest.mark.parametrize("T", [1, 3])
@pytest.mark.parametrize("kernel,eb,bias,pm,weighted,idx_dtype,out_ty", _FP8_CASES)
def test_fp8_exponent_params(pkg, oracle, gpu, T, eb, bias, pm, weighted, idx_dtype, out_ty, kernel):
    seed = (eb * 131 + bias * 7 + pm * 3 + T) & 0xFFFF
    m, idx, off, psw = _fp8_case(pkg, gpu, seed, T, eb, bias, pm, weighted, idx_dtype, out_ty)
    flags = pkg.capi.TBE_FLAG_FORCE_STREAM if kernel == "stream" else None
    _check_module(oracle, m, idx, off, psw, f"fp8 ({eb},{bias}) T={T} pm={pm} w={weighted} {idx_dtype} out={out_ty}",
                  flags=flags)


# ----------------------------------------------------------------- plan cache

def test_plan_cache_survives_reallocated_metadata(pkg, oracle, gpu):
    """Modules built and freed in turn, with the same table count and weight bytes but
    a different table order (so different types, D and offsets): each call must use
    its own module's layout even when the allocator hands out the freed addresses."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    a = [(1000, 128, SparseType.INT4), (2000, 64, SparseType.INT8)]  # 80 + 80 byte rows
    b = [(2000, 64, SparseType.INT8), (1000, 128, SparseType.INT4)]
    c = [(1000, 128, SparseType.INT8), (2000, 32, SparseType.FP16)]  # 144 + 64 byte rows, other total
    for it in range(6):
        specs = (a, b, c)[it % 3]
        m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, output_dtype=FP32)
        m.fill_random_weights(it)
        g = torch.Generator(device=gpu)
        g.manual_seed(it)
        B, L = 16, 9
        off = torch.arange(0, 2 * B * L + 1, L, dtype=torch.int32, device=gpu)
        idx = torch.cat([torch.randint(0, E, (B * L,), device=gpu, generator=g) for E, _, _ in specs]).to(torch.int32)
        _check_module(oracle, m, idx, off, None, f"plan cache round {it}")
        del m, idx, off


def test_plan_cache_sees_in_place_metadata_writes(pkg, oracle, gpu):
    """An in-place write to weights_tys (same tensor, same address) replans."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(500, 64, SparseType.FP16), (500, 64, SparseType.BF16)],
                                                device=gpu, output_dtype=FP32)
    m.fill_random_weights(3)
    idx = torch.randint(0, 500, (80,), device=gpu, dtype=torch.int32)
    off = torch.arange(0, 81, 10, dtype=torch.int32, device=gpu)
    first = m(idx, off, None)
    m.weights_tys[0] = int(SparseType.BF16)  # rows now read as bf16
    m.specs[0] = (500, 64, SparseType.BF16)
    second = m(idx, off, None)
    torch.cuda.synchronize()
    assert not torch.equal(first[:, :64], second[:, :64])
    _check_module(oracle, m, idx, off, None, "in-place weights_tys")


# ----------------------------------------------------------------- nobag rows outside every segment

@pytest.mark.parametrize("out_ty", [FP32, FP16])
@pytest.mark.parametrize("case", ["leading", "trailing", "ragged"])
def test_nobag_rows_outside_segments_are_zero(pkg, oracle, gpu, out_ty, case):
    """offsets[0] > 0, indices past offsets[T*B], and len(offsets)-1 not a multiple of
    T: those output rows are zero (the reference allocates the output with zeros,
    A:135).  The output memory is poisoned beforehand so stale values would show."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    specs = [(300, 16, SparseType.FP32), (200, 16, SparseType.INT8), (100, 16, SparseType.FP16)]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=2, output_dtype=out_ty)
    m.fill_random_weights(9)
    T, B = 3, 5
    lens = [3, 0, 4, 1, 2] * T
    base = {"leading": 70, "trailing": 0, "ragged": 0}[case]
    off = [base] + list(base + np.cumsum(lens))
    if case == "ragged":
        off = off + [off[-1] + 6, off[-1] + 9]  # two extra bags: (len(offsets) - 1) % T != 0
    n_extra = {"leading": 20, "trailing": 150, "ragged": 0}[case]
    N = off[-1] + n_extra
    rs = np.random.RandomState(len(case))
    idx_np = rs.randint(0, 100, N).astype(np.int32)
    for _ in range(3):
        junk = torch.full((N * 16 * 4,), float("nan"), device=gpu)
        del junk
    off_np = np.asarray(off, np.int32)
    out = m(torch.from_numpy(idx_np).to(gpu), torch.from_numpy(off_np).to(gpu), None)
    torch.cuda.synchronize()
    ref, _ = oracle.forward(m.weights_dev.cpu().numpy(), m.weights_offsets.cpu().numpy(),
                            m.weights_tys.cpu().numpy(), m.D_offsets.cpu().numpy(), idx_np, off_np, 2, None,
                            out_ty)
    got = out.cpu()
    assert tuple(got.shape) == ref.shape == (N, 16)
    bits = got.numpy() if out_ty == FP32 else got.view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bits, ref)  # fp16 output: the oracle returns the bit patterns
    first, last = off[0], off[T * ((len(off) - 1) // T)]
    outside = np.r_[0:first, last:N]
    assert not got[outside].float().any()


# ----------------------------------------------------------------- packer: float -> quantised -> op

def _dequantised_table(oracle, m, t):
    """Float rows of table t as the oracle decodes them (nobag over every row)."""
    E, D, ty = m.specs[t]
    rows = m.table_rows(t).cpu().numpy().reshape(-1)
    out, _ = oracle.forward(rows, np.zeros(1, np.int64), np.array([int(ty)], np.uint8),
                            np.array([0, D], np.int32), np.arange(E, dtype=np.int32),
                            np.array([0, E], np.int32), 2, None, FP32,
                            fp8_exponent_bits=m.fp8_exponent_bits, fp8_exponent_bias=m.fp8_exponent_bias)
    return out.astype(np.float64)


def _quant_bound(m, t, w):
    """Per-row bound of |dequantised - float| after load_float_weights."""
    E, D, ty = m.specs[t]
    w = w.double()
    if ty == FP8:
        from fbgemm_ascend_amd import fp8_code_values
        vals = fp8_code_values(m.fp8_exponent_bits, m.fp8_exponent_bias).double()
        k = torch.searchsorted(vals, w.abs()).clamp(1, 127)
        return ((vals[k] - vals[k - 1]) / 2).max(1).values
    bits = {INT8: 8, INT4: 4, INT2: 2}[int(ty)]
    lo, hi = w.min(1).values, w.max(1).values
    step = (hi - lo) / ((1 << bits) - 1)
    # half a step, plus the fp16 rounding of scale (times the largest code) and of bias
    return step / 2 + ((1 << bits) - 1) * step.abs() * 2.0 ** -11 + lo.abs() * 2.0 ** -11 + 1e-7


@pytest.mark.parametrize("ty", [INT8, INT4, INT2, FP8])
@pytest.mark.parametrize("pm,weighted", [(0, False), (1, True)])
def test_packer_float_to_op(pkg, oracle, gpu, ty, pm, weighted):
    """T:121-156 builds a module, fills its rows and runs the op.  Here: float tables
    -> load_float_weights -> the HIP op, checked (1) against F.embedding_bag over the
    oracle's dequantised tables (fp32 tolerance of the parity tests) and (2) against
    F.embedding_bag over the float tables within sum_i |w_i| * (quantisation bound)."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    specs = [(3000, 128, SparseType(ty)), (1500, 64, SparseType(ty)), (700, 32, SparseType(ty))]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=pm, output_dtype=FP32,
                                                fp8_exponent_bits=4 if ty == FP8 else None,
                                                fp8_exponent_bias=7 if ty == FP8 else None)
    g = torch.Generator(device=gpu)
    g.manual_seed(ty * 10 + pm)
    floats = []
    for t, (E, D, _) in enumerate(specs):
        w = torch.randn(E, D, device=gpu, generator=g) * 0.5
        m.load_float_weights(t, w)
        floats.append(w)
    B = 64
    lens = torch.randint(0, 60, (len(specs) * B,), device=gpu, generator=g)
    off = torch.zeros(len(specs) * B + 1, dtype=torch.int64, device=gpu)
    torch.cumsum(lens, 0, out=off[1:])
    offs = off.cpu()
    idx = torch.cat([torch.randint(0, E, (int(offs[(t + 1) * B] - offs[t * B]),), device=gpu, generator=g)
                     for t, (E, _, _) in enumerate(specs)])
    psw = torch.rand(idx.numel(), device=gpu, generator=g) if weighted else None
    _say(f"[gpu] packer ty={ty} pm={pm} w={weighted}")
    out = m(idx, off, psw).double().cpu()

    def bag_sum(it, table, bo, pw, n):
        # SUM; MEAN = weighted sum x float(1)/float(L) (P:355), not a weighted average
        r = torch.nn.functional.embedding_bag(it, table, bo, mode="sum", per_sample_weights=pw)
        if pm == 1:
            L = torch.diff(torch.cat([bo, torch.tensor([n])])).clamp(min=1).double()
            r = r / L[:, None]
        return r
    for t, (E, D, _) in enumerate(specs):
        lo, hi = int(offs[t * B]), int(offs[(t + 1) * B])
        it = idx[lo:hi].cpu()
        bo = (offs[t * B:(t + 1) * B] - lo).cpu()
        pw = psw[lo:hi].double().cpu() if weighted else None
        cols = slice(int(m.D_offsets[t]), int(m.D_offsets[t + 1]))
        got = out[:, cols]
        # (1) the dequantised table
        deq = torch.from_numpy(_dequantised_table(oracle, m, t))
        n = hi - lo
        ref = bag_sum(it, deq, bo, pw, n)
        rowmax = deq.abs().max(1).values
        mag = bag_sum(it, rowmax[:, None], bo, None if pw is None else pw.abs(), n)
        assert bool(((got - ref).abs() <= 1e-5 * (mag + ref.abs()) + 1e-30).all()), f"table {t} vs dequantised"
        # (2) the float table within the quantisation bound
        fl = floats[t].double().cpu()
        ref_f = bag_sum(it, fl, bo, pw, n)
        qb = _quant_bound(m, t, floats[t].cpu())
        bound = bag_sum(it, qb[:, None], bo, None if pw is None else pw.abs(), n)
        err = (got - ref_f).abs()
        assert bool((err <= bound * (1 + 1e-6) + 1e-5 * (mag + ref_f.abs())).all()), f"table {t} vs float"
        # the quantisation is not a no-op: the bound is tight enough to matter
        assert float(err.max()) > 0


# ----------------------------------------------------------------- the module's bound forward

def _op_call(m, idx, off, psw):
    return torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
        dev_weights=m.weights_dev, uvm_weights=m.weights_uvm, weights_placements=m.weights_placements,
        weights_offsets=m.weights_offsets, weights_tys=m.weights_tys, D_offsets=m.D_offsets,
        total_D=m.total_D, max_int2_D=m.max_int2_D, max_int4_D=m.max_int4_D, max_int8_D=m.max_int8_D,
        max_float16_D=m.max_float16_D, max_float32_D=m.max_float32_D, indices=idx, offsets=off,
        pooling_mode=int(m.pooling_mode), indice_weights=psw, output_dtype=m.output_dtype,
        lxu_cache_weights=None, lxu_cache_locations=None, row_alignment=m.row_alignment,
        max_float8_D=m.max_float8_D, fp8_exponent_bits=m.fp8_exponent_bits,
        fp8_exponent_bias=m.fp8_exponent_bias)


@pytest.mark.parametrize("ty,pm,weighted,out_ty", [(INT4, 0, False, FP16), (INT8, 1, True, FP32),
                                                   (FP8, 2, False, BF16), (INT2, 0, True, FP32)])
def test_module_forward_equals_op(pkg, gpu, ty, pm, weighted, out_ty):
    """The module's forward (its bound C++ call) returns the op's output bit for bit."""
    m, idx, off, psw = _random_case(pkg, gpu, 77, 3, ty, pm, weighted, torch.int32, out_ty, B=32, L=40)
    got, want = m(idx, off, psw), _op_call(m, idx, off, psw)
    torch.cuda.synchronize()
    assert got.dtype == want.dtype and got.shape == want.shape
    assert torch.equal(got, want)


def test_module_rebinds_after_changes(pkg, gpu):
    """Attribute writes, buffer replacement and .to() drop the bound call; the next
    forward follows the module's current state."""
    m, idx, off, _ = _random_case(pkg, gpu, 78, 2, INT8, 0, False, torch.int64, FP16, B=16, L=20)
    first = m(idx, off)
    assert first.dtype == torch.float16
    m.output_dtype = FP32
    second = m(idx, off)
    assert second.dtype == torch.float32
    assert torch.equal(second, _op_call(m, idx, off, None))
    m.weights_dev = torch.zeros_like(m.weights_dev)  # every row: scale 0, bias 0
    assert torch.count_nonzero(m(idx, off)) == 0
    m.fill_random_weights(5)  # in place: same tensor, bound call kept
    assert torch.equal(m(idx, off), _op_call(m, idx, off, None))
    m = m.to(gpu)
    assert torch.equal(m(idx, off), _op_call(m, idx, off, None))
    m.register_buffer("weights_dev", torch.zeros_like(m.weights_dev))
    assert torch.count_nonzero(m(idx, off)) == 0
    torch.cuda.synchronize()
