"""GPU parity: the HIP path against the CPU oracle on identical inputs.

Runs under `-m gpu` on an MI355X.  Every comparison uses the tolerance stated in
tests/_parity.py (bit-exact where the inputs make the arithmetic exact).  The
test matrix follows the reference's own test (reference
bench/tbe_inference/.../test_int_nbit_split_embedding_codegen_lookup_function.py,
"T"): FP8 tables, SUM/MEAN/NONE x weighted x int32/int64 x fp16/fp32/bf16 x
1..10 random tables (T:372-414), the fixed two-table bag/nobag lists (T:417-487),
and the same matrix for the INT8/INT4/INT2/FP16/FP32/BF16 row formats.
"""
import random
import sys
import zlib

import numpy as np
import pytest
import torch

from _parity import RTOL, assert_bag_parity, compact_problem, run_oracle, ulp_stats
from test_oracle import _kat_problem, kat_expected

pytestmark = pytest.mark.gpu

FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6
OUT_TORCH = {FP32: torch.float32, FP16: torch.float16, BF16: torch.bfloat16}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _op(module, indices, offsets, psw):
    return module(indices, offsets, psw)


def _capi_run(pkg, module, indices, offsets, psw, flags):
    """The forward through the C ABI with TBE_FLAG_* switches (same inputs as the op)."""
    return pkg.capi.forward_tensors(module.weights_dev, module.weights_offsets, module.weights_tys, module.D_offsets,
                                    indices, offsets, int(module.pooling_mode), psw, module.output_dtype,
                                    module.row_alignment, getattr(module, "fp8_exponent_bits", -1),
                                    getattr(module, "fp8_exponent_bias", -1), flags=flags)


def _check_module(oracle, module, indices, offsets, psw, label, b_sel=None, flags=None, ulps=None):
    """Run the op on the GPU (through the C ABI with `flags` when given) and compare
    with the oracle on the (sub)problem.  `ulps` (a dict) receives the distance in
    output-dtype ulps to the oracle's own output."""
    import fbgemm_ascend_amd as pkg
    _say(f"[gpu] {label}: T={len(module.specs)} N={indices.numel()} bags={offsets.numel() - 1} flags={flags}")
    if flags is None:
        out = _op(module, indices, offsets, psw)
    else:
        out = _capi_run(pkg, module, indices, offsets, psw if int(module.pooling_mode) != 2 else None, flags)
    torch.cuda.synchronize()
    pm = int(module.pooling_mode)
    prob = compact_problem(module, indices, offsets, psw if pm != 2 else None, b_sel)
    ref, ref32 = run_oracle(oracle, prob, pm, module.output_dtype, module.row_alignment)
    got = out if (b_sel is None or pm == 2) else out[prob["b_sel"]]
    assert got.dtype == OUT_TORCH[module.output_dtype]
    assert tuple(got.shape) == ref32.shape
    ratio = assert_bag_parity(got, prob, ref32, pm, module.output_dtype, label)
    if ulps is not None:
        ulps["max"], ulps["equal"] = ulp_stats(got, ref, module.output_dtype)
    return ratio


# ----------------------------------------------------------------- exact known answers

def _module_from_arrays(pkg, gpu, w, wo, wt, do, pm, out_ty, fp8=(4, 7)):
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    T = len(wo)
    specs = []
    for t in range(T):
        D = int(do[t + 1] - do[t])
        specs.append((1, D, SparseType(int(wt[t]))))  # E fixed up below
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=pm, output_dtype=out_ty,
                                                fp8_exponent_bits=fp8[0], fp8_exponent_bias=fp8[1])
    # install the prepared buffer and offsets verbatim
    m.weights_dev = torch.from_numpy(np.ascontiguousarray(w)).to(gpu)
    m.weights_offsets = torch.from_numpy(np.asarray(wo, np.int64)).to(gpu)
    E = [int(((wo[t + 1] if t + 1 < T else len(w)) - wo[t]) // m.row_strides[t]) for t in range(T)]
    m.specs = [(E[t], s[1], s[2]) for t, s in enumerate(m.specs)]
    m._offs = [int(x) for x in wo]
    return m


@pytest.mark.parametrize("idx_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("pm", [0, 1])
def test_kat_bit_exact(pkg, oracle, gpu, idx_dtype, pm):
    rs = np.random.RandomState(7)
    tables = [(37, 16, INT8), (53, 32, INT4), (29, 64, INT2), (41, 8, FP16), (23, 12, FP32),
              (31, 20, FP8), (19, 6, BF16), (300, 128, INT4), (200, 128, INT8), (50, 4096, FP8),
              # every lanes-per-row width (1..64) with and without the scale/bias header
              (29, 32, INT8), (31, 64, INT4), (33, 128, INT2), (20, 4, FP32), (21, 16, INT2),
              (22, 8, INT4), (23, 4, INT8), (24, 2, FP16), (25, 32, INT2), (26, 256, INT8),
              (27, 512, INT4), (28, 64, FP32)]
    B = 13
    w, wo, wt, do, idx, off, vals, lengths = _kat_problem(rs, tables, B, idx_dtype, Lmax=150)
    m = _module_from_arrays(pkg, gpu, w, wo, wt, do, pm, FP32)
    _say(f"[gpu] kat pm={pm} idx={np.dtype(idx_dtype).name}")
    out = m(torch.from_numpy(idx).to(gpu), torch.from_numpy(off).to(gpu), None)
    ref, _ = oracle.forward(w, wo, wt, do, idx, off, pm, None, FP32, fp8_exponent_bits=4,
                            fp8_exponent_bias=7)
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got, ref)
    if pm == 0:
        np.testing.assert_array_equal(got, kat_expected(vals, do, idx, off, B, lengths, 0).astype(np.float32))


def test_kat_nobag_bit_exact(pkg, oracle, gpu):
    rs = np.random.RandomState(8)
    for D, tys in ((32, (INT8, INT4, FP16, INT2)), (256, (FP8, FP32, BF16, INT4))):
        tables = [(37 + 11 * i, D, ty) for i, ty in enumerate(tys)]
        w, wo, wt, do, idx, off, vals, lengths = _kat_problem(rs, tables, 9, np.int32)
        m = _module_from_arrays(pkg, gpu, w, wo, wt, do, 2, FP32)
        _say(f"[gpu] kat nobag D={D}")
        out = m(torch.from_numpy(idx).to(gpu), torch.from_numpy(off).to(gpu), None)
        ref, _ = oracle.forward(w, wo, wt, do, idx, off, 2, None, FP32, fp8_exponent_bits=4,
                                fp8_exponent_bias=7)
        np.testing.assert_array_equal(out.cpu().numpy(), ref)


# ----------------------------------------------------------------- golden library vectors

@pytest.mark.parametrize("B", [1, 2, 7, 31])
def test_small_batches_cover_every_bag(pkg, oracle, gpu, B):
    """Launches with fewer blocks than XCDs still pool every bag."""
    rs = np.random.RandomState(B)
    tables = [(40, 16, INT8), (30, 32, INT8), (20, 128, INT4)]
    w, wo, wt, do, idx, off, vals, lengths = _kat_problem(rs, tables, B, np.int64, Lmax=9)
    m = _module_from_arrays(pkg, gpu, w, wo, wt, do, 0, FP32)
    out = m(torch.from_numpy(idx).to(gpu), torch.from_numpy(off).to(gpu), None)
    np.testing.assert_array_equal(out.cpu().numpy(),
                                  kat_expected(vals, do, idx, off, B, lengths, 0).astype(np.float32))


def test_golden_library_vectors_gpu(pkg, golden, gpu):
    for name in [str(n) for n in golden["case_names"]]:
        g = {k: golden[f"{name}/{k}"] for k in ("weights", "weights_offsets", "weights_tys", "D_offsets",
                                                 "indices", "offsets", "psw", "pooling_mode", "expected")}
        pm = int(g["pooling_mode"])
        m = _module_from_arrays(pkg, gpu, g["weights"], g["weights_offsets"], g["weights_tys"],
                                g["D_offsets"], pm, FP32)
        psw = torch.from_numpy(g["psw"]).to(gpu) if g["psw"].size else None
        _say(f"[gpu] golden {name}")
        out = m(torch.from_numpy(g["indices"]).to(gpu), torch.from_numpy(g["offsets"]).to(gpu), psw)
        np.testing.assert_allclose(out.cpu().numpy(), g["expected"], rtol=1e-5, atol=1e-5, err_msg=name)


# ----------------------------------------------------------------- reference test matrix

def _random_case(pkg, gpu, seed, T, ty, pm, weighted, idx_dtype, out_ty, B=64, L=100,
                 tables=None, L_list=None):
    """T:159-277: E ~ U[1,20000], D = align * U[1, 1024/...], fixed L_t ~ U[1,L] per table."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    rnd = random.Random(seed)
    ty = SparseType(ty)
    align = max(ty.align_size(), 4)
    dmax = 4096 if ty.bit_rate() <= 8 else 1024  # rows of at most 4 KiB, like the FP8 cases
    if tables is None:
        tables, L_list = [], []
        Dn = align * rnd.randint(1, dmax // align)
        for _ in range(T):
            D = Dn if pm == 2 else align * rnd.randint(1, dmax // align)
            tables.append((rnd.randint(1, 20000), D))
            L_list.append(rnd.randint(1, L))
    specs = [(E, D, ty) for E, D in tables]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=pm, output_dtype=out_ty,
                                                indices_dtype=idx_dtype)
    m.fill_random_weights(seed)
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    idx = torch.cat([torch.randint(0, E, (B * Lt,), device=gpu, generator=g)
                     for (E, _), Lt in zip(tables, L_list)]).to(idx_dtype)
    lens = torch.tensor([Lt for Lt in L_list for _ in range(B)], device=gpu)
    off = torch.zeros(len(tables) * B + 1, dtype=torch.int64, device=gpu)
    torch.cumsum(lens, 0, out=off[1:])
    psw = torch.rand(idx.numel(), device=gpu, generator=g) if weighted else None
    return m, idx, off.to(idx_dtype), psw


def _matrix_params(types):
    params = []
    for ty in types:
        for pm in (0, 1, 2):
            for weighted in (True, False):
                for idx_dtype in (torch.int32, torch.int64):
                    for out_ty in (FP16, FP32, BF16):
                        if pm == 2 and (weighted or idx_dtype != torch.int32):
                            continue  # T:398-402
                        params.append((ty, pm, weighted, idx_dtype, out_ty))
    return params


@pytest.mark.parametrize("kernel", ["default", "stream"])
@pytest.mark.parametrize("T", list(range(1, 11)))
@pytest.mark.parametrize("ty,pm,weighted,idx_dtype,out_ty", _matrix_params([FP8]))
def test_random_multi_table_forward_fp8(pkg, oracle, gpu, T, ty, pm, weighted, idx_dtype, out_ty, kernel):
    seed = zlib.crc32(repr((T, ty, pm, weighted, str(idx_dtype), out_ty)).encode()) & 0xFFFF
    m, idx, off, psw = _random_case(pkg, gpu, seed, T, ty, pm, weighted, idx_dtype, out_ty)
    flags = pkg.capi.TBE_FLAG_FORCE_STREAM if kernel == "stream" else None
    _check_module(oracle, m, idx, off, psw, f"fp8 T={T} pm={pm} w={weighted} {idx_dtype} out={out_ty}", flags=flags)


@pytest.mark.parametrize("kernel", ["default", "stream"])
@pytest.mark.parametrize("T", [2, 5])
@pytest.mark.parametrize("ty,pm,weighted,idx_dtype,out_ty", _matrix_params([INT8, INT4, INT2, FP16, FP32, BF16]))
def test_random_multi_table_forward_types(pkg, oracle, gpu, T, ty, pm, weighted, idx_dtype, out_ty, kernel):
    seed = zlib.crc32(repr((T, ty, pm, weighted, str(idx_dtype), out_ty, "t")).encode()) & 0xFFFF
    m, idx, off, psw = _random_case(pkg, gpu, seed, T, ty, pm, weighted, idx_dtype, out_ty)
    flags = pkg.capi.TBE_FLAG_FORCE_STREAM if kernel == "stream" else None
    _check_module(oracle, m, idx, off, psw, f"ty={ty} T={T} pm={pm} w={weighted} {idx_dtype} out={out_ty}",
                  flags=flags)


# INT4 rows of 17-32 payload words: tables with an even word count read two words
# per lane in the per-bag kernel, odd ones (D=136, 248) one; mixed in one call
# they form two groups.  TBE_FLAG_NARROW_WORDS keeps one word per lane.
INT4_WIDE_TABLES = [[(3000, 256), (2000, 192)], [(3000, 144), (2000, 136), (1000, 248), (500, 256)],
                    [(20000, 240)]]


@pytest.mark.parametrize("words", ["default", "narrow"])
@pytest.mark.parametrize("tables", list(range(len(INT4_WIDE_TABLES))))
@pytest.mark.parametrize("pm,weighted,out_ty", [(0, False, FP16), (1, True, FP32), (0, True, BF16), (1, False, FP16)])
def test_int4_wide_word_lanes(pkg, oracle, gpu, tables, pm, weighted, out_ty, words):
    tabs = INT4_WIDE_TABLES[tables]
    seed = 0x44 + 7 * tables + 3 * pm + int(weighted)
    m, idx, off, psw = _random_case(pkg, gpu, seed, len(tabs), INT4, pm, weighted, torch.int32, out_ty, B=97,
                                    tables=tabs, L_list=[1 + (13 * k + seed) % 150 for k in range(len(tabs))])
    flags = pkg.capi.TBE_FLAG_NARROW_WORDS if words == "narrow" else 0
    _check_module(oracle, m, idx, off, psw, f"int4 wide {tabs} pm={pm} w={weighted} out={out_ty} {words}",
                  flags=flags)


BAG_TABLES = [[(1000, 16), (2000, 16)], [(2000, 256), (1000, 256)], [(2000, 512), (1000, 512)],
              [(2000, 1024), (1000, 1024)], [(2000, 2048), (1000, 2048)], [(2000, 4096), (1000, 4096)],
              [(2000, 16), (1000, 256)], [(2000, 16), (1000, 512)], [(2000, 16), (1000, 1024)],
              [(2000, 16), (1000, 2048)], [(2000, 16), (1000, 4096)]]  # T:418-425
NOBAG_TABLES = [[(1000, 16), (2000, 16)], [(1000, 32), (2000, 32)], [(1000, 64), (2000, 64)],
                [(1000, 128), (2000, 128)], [(2000, 256), (1000, 256)], [(2000, 512), (1000, 512)],
                [(2000, 1024), (1000, 1024)], [(2000, 2048), (1000, 2048)],
                [(2000, 4096), (1000, 4096)]]  # T:428-433


@pytest.mark.parametrize("tables", BAG_TABLES, ids=lambda t: "-".join(f"{e}x{d}" for e, d in t))
@pytest.mark.parametrize("out_ty", [FP16, FP32, BF16])
@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("weighted", [True, False])
@pytest.mark.parametrize("pm", [0, 1])
def test_double_table_forward_bag(pkg, oracle, gpu, tables, out_ty, idx_dtype, weighted, pm):
    m, idx, off, psw = _random_case(pkg, gpu, 1234, 2, FP8, pm, weighted, idx_dtype, out_ty,
                                    tables=tables, L_list=[40, 50])
    _check_module(oracle, m, idx, off, psw, f"double bag {tables} pm={pm} w={weighted}")


@pytest.mark.parametrize("tables", NOBAG_TABLES, ids=lambda t: "-".join(f"{e}x{d}" for e, d in t))
@pytest.mark.parametrize("out_ty", [FP16, FP32, BF16])
def test_double_table_forward_nobag(pkg, oracle, gpu, tables, out_ty):
    m, idx, off, psw = _random_case(pkg, gpu, 4321, 2, FP8, 2, False, torch.int32, out_ty,
                                    tables=tables, L_list=[40, 50])
    _check_module(oracle, m, idx, off, psw, f"double nobag {tables}")


# ----------------------------------------------------------------- boundary behaviour

def test_c_abi_matches_torch_op(pkg, gpu):
    """The C ABI called directly (ctypes) gives the torch op's exact output, with and
    without the XCD block renumbering, and with the table groups on the caller's
    stream instead of the two group streams."""
    from fbgemm_ascend_amd.workloads import make_workload
    for cid in (1, 3):
        wl = make_workload(cid, device=gpu, scale_rows=0.01, batch=256)
        m = wl.module
        _say(f"[gpu] c-abi cfg{cid}")
        a = wl.run()
        for flags in (0, pkg.capi.TBE_FLAG_NO_XCD_REMAP, pkg.capi.TBE_FLAG_SERIAL_GROUPS):
            b = pkg.capi.forward_tensors(m.weights_dev, m.weights_offsets, m.weights_tys, m.D_offsets,
                                         wl.indices, wl.offsets, int(m.pooling_mode),
                                         wl.per_sample_weights, m.output_dtype, flags=flags)
            torch.cuda.synchronize()
            assert torch.equal(a, b)


def test_edge_cases(pkg, oracle, gpu):
    """Empty bags, bags longer than one 64-index chunk, out-of-range rows, a batch of 1."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    specs = [(500, 128, SparseType.INT4), (300, 64, SparseType.INT8), (200, 32, SparseType.INT2),
             (100, 48, SparseType.FP16)]
    for B in (1, 37):
        m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=1,
                                                    output_dtype=FP32)
        m.fill_random_weights(5)
        g = torch.Generator(device=gpu)
        g.manual_seed(B)
        lens = torch.randint(0, 300, (len(specs) * B,), device=gpu, generator=g)
        lens[::3] = 0
        off = torch.zeros(len(lens) + 1, dtype=torch.int64, device=gpu)
        torch.cumsum(lens, 0, out=off[1:])
        N = int(off[-1])
        idx = torch.randint(-5, 520, (N,), device=gpu, generator=g)  # some rows out of range
        psw = torch.rand(N, device=gpu, generator=g)
        _check_module(oracle, m, idx, off, psw, f"edge B={B}")


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_degenerate_sizes(pkg, gpu, idx_dtype):
    """Calls with no indices at all (B = 0, or every bag empty): the op rejects them
    as the reference does (A:117, "indices can not be empty tensor."); the C ABI
    accepts them and leaves every bag zero (A:155) or the output empty."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    specs = [(50, 64, SparseType.INT4), (40, 32, SparseType.INT8), (30, 16, SparseType.FP16)]
    for pm in (0, 1, 2):
        sp = specs if pm != 2 else [(50, 32, SparseType.INT4), (40, 32, SparseType.INT8)]
        m = IntNBitTableBatchedEmbeddingBagsCodegen(sp, device=gpu, pooling_mode=pm,
                                                    output_dtype=FP16, indices_dtype=idx_dtype)
        m.fill_random_weights(3)
        no_idx = torch.zeros(0, dtype=idx_dtype, device=gpu)
        for B in (0, 5):
            off = torch.zeros(len(sp) * B + 1, dtype=idx_dtype, device=gpu)
            _say(f"[gpu] degenerate pm={pm} B={B} {idx_dtype}")
            with pytest.raises(RuntimeError, match="indices can not be empty tensor"):
                _op(m, no_idx, off, None)
            out = _capi_run(pkg, m, no_idx, off, None, 0)
            torch.cuda.synchronize()
            rows = 0 if pm == 2 else B
            assert tuple(out.shape) == (rows, m.total_D if pm != 2 else 32)
            assert out.numel() == 0 or int(torch.count_nonzero(out)) == 0


def test_malformed_offsets_stay_in_bounds(pkg, gpu):
    """Offsets past the index array are clamped to it (no out-of-bounds read)."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(100, 64, SparseType.INT8)], device=gpu, output_dtype=FP32)
    m.fill_random_weights(1)
    idx = torch.randint(0, 100, (40,), device=gpu)
    off = torch.tensor([0, 10, 30, 10 ** 6, 40], device=gpu)
    out = m(idx, off, None)
    good = torch.tensor([0, 10, 30, 40, 40], device=gpu)
    ref = m(idx, good, None)
    torch.cuda.synchronize()
    assert torch.equal(out[:2], ref[:2]) and torch.equal(out[3], torch.zeros_like(out[3]))


def test_validation_errors(pkg, gpu):
    """The adapter's argument checks (A:116-151, H:110-204) raise instead of launching."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(10, 16, SparseType.INT8), (10, 32, SparseType.INT4)],
                                                device=gpu, output_dtype=FP32)
    idx = torch.randint(0, 10, (8,), device=gpu, dtype=torch.int32)
    off = torch.tensor([0, 2, 4, 6, 8], device=gpu, dtype=torch.int32)
    op = torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function

    def call(**kw):
        args = dict(dev_weights=m.weights_dev, uvm_weights=m.weights_uvm,
                    weights_placements=m.weights_placements, weights_offsets=m.weights_offsets,
                    weights_tys=m.weights_tys, D_offsets=m.D_offsets, total_D=m.total_D,
                    max_int2_D=0, max_int4_D=32, max_int8_D=16, max_float16_D=0, max_float32_D=0,
                    indices=idx, offsets=off, pooling_mode=0, indice_weights=None, output_dtype=0,
                    lxu_cache_weights=None, lxu_cache_locations=None, row_alignment=16,
                    max_float8_D=0, fp8_exponent_bits=-1, fp8_exponent_bias=-1)
        args.update(kw)
        return op(**args)

    call()
    with pytest.raises(RuntimeError, match="indices can not be empty"):
        call(indices=idx[:0], offsets=off[:1])
    with pytest.raises(RuntimeError, match="is incorrect for feature count"):
        call(offsets=off[:4])
    with pytest.raises(RuntimeError, match="Unsupported output_dtype"):
        call(output_dtype=3)
    # A:125-129: mixed tables fail the reference's own check, with its message
    with pytest.raises(RuntimeError, match="int8 output_dtype requires all tables to use int8 weights"):
        call(output_dtype=2)
    # all-INT8 tables pass it and meet the kernels' rejection (P:336-338)
    m8 = IntNBitTableBatchedEmbeddingBagsCodegen([(10, 16, SparseType.INT8)], device=gpu, output_dtype=FP32)
    with pytest.raises(RuntimeError, match="INT8 output_dtype is not supported"):
        op(dev_weights=m8.weights_dev, uvm_weights=m8.weights_uvm, weights_placements=m8.weights_placements,
           weights_offsets=m8.weights_offsets, weights_tys=m8.weights_tys, D_offsets=m8.D_offsets,
           total_D=m8.total_D, max_int2_D=0, max_int4_D=0, max_int8_D=16, max_float16_D=0, max_float32_D=0,
           indices=idx, offsets=off[:3], pooling_mode=0, indice_weights=None, output_dtype=2,
           lxu_cache_weights=None, lxu_cache_locations=None, row_alignment=16, max_float8_D=0,
           fp8_exponent_bits=-1, fp8_exponent_bias=-1)
    with pytest.raises(RuntimeError, match="Len mismatch"):
        call(indice_weights=torch.rand(3, device=gpu))
    with pytest.raises(RuntimeError, match="pooling mode"):
        call(pooling_mode=4)
    with pytest.raises(RuntimeError, match="nobag mode requires"):
        call(pooling_mode=2)
    with pytest.raises(RuntimeError, match="weights_tys size"):
        call(weights_tys=m.weights_tys[:1])
    # offsets of another integer type follow the indices' dtype (A:110-113)
    a = call(offsets=off.to(torch.int64))
    b = call()
    assert torch.equal(a, b)


# ----------------------------------------------------------------- the five benchmark configurations

def _assert_16bit_close(module, u):
    """fp16 / bf16 outputs: beyond the summed-magnitude limit, nearly every element equals
    the oracle's rounded output and none is more than a few ulps away (only the fp32
    summation order differs).  fp32 outputs are held to the limit alone: near-zero sums
    make ulp distances meaningless there."""
    if module.output_dtype in (FP16, BF16):
        assert u["max"] <= 4 and u["equal"] >= 0.999, u

def _free_gib():
    free, _ = torch.cuda.mem_get_info()
    return free / 2 ** 30


@pytest.mark.parametrize("cid", [0, 1, 2, 3])
def test_config_full_parity(pkg, oracle, gpu, cid):
    from fbgemm_ascend_amd.workloads import make_workload
    wl = make_workload(cid, device=gpu)
    u = {}
    ratio = _check_module(oracle, wl.module, wl.indices, wl.offsets, wl.per_sample_weights,
                          f"config {cid} ({wl.spec.description})", ulps=u)
    _say(f"[gpu] config {cid}: max err/limit = {ratio:.3f}, max distance to the oracle's output "
         f"{u['max']} ulp, bit-identical {100 * u['equal']:.3f} %")
    _assert_16bit_close(wl.module, u)
    del wl
    torch.cuda.empty_cache()


@pytest.mark.parametrize("cid", [0, 1, 2, 3])
@pytest.mark.parametrize("kernel", ["per_bag", "stream"])
def test_config_kernel_choice_parity(pkg, oracle, gpu, cid, kernel):
    """Both pooled kernels meet the same bar whatever the default choice for the
    group: TBE_FLAG_NO_STREAM forces the per-bag kernel, TBE_FLAG_FORCE_STREAM the
    row-stream kernel for every eligible group (configs at 1/8 batch)."""
    from fbgemm_ascend_amd.workloads import make_workload
    wl = make_workload(cid, device=gpu, batch=max(1, {0: 512, 1: 2048, 2: 8192, 3: 16384}[cid] // 8))
    m = wl.module
    flags = pkg.capi.TBE_FLAG_NO_STREAM if kernel == "per_bag" else pkg.capi.TBE_FLAG_FORCE_STREAM
    _say(f"[gpu] {kernel} kernel, config {cid}")
    out = pkg.capi.forward_tensors(m.weights_dev, m.weights_offsets, m.weights_tys, m.D_offsets, wl.indices,
                                   wl.offsets, int(m.pooling_mode), wl.per_sample_weights, m.output_dtype,
                                   flags=flags)
    torch.cuda.synchronize()
    prob = compact_problem(m, wl.indices, wl.offsets, wl.per_sample_weights, None)
    _, ref32 = run_oracle(oracle, prob, int(m.pooling_mode), m.output_dtype, m.row_alignment)
    assert_bag_parity(out, prob, ref32, int(m.pooling_mode), m.output_dtype, f"{kernel} config {cid}")
    del wl
    torch.cuda.empty_cache()


def test_double_table_forward_bag_stream(pkg, oracle, gpu):
    """The reference's fixed two-table bag lists (T:418-425) through the row-stream
    kernel, every output dtype, weighted MEAN and plain SUM."""
    for tables in BAG_TABLES:
        for out_ty in (FP16, FP32, BF16):
            for pm, weighted in ((0, False), (1, True)):
                m, idx, off, psw = _random_case(pkg, gpu, 1234, 2, FP8, pm, weighted, torch.int64, out_ty,
                                                tables=tables, L_list=[40, 50])
                _check_module(oracle, m, idx, off, psw, f"double bag {tables} pm={pm} out={out_ty}",
                              flags=pkg.capi.TBE_FLAG_FORCE_STREAM)


@pytest.mark.parametrize("kernel", ["per_bag", "stream"])
def test_table_above_2gib_32bit_addressing(pkg, oracle, gpu, kernel):
    """A 2.3 GB FP16 table (rows beyond the 2 GiB byte offset) next to a small INT4
    table, addressed with 32-bit offsets; indices hit the table's last rows."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    if _free_gib() < 8:
        pytest.skip("needs ~3 GiB of free HBM")
    rows = 4_500_000
    m = IntNBitTableBatchedEmbeddingBagsCodegen([(rows, 256, SparseType.FP16), (1000, 128, SparseType.INT4)],
                                                device=gpu, pooling_mode=0, output_dtype=FP32)
    m.fill_random_weights(11)
    g = torch.Generator(device=gpu)
    g.manual_seed(11)
    B, L = 64, 24
    off = torch.arange(0, 2 * B * L + 1, L, dtype=torch.int64, device=gpu)
    big = torch.randint(rows - 20000, rows + 3, (B * L,), device=gpu, generator=g)  # last rows, a few out of range
    big[::7] = torch.randint(0, rows, (big[::7].numel(),), device=gpu, generator=g)
    small = torch.randint(0, 1000, (B * L,), device=gpu, generator=g)
    idx = torch.cat([big, small])
    flags = pkg.capi.TBE_FLAG_NO_STREAM if kernel == "per_bag" else pkg.capi.TBE_FLAG_FORCE_STREAM
    _check_module(oracle, m, idx, off, None, f"2.3 GB table, {kernel}", flags=flags)
    del m
    torch.cuda.empty_cache()


def test_stream_kernel_bag_splits(pkg, oracle, gpu):
    """Row-stream kernel: one very long bag among short and empty ones (slots that get
    no bag, a bag that spans several index chunks, empty bags at a wave's start and
    end), every bags-per-wave boundary position (B = 1..70)."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    specs = [(300, 128, SparseType.INT4), (200, 128, SparseType.INT8), (100, 256, SparseType.FP16)]
    rnd = random.Random(7)
    for B in (1, 2, 31, 32, 33, 63, 64, 65, 70):
        for pm, weighted in ((0, False), (1, True)):
            m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=pm, output_dtype=FP32)
            m.fill_random_weights(B)
            lens = [rnd.choice([0, 0, 1, 3, 17, 40]) for _ in range(3 * B)]
            lens[0] = 0
            lens[-1] = 0
            lens[rnd.randrange(1, 3 * B - 1)] = 700
            off = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int64, device=gpu)
            N = int(off[-1])
            g = torch.Generator(device=gpu)
            g.manual_seed(B)
            idx = torch.randint(-3, 320, (N,), device=gpu, generator=g)
            psw = torch.rand(N, device=gpu, generator=g) if weighted else None
            _check_module(oracle, m, idx, off, psw, f"stream splits B={B} pm={pm}",
                          flags=pkg.capi.TBE_FLAG_FORCE_STREAM)


def test_config4_sampled_parity(pkg, oracle, gpu):
    """200 x 10M INT4 rows (~160 GB) resident in HBM; parity on 1024 sampled samples
    (all 200 tables each), rows taken from device memory."""
    from fbgemm_ascend_amd.workloads import make_workload
    if _free_gib() < 200:
        pytest.skip(f"config 4 needs ~175 GiB of free HBM, have {_free_gib():.0f}")
    wl = make_workload(4, device=gpu)
    g = torch.Generator(device=gpu)
    g.manual_seed(4)
    b_sel = torch.randperm(wl.spec.B, device=gpu, generator=g)[:1024].sort().values
    u = {}
    ratio = _check_module(oracle, wl.module, wl.indices, wl.offsets, None, "config 4 sampled", b_sel, ulps=u)
    _say(f"[gpu] config 4 (sampled): max err/limit = {ratio:.3f}, max distance to the oracle's output "
         f"{u['max']} ulp, bit-identical {100 * u['equal']:.3f} %")
    _assert_16bit_close(wl.module, u)
    del wl
    torch.cuda.empty_cache()
