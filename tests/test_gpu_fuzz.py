"""Seeded random mixes against the oracle: modules whose tables mix every row type,
width and row alignment (so the planner forms several groups, the group streams
run and each group gets its own kernel shape), with random bag lengths (empty bags
included), pooling modes, per-sample weights, index widths, output dtypes, FP8
parameters and kernel switches (default, row-stream forced, per-bag only, one word
per lane, serial groups, hardware block order).

The matrices of test_gpu_parity.py hold one row type per module; these cases cover
the combinations between them.  Each case is small (T <= 10, B <= 48) and checked
with the same tolerance (tests/_parity.py).
"""
import random

import pytest
import torch

from test_gpu_parity import _check_module

pytestmark = pytest.mark.gpu

FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6


def _case(pkg, gpu, seed):
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    rnd = random.Random(seed)
    pm = rnd.choice([0, 0, 1, 2])
    T = rnd.randint(1, 10)
    types = [rnd.choice([FP32, FP16, BF16, INT8, INT4, INT2, FP8]) for _ in range(T)]
    if pm == 2:
        D = 16 * rnd.randint(1, 32)  # nobag: one D for every table, a multiple of every alignment
        dims = [D] * T
    else:
        steps = [max(SparseType(ty).align_size(), 4) for ty in types]
        dims = [a * rnd.randint(1, 512 // a) for a in steps]
    specs = [(rnd.randint(1, 3000), D, SparseType(ty)) for ty, D in zip(types, dims)]
    out_ty = rnd.choice([FP32, FP16, BF16])
    idx_dtype = rnd.choice([torch.int32, torch.int64])
    row_alignment = rnd.choice([4, 8, 16, 16, 32])
    fp8 = rnd.choice([(4, 7), (5, 15), (3, 3), (4, 10)])
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=pm, output_dtype=out_ty,
                                                indices_dtype=idx_dtype, row_alignment=row_alignment,
                                                fp8_exponent_bits=fp8[0], fp8_exponent_bias=fp8[1])
    m.fill_random_weights(seed)
    B = rnd.randint(1, 48)
    Lmax = rnd.choice([1, 3, 30, 100])
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    lens = torch.randint(0, Lmax + 1, (T * B,), device=gpu, generator=g)
    off = torch.zeros(T * B + 1, dtype=torch.int64, device=gpu)
    torch.cumsum(lens, 0, out=off[1:])
    offs = off.tolist()
    parts = [torch.randint(0, E, (offs[(t + 1) * B] - offs[t * B],), device=gpu, generator=g)
             for t, (E, _, _) in enumerate(specs)]
    idx = torch.cat(parts).to(idx_dtype)
    weighted = pm != 2 and rnd.random() < 0.4
    psw = torch.rand(idx.numel(), device=gpu, generator=g) if weighted else None
    flags = rnd.choice([None, None, pkg.capi.TBE_FLAG_FORCE_STREAM, pkg.capi.TBE_FLAG_NO_STREAM,
                        pkg.capi.TBE_FLAG_NARROW_WORDS, pkg.capi.TBE_FLAG_SERIAL_GROUPS,
                        pkg.capi.TBE_FLAG_NO_XCD_REMAP])
    label = (f"fuzz seed={seed} T={T} types={types} D={dims} pm={pm} out={out_ty} {idx_dtype} "
             f"align={row_alignment} fp8={fp8} B={B} Lmax={Lmax} w={weighted} flags={flags}")
    return m, idx, off.to(idx_dtype), psw, flags, label


@pytest.mark.parametrize("seed", range(240))
def test_random_mixed_modules(pkg, oracle, gpu, seed):
    m, idx, off, psw, flags, label = _case(pkg, gpu, 0xF022 + seed)
    if idx.numel() == 0:
        pytest.skip("no lookups (the op requires at least one index, A:117)")
    _check_module(oracle, m, idx, off, psw, label, flags=flags)


# ----------------------------------------------------------------- block_bucketize

@pytest.mark.parametrize("seed", range(120))
def test_random_bucketize(pkg, oracle, gpu, seed):
    """Random shapes and options of block_bucketize_sparse_features against the oracle:
    my_size on both sides of 64 (LDS and memory counters), rows from empty to several
    512-index chunks, optional total_num_blocks, batch_size_per_feature, position
    lists, weights, sequence, keep_orig_idx, and indices past the blocks (the general
    index map, in the general scatter pass)."""
    import numpy as np
    from _bucketize_cases import Case
    from test_gpu_sparse_ops import _beyond_blocks, _check
    rnd = random.Random(0xB0C4 + seed)
    dtype = rnd.choice([np.int32, np.int64])
    my = rnd.choice([1, 2, 3, 5, 16, 33, 63, 64, 65, 100])
    lo = rnd.choice([0, 0, 4, 100])
    hi = lo + rnd.choice([3, 30, 300, 900])
    case = Case(f"fuzz{seed}", rnd.randint(1, 12), rnd.randint(1, 96), lo, hi, 1, rnd.randint(1, 64), my, dtype)
    tnb = rnd.choice([None, None, "multiple", "rand"])
    pos = rnd.random() < 0.25
    # indices past a feature's blocks (put there on purpose, or by batch_size_per_feature
    # giving a row to a feature with smaller blocks than the one its indices were drawn
    # for) are left out when total_num_blocks is not a multiple of my_size, and the
    # output tail past the kept ones is then unwritten: that case has its own test
    # (test_bucketize_bucket_past_my_size_dropped), so "rand" goes without them here
    bspf = tnb != "rand" and not pos and rnd.random() < 0.25
    mutate = _beyond_blocks(dtype, my) if (tnb != "rand" and not pos and rnd.random() < 0.3) else None
    _check(oracle, gpu, case, seed, weights=rnd.random() < 0.5, bucketize_pos=rnd.random() < 0.5,
           sequence=rnd.random() < 0.5, keep=rnd.random() < 0.3, tnb=tnb, bspf=bspf, pos=pos, mutate=mutate)
