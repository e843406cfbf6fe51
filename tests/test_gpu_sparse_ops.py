"""GPU parity of block_bucketize_sparse_features: the HIP kernels (through
torch.ops.fbgemm / torch.ops.mxrec and through the C ABI) against the CPU oracle,
exactly (integer outputs and copied weights), on the reference test's case list and
option grid (reference bench/sparse/block_bucketize_sparse_features_test/
test_block_bucketize_sparse_features_perf.py:96-198: weights x bucketize_pos x
sequence x keep_orig_idx, total_num_blocks rand/multiple, batch_size_per_feature with
max_B, block_bucketize_pos).  Outputs are compared in full order: both sides keep
row order inside every segment."""
import itertools
import zlib

import numpy as np
import pytest
import torch

from _bucketize_cases import CASES, gen_batch_size_per_feature, gen_bucketize_pos, gen_case, gen_total_num_blocks

pytestmark = pytest.mark.gpu


def _check(oracle, gpu, case, seed, *, weights=False, bucketize_pos=False, sequence=False, keep=False, tnb=None,
           bspf=False, pos=False, via="fbgemm", mutate=None):
    lengths, indices, block_sizes, w = gen_case(case, seed, weights)
    if mutate is not None:
        indices = mutate(indices)
    kw = {}
    if tnb:
        kw["total_num_blocks"] = gen_total_num_blocks(block_sizes, case.my_size, tnb, seed)
    max_B = -1
    if bspf:
        kw["batch_size_per_feature"], max_B = gen_batch_size_per_feature(case.num_features, case.batch_size,
                                                                         lengths.dtype, seed)
    if pos:
        kw["block_bucketize_pos"] = gen_bucketize_pos(block_sizes, case.my_size, seed)
    print(f"[gpu] block_bucketize {case.name} seed={seed} w={weights} pos={bucketize_pos} seq={sequence} "
          f"keep={keep} tnb={tnb} bspf={bspf} poslist={pos} via={via} N={indices.size}", flush=True)
    want = oracle.block_bucketize_sparse_features(lengths, indices, bucketize_pos, sequence, block_sizes,
                                                  case.my_size, weights=w, keep_orig_idx=keep, **kw)
    d = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    if via == "capi":
        from fbgemm_ascend_amd import capi
        got, _ = capi.block_bucketize_sparse_features(
            d(lengths), d(indices), bucketize_pos, sequence, d(block_sizes), case.my_size, weights=d(w),
            batch_size_per_feature=d(kw.get("batch_size_per_feature")),
            block_bucketize_pos=None if not pos else [d(p) for p in kw["block_bucketize_pos"]],
            keep_orig_idx=keep, total_num_blocks=d(kw.get("total_num_blocks")))
    else:
        op = getattr(torch.ops, via).block_bucketize_sparse_features
        got = op(d(lengths), d(indices), bucketize_pos, sequence, d(block_sizes), case.my_size, weights=d(w),
                 batch_size_per_feature=d(kw.get("batch_size_per_feature")), max_B=max_B,
                 block_bucketize_pos=None if not pos else [d(p) for p in kw["block_bucketize_pos"]],
                 keep_orig_idx=keep, total_num_blocks=d(kw.get("total_num_blocks")))
        torch.cuda.synchronize()
    names = ["new_lengths", "new_indices", "new_weights", "new_pos", "unbucketize_permute"]
    for name, g, e in zip(names, got, want):
        if e is None:
            assert g is None, name
            continue
        g = g.cpu().numpy()
        assert g.dtype == e.dtype, name
        assert np.array_equal(g, e), f"{name} differs"


OPTIONS = list(itertools.product([False, True], repeat=4))  # weights, bucketize_pos, sequence, keep


@pytest.mark.parametrize("case", CASES, ids=lambda c: c.name)
@pytest.mark.parametrize("opt", [OPTIONS[0], OPTIONS[5], OPTIONS[10], OPTIONS[15]],
                         ids=lambda o: "w%d_p%d_s%d_k%d" % o)
def test_bucketize_options(pkg, oracle, gpu, case, opt):
    w, bp, seq, keep = opt
    _check(oracle, gpu, case, zlib.crc32(case.name.encode()) % 10000, weights=w, bucketize_pos=bp, sequence=seq,
           keep=keep)


@pytest.mark.parametrize("opt", OPTIONS, ids=lambda o: "w%d_p%d_s%d_k%d" % o)
def test_bucketize_full_option_grid(pkg, oracle, gpu, opt):
    w, bp, seq, keep = opt
    _check(oracle, gpu, CASES[9], 77, weights=w, bucketize_pos=bp, sequence=seq, keep=keep)


@pytest.mark.parametrize("case", CASES, ids=lambda c: c.name)
@pytest.mark.parametrize("tnb", ["rand", "multiple"])
def test_bucketize_total_num_blocks(pkg, oracle, gpu, case, tnb):
    _check(oracle, gpu, case, 11, tnb=tnb)


@pytest.mark.parametrize("case", [c for c in CASES if c.batch_size > 1], ids=lambda c: c.name)
def test_bucketize_batch_size_per_feature(pkg, oracle, gpu, case):
    _check(oracle, gpu, case, 13, bspf=True, sequence=True)


@pytest.mark.parametrize("case", CASES, ids=lambda c: c.name)
def test_bucketize_pos_lists(pkg, oracle, gpu, case):
    _check(oracle, gpu, case, 17, pos=True, sequence=True, bucketize_pos=True)


@pytest.mark.parametrize("via", ["mxrec", "capi"])
def test_bucketize_entry_points(pkg, oracle, gpu, via):
    _check(oracle, gpu, CASES[1], 19, weights=True, bucketize_pos=True, sequence=True, via=via)


def test_bucketize_mixed_dtypes(pkg, oracle, gpu):
    # int64 lengths with int32 indices and the reverse
    lengths = np.array([3, 0, 2, 4], np.int64)
    indices = np.array([1, 9, 17, 4, 30, 2, 3, 25, 8], np.int32)
    bs = np.array([4, 8], np.int32)
    for L_, I_ in ((lengths, indices), (lengths.astype(np.int32), indices.astype(np.int64))):
        want = oracle.block_bucketize_sparse_features(L_, I_, True, True, bs.astype(I_.dtype), 3)
        got = torch.ops.fbgemm.block_bucketize_sparse_features(
            torch.from_numpy(L_).to(gpu), torch.from_numpy(I_).to(gpu), True, True,
            torch.from_numpy(bs.astype(I_.dtype)).to(gpu), 3)
        for g, e in zip(got, want):
            if e is not None:
                assert np.array_equal(g.cpu().numpy(), e)


def test_bucketize_empty_inputs(pkg, oracle, gpu):
    lengths = np.zeros(6, np.int32)
    indices = np.zeros(0, np.int32)
    got = torch.ops.fbgemm.block_bucketize_sparse_features(
        torch.from_numpy(lengths).to(gpu), torch.from_numpy(indices).to(gpu), False, True,
        torch.tensor([3, 5], dtype=torch.int32, device=gpu), 4)
    assert got[0].cpu().tolist() == [0] * 24 and got[1].numel() == 0 and got[4].numel() == 0


@pytest.mark.parametrize("my_size", [63, 64, 65, 200])
@pytest.mark.parametrize("sequence", [False, True])
def test_bucketize_my_size_paths(pkg, oracle, gpu, my_size, sequence):
    # my_size <= 64 keeps counters in registers, above that in memory with atomics
    from _bucketize_cases import Case
    case = Case(f"my{my_size}", 6, 50, 0, 150, 3, 9, my_size, np.int64)
    _check(oracle, gpu, case, my_size, weights=True, bucketize_pos=True, sequence=sequence)
    _check(oracle, gpu, case, my_size + 1, tnb="rand", sequence=sequence)


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("my_size", [3, 16, 40])
def test_bucketize_rows_over_several_chunks(pkg, oracle, gpu, dtype, my_size):
    # rows of 400-1800 indices span several 512-index chunks of the scatter
    # phase: the per-bucket cursors carry over from one chunk to the next
    from _bucketize_cases import Case
    case = Case(f"long_rows_my{my_size}", 4, 12, 400, 1800, 8, 40, my_size, dtype)
    _check(oracle, gpu, case, 5 + my_size, weights=True, sequence=True)
    _check(oracle, gpu, case, 6 + my_size, bucketize_pos=True, sequence=True, keep=True)
    _check(oracle, gpu, case, 7 + my_size, weights=True, pos=True, sequence=True)


def _beyond_blocks(dtype, my_size):
    """About one index in ten moved at or above block_size * total_num_blocks
    (int64: some at or above 2^32), so steps mix the multiply-shift division
    with the general path."""
    hi = np.iinfo(dtype).max

    def mutate(ix):
        rng = np.random.default_rng(my_size)
        ix = ix.copy()
        sel = rng.random(ix.size) < 0.1
        big = rng.integers(0, hi, ix.size, dtype=np.int64, endpoint=False)
        if dtype == np.int64:
            big = np.where(rng.random(ix.size) < 0.5, big % (1 << 34), big)
        ix[sel] = big[sel].astype(dtype)
        return ix

    return mutate


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("my_size", [5, 16, 100])
@pytest.mark.parametrize("tnb", [None, "multiple"])
def test_bucketize_indices_beyond_blocks(pkg, oracle, gpu, dtype, my_size, tnb):
    # total_num_blocks absent or a multiple of my_size: every bucket of an index
    # at or above the blocks, (idx % gb) / (gb / my_size), is below my_size
    from _bucketize_cases import Case
    case = Case(f"beyond_my{my_size}", 5, 40, 0, 200, 8, 40, my_size, dtype)
    mutate = _beyond_blocks(dtype, my_size)
    _check(oracle, gpu, case, 31, tnb=tnb, sequence=True, mutate=mutate)
    _check(oracle, gpu, case, 32, tnb=tnb, weights=True, keep=True, mutate=mutate)


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("my_size", [16, 40])
@pytest.mark.parametrize("at", [5, 600, 1500])
def test_bucketize_high_index_in_one_chunk(pkg, oracle, gpu, dtype, my_size, at):
    # rows of 400-1800 indices, every third one with a single index at or above the
    # blocks at position `at`: the fast scatter pass writes the chunks before it,
    # gives the row up at that chunk, and the general pass rewrites the whole row
    from _bucketize_cases import Case
    case = Case(f"high_at{at}_my{my_size}", 4, 12, 400, 1800, 8, 40, my_size, dtype)
    for seed, kw in ((51, dict(weights=True, sequence=True)), (52, dict(sequence=True, keep=True)),
                     (53, dict(weights=True, bucketize_pos=True))):
        lengths = gen_case(case, seed, kw.get("weights", False))[0]
        off = np.concatenate([[0], np.cumsum(lengths)])

        def mutate(ix, lengths=lengths, off=off):
            ix = ix.copy()
            hi = np.iinfo(ix.dtype).max
            for r in range(0, lengths.size, 3):
                if lengths[r] > at:
                    ix[off[r] + at] = hi - r
            return ix

        _check(oracle, gpu, case, seed, mutate=mutate, **kw)


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("my_size", [5, 100])
def test_bucketize_bucket_past_my_size_dropped(pkg, oracle, gpu, dtype, my_size):
    # total_num_blocks not a multiple of my_size and indices at or above the
    # blocks give buckets >= my_size, for which the reference adds past the end
    # of new_lengths (BK:455, undefined there).  Here such indices are left out:
    # new_lengths and the filled prefix of new_indices / new_weights match the
    # oracle, which leaves them out too; the tail past sum(new_lengths) is
    # unwritten, as in the reference (at::empty, BA:156-157).
    from _bucketize_cases import Case
    case = Case(f"drop_my{my_size}", 5, 40, 0, 200, 8, 40, my_size, dtype)
    lengths, indices, block_sizes, w = gen_case(case, 33, True)
    indices = _beyond_blocks(dtype, my_size)(indices)
    tnb = gen_total_num_blocks(block_sizes, my_size, "rand", 33)
    want = oracle.block_bucketize_sparse_features(lengths, indices, False, False, block_sizes, my_size, weights=w,
                                                  total_num_blocks=tnb)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    got = torch.ops.fbgemm.block_bucketize_sparse_features(d(lengths), d(indices), False, False, d(block_sizes),
                                                           my_size, weights=d(w), total_num_blocks=d(tnb))
    total = int(want[0].sum())
    assert total < indices.size, "the case must drop some indices"
    assert np.array_equal(got[0].cpu().numpy(), want[0])
    assert np.array_equal(got[1].cpu().numpy()[:total], want[1][:total])
    assert np.array_equal(got[2].cpu().numpy()[:total], want[2][:total])


@pytest.mark.parametrize("my_size", [64, 100])
def test_bucketize_many_segments(pkg, oracle, gpu, my_size):
    # my_size * rows above 2^21 segments: the device scan of new_lengths takes
    # more than one pass over its tile sums
    from _bucketize_cases import Case
    case = Case(f"segments_my{my_size}", 8, 5000, 0, 3, 4, 8, my_size, np.int64)
    _check(oracle, gpu, case, 41, weights=True, sequence=True)
