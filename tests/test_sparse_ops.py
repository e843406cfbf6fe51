"""block_bucketize_sparse_features: the CPU oracle (oracle/tbe_oracle.c) pinned by a
hand-derived example and by an independent numpy formulation of the bucket rule
(a stable sort by (bucket, row) instead of the oracle's running write cursors),
with numpy.searchsorted for the bucketize-position lists; plus host checks of the
op registration and the C ABI (no GPU needed)."""
import zlib

import numpy as np
import pytest
import torch

from _bucketize_cases import CASES, gen_batch_size_per_feature, gen_bucketize_pos, gen_case, gen_total_num_blocks


def test_hand_example(oracle):
    # 4 features x 2 samples; block sizes 5, 15, 10, 20; my_size 2 (no total_num_blocks: an
    # index below 2*blk goes to bucket idx // blk as idx % blk).  Rows: r1 (f0) [3, 4] ->
    # b0 (3, 4); r2 (f1) [15] -> b1 (0); r3 (f1) [11, 28, 29] -> b0 (11), b1 (13, 14);
    # r4 (f2) [1, 10] -> b0 (1), b1 (0); r5 (f2) [11, 12, 13] -> b1 (1, 2, 3);
    # r6 (f3) [11, 22, 20] -> b0 (11), b1 (2, 0); r7 (f3) [20] -> b1 (0).
    lengths = np.array([0, 2, 1, 3, 2, 3, 3, 1], np.int32)
    indices = np.array([3, 4, 15, 11, 28, 29, 1, 10, 11, 12, 13, 11, 22, 20, 20], np.int32)
    nl, ni, nw, npos, unb = oracle.block_bucketize_sparse_features(
        lengths, indices, True, True, np.array([5, 15, 10, 20], np.int32), 2)
    assert nl.tolist() == [0, 2, 0, 1, 1, 0, 1, 0, 0, 0, 1, 2, 1, 3, 2, 1]
    assert ni.tolist() == [3, 4, 11, 1, 11, 0, 13, 14, 0, 1, 2, 3, 2, 0, 0]
    assert unb.tolist() == [0, 1, 5, 2, 6, 7, 3, 8, 9, 10, 11, 4, 12, 13, 14]
    assert npos.tolist() == [0, 1, 0, 0, 0, 0, 1, 2, 1, 0, 1, 2, 1, 2, 0]
    assert nw is None


def numpy_bucketize(lengths, indices, block_sizes, my, weights=None, bspf=None, tnb=None, pos=None, keep=False):
    """Vectorised restatement: per-index (bucket, new index) with numpy arithmetic, then a
    stable argsort by bucket * L + row gives every output position."""
    L, F = lengths.size, block_sizes.size
    u = indices.astype(np.uint64) & (np.uint64(0xFFFFFFFF) if indices.itemsize == 4 else np.uint64(~0 & (2**64 - 1)))
    rows = np.repeat(np.arange(L), lengths.astype(np.int64))
    if bspf is None:
        feat = rows // (L // F)
    else:
        bso = np.concatenate([[0], np.cumsum(bspf.astype(np.int64))])
        feat = np.searchsorted(bso, rows, side="right") - 1
    blk = block_sizes.astype(np.int64)[feat].astype(np.uint64)
    gb = (np.full(F, my, np.int64) if tnb is None else np.where(tnb > 0, tnb, my)).astype(np.int64)
    lbk = np.ones(F, np.int64) if tnb is None else np.maximum(gb // my, 1)
    gbi, lbi = gb[feat].astype(np.uint64), lbk[feat].astype(np.uint64)
    bucket = np.empty(u.size, np.int64)
    new = np.empty(u.size, np.int64)
    if pos is None:
        inr = (blk != 0) & (u < blk * gbi)
        lsz = np.where(inr, blk * lbi, np.uint64(1))
        bucket = np.where(inr, u // lsz, (u % gbi) // lbi).astype(np.int64)
        new = np.where(inr, u % lsz, u // gbi).astype(np.int64)
    else:
        for k in range(u.size):
            p = pos[feat[k]].astype(np.int64)
            lb = int(np.searchsorted(p, int(u[k]), side="right")) - 1
            inb = 0 <= lb < my
            bucket[k] = lb if inb else int(u[k]) % my
            new[k] = int(u[k]) - int(p[lb]) if inb else int(u[k]) // my
    if keep:
        new = u.astype(np.int64)
    order = np.argsort(bucket * L + rows, kind="stable")
    new_lengths = np.bincount(bucket * L + rows, minlength=my * L)
    unb = np.empty(u.size, np.int64)
    unb[order] = np.arange(u.size)
    starts = np.concatenate([[0], np.cumsum(lengths.astype(np.int64))])[:-1]
    posn = np.arange(u.size) - starts[rows]
    return (new_lengths, new[order], None if weights is None else weights[order], posn[order], unb)


@pytest.mark.parametrize("case", [c for c in CASES if c.name not in ("i64_stress", "i64_rank64", "i64_ultra_batch")],
                         ids=lambda c: c.name)
@pytest.mark.parametrize("variant", ["plain", "keep", "tnb_multiple", "bspf", "pos"])
def test_oracle_matches_numpy_formulation(oracle, case, variant):
    seed = zlib.crc32(f"{case.name}:{variant}".encode()) % 100000
    lengths, indices, block_sizes, w = gen_case(case, seed, weights=True)
    kw = {}
    if variant == "keep":
        kw["keep_orig_idx"] = True
    if variant == "tnb_multiple":
        kw["total_num_blocks"] = gen_total_num_blocks(block_sizes, case.my_size, "multiple", seed)
    if variant == "bspf":
        if case.batch_size <= 1:
            pytest.skip("batch_size_per_feature needs batch_size > 1")
        kw["batch_size_per_feature"], _ = gen_batch_size_per_feature(case.num_features, case.batch_size,
                                                                     lengths.dtype, seed)
    if variant == "pos":
        kw["block_bucketize_pos"] = gen_bucketize_pos(block_sizes, case.my_size, seed)
    got = oracle.block_bucketize_sparse_features(lengths, indices, True, True, block_sizes, case.my_size, weights=w,
                                                 **kw)
    want = numpy_bucketize(lengths, indices, block_sizes, case.my_size, weights=w,
                           bspf=kw.get("batch_size_per_feature"), tnb=kw.get("total_num_blocks"),
                           pos=kw.get("block_bucketize_pos"), keep=kw.get("keep_orig_idx", False))
    for g, e in zip(got, want):
        assert np.array_equal(np.asarray(g, np.float64), np.asarray(e, np.float64))


def test_oracle_rand_total_num_blocks_sums(oracle):
    # total_num_blocks off multiples of my_size: every index still lands in [0, my_size)
    c = CASES[1]
    lengths, indices, block_sizes, _ = gen_case(c, 5)
    tnb = gen_total_num_blocks(block_sizes, c.my_size, "rand", 5)
    nl, ni, *_ = oracle.block_bucketize_sparse_features(lengths, indices, False, False, block_sizes, c.my_size,
                                                        total_num_blocks=tnb)
    assert int(nl.sum()) == indices.size


def test_schemas_registered(pkg):
    for qual in ("fbgemm::block_bucketize_sparse_features", "mxrec::block_bucketize_sparse_features"):
        assert torch._C._dispatch_find_schema_or_throw(qual, "") is not None


def test_c_abi_rejects_bad_args_without_gpu(pkg):
    import ctypes
    c = pkg.capi
    a = c.TbeBlockBucketizeArgs()
    a.my_size, a.index_size, a.offset_size, a.num_features, a.lengths_size = 0, 4, 4, 1, 4
    assert c.lib().tbe_block_bucketize_sparse_features(ctypes.byref(a), None) != 0
    assert "my_size must be positive" in c.last_error()
    a.my_size, a.lengths_size, a.num_features = 2, 5, 2
    assert c.lib().tbe_block_bucketize_sparse_features(ctypes.byref(a), None) != 0
    assert "divisible" in c.last_error()
    a.lengths_size = 4
    assert c.lib().tbe_block_bucketize_sparse_features(ctypes.byref(a), None) != 0
    assert "workspace" in c.last_error()
    assert c.lib().tbe_block_bucketize_workspace_bytes(2, 4, 4) > 0
