"""Input generators for block_bucketize_sparse_features tests, after the reference's
perf-case generator (reference bench/sparse/block_bucketize_sparse_features_test/
block_bucketize_sparse_features_perf_cases.py:44-118, 185-230: the same case list,
lengths in [min, max], block sizes in a range (>= 1), indices in [0, block_size *
my_size) per feature, total_num_blocks "rand"/"multiple", batch_size_per_feature,
monotone per-feature bucketize positions)."""
from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Case:
    name: str
    num_features: int
    batch_size: int
    min_length: int
    max_length: int
    block_lo: int
    block_hi: int
    my_size: int
    dtype: type


CASES = (
    Case("i32_pow2_basic", 4, 64, 0, 16, 8, 16, 2, np.int32),
    Case("i32_nonpow2_rank6", 24, 32, 4, 20, 16, 32, 6, np.int32),
    Case("i32_mysize1", 2, 16, 0, 4, 2, 4, 1, np.int32),
    Case("i32_batch1_pow2", 8, 1, 4, 32, 8, 16, 4, np.int32),
    Case("i32_batch1_nonpow2", 12, 1, 2, 16, 4, 8, 3, np.int32),
    Case("i32_many_features", 96, 128, 32, 128, 32, 64, 8, np.int32),
    Case("i32_single_feature", 1, 4096, 0, 64, 16, 64, 4, np.int32),
    Case("i32_quickdiv_guaranteed", 8, 64, 4, 16, 4, 8, 3, np.int32),
    Case("i64_pow2_basic", 16, 64, 2, 48, 8, 24, 8, np.int64),
    Case("i64_nonpow2_rank5", 5, 180, 0, 128, 16, 24, 5, np.int64),
    Case("i64_nonpow2_rank12", 48, 32, 8, 40, 16, 24, 12, np.int64),
    Case("i64_batch1_pow2", 16, 1, 8, 32, 16, 32, 8, np.int64),
    Case("i64_batch1_nonpow2", 6, 1, 4, 24, 8, 16, 5, np.int64),
    Case("i64_rank64", 4, 4096, 32, 256, 64, 128, 64, np.int64),
    Case("i64_ultra_batch", 8, 4096, 0, 64, 16, 32, 4, np.int64),
    Case("i64_stress", 16, 8192, 128, 512, 128, 256, 16, np.int64),
    Case("i64_long_seq", 2, 512, 64, 128, 64, 128, 2, np.int64),
)


def gen_case(case: Case, seed: int, weights: bool = False):
    rng = np.random.default_rng(seed)
    dt = case.dtype
    F, B = case.num_features, case.batch_size
    lengths = rng.integers(case.min_length, case.max_length + 1, F * B).astype(dt)
    block_sizes = np.maximum(rng.integers(case.block_lo, case.block_hi + 1, F), 1).astype(dt)
    parts = []
    for f in range(F):
        limit = max(int(block_sizes[f]) * case.my_size, 1)
        n = int(lengths[f * B:(f + 1) * B].sum())
        parts.append(rng.integers(0, limit, n))
    indices = (np.concatenate(parts) if parts else np.zeros(0)).astype(dt)
    w = rng.uniform(-1, 1, indices.size).astype(np.float32) if weights else None
    return lengths, indices, block_sizes, w


def gen_total_num_blocks(block_sizes, my_size: int, kind: str, seed: int):
    rng = np.random.default_rng(seed)
    F = block_sizes.size
    if kind == "rand":  # in [my, 2*my], nudged off multiples of my
        v = rng.integers(my_size, max(2 * my_size, my_size + 1) + 1, F)
        if my_size > 1:
            v = np.where(v % my_size == 0, np.minimum(v + 1, max(2 * my_size, my_size + 1)), v)
    else:  # "multiple": my * [1, 20]
        v = rng.integers(1, 21, F) * my_size
    return v.astype(block_sizes.dtype)


def gen_batch_size_per_feature(F: int, batch_size: int, dtype, seed: int):
    rng = np.random.default_rng(seed)
    target = batch_size * F
    low, high = max(1, batch_size // 2), max(max(1, batch_size // 2) + 1, batch_size * 2)
    v = rng.integers(low, high + 1, F).astype(np.float64)
    v = np.maximum(np.round(v * (target / v.sum())), 1).astype(np.int64)
    i = 0
    while v.sum() != target:
        step = 1 if v.sum() < target else -1
        if v[i] + step >= 1:
            v[i] += step
        i = (i + 1) % F
    return v.astype(dtype), int(v.max())


def gen_bucketize_pos(block_sizes, my_size: int, seed: int):
    rng = np.random.default_rng(seed)
    out = []
    for b in block_sizes:
        steps = rng.integers(1, max(int(b), 1) + 1, my_size)
        out.append(np.concatenate([[0], np.cumsum(steps)]).astype(block_sizes.dtype))
    return out
