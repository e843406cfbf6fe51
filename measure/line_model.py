"""CPU model of the 128-byte line fetches of the per-bag kernel on configuration 2
(26 INT4 tables x 4M rows of 80 bytes, B = 8192, Poisson(30) bags, Zipf(1.05) rows).

It replays batches drawn from the configuration's distributions (numpy generators:
the same distributions as fbgemm-ascend_amd/workloads.py, not the same random
stream as the bench's device generator) in the per-bag kernel's order:

  * items (table-major bags) are split into 8 contiguous parts, one per XCD;
  * a part's items are interleaved over its waves: 640 resident waves per XCD, and
    the grid holds two rounds of them (1280 waves), wave w taking items w, w + 1280, ...;
    a second-round wave starts when the first-round wave of its slot ends;
  * a wave takes `speed` time units per bag (per-wave speeds drawn uniformly from
    [spread, 1]: 1.0 is lockstep), and reads the rows of a bag in index order
    across that time;

and feeds each XCD's stream of row lines (a 68-byte row at an 80-byte stride spans
one or two lines) through a 4 MiB, 16-way LRU cache (2048 sets, hashed set index).
It counts, per batch:

  compulsory   distinct lines of the batch (any cache, any order)
  per-XCD      sum over XCDs of the distinct lines each XCD touches
  LRU misses   misses of the per-XCD caches for the modelled order

Variants: `interleaved` (the kernel: both rounds interleaved over the whole part),
`halves` (round 1 takes the first half of the part, round 2 the rest), `one-round`
(640 waves per XCD, no second round).  Index lines (4 bytes per lookup) and output
lines are not in the model; the measured L2 -> memory read requests
(TCC_EA0_RDREQ) include the index lines (~0.2 M per call).

    python3 measure/line_model.py [--batches 1] [--spread 1.0 0.8] [--variants interleaved halves]

Needs gcc (it compiles measure/l2sim.c into measure/_build/ on first use) and ~6 GB
of memory; one variant of one batch takes ~20 s.
"""
from __future__ import annotations

import argparse
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
T, B, E, STRIDE, ROW_BYTES, LINE = 26, 8192, 4_000_000, 80, 68, 128
XCDS, WAVES_PER_XCD = 8, 640
SETS, WAYS = 2048, 16


def _lib():
    so = os.path.join(HERE, "_build", "libl2sim.so")
    src = os.path.join(HERE, "l2sim.c")
    if not os.path.exists(so) or os.path.getmtime(so) < os.path.getmtime(src):
        os.makedirs(os.path.dirname(so), exist_ok=True)
        subprocess.run(["gcc", "-O2", "-shared", "-fPIC", src, "-o", so], check=True)
    lib = ctypes.CDLL(so)
    lib.lru_misses.restype = ctypes.c_int64
    lib.lru_misses.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    return lib


def make_batch(seed: int, alpha: float = 1.05):
    """Bag lengths Poisson(30) clipped to [1, 100]; rows Zipf(alpha) by inverse CDF over a
    table's rows, ranks mapped to rows by a permutation fixed per table."""
    rs = np.random.default_rng(seed)
    lengths = np.clip(rs.poisson(30, T * B), 1, 100).astype(np.int64)
    w = np.arange(1, E + 1, dtype=np.float64) ** (-alpha)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    per_table = lengths.reshape(T, B).sum(1)
    idx = []
    for t in range(T):
        perm = np.random.default_rng(1000 + t).permutation(E)
        idx.append(perm[np.minimum(np.searchsorted(cdf, rs.random(per_table[t])), E - 1)])
    offsets = np.zeros(T * B + 1, np.int64)
    np.cumsum(lengths, out=offsets[1:])
    return np.concatenate(idx), offsets


def row_lines(table, rows):
    """First and last 128-byte line of each row (tables laid out back to back)."""
    first = table.astype(np.int64) * (E * STRIDE) + rows * STRIDE
    return first // LINE, (first + ROW_BYTES - 1) // LINE


def lookups(items, offsets):
    """Per lookup of `items` (in item order): the item's position, the lookup's rank
    in its bag, its index position, and each item's bag length."""
    s, e = offsets[items], offsets[items + 1]
    L = e - s
    pos = np.repeat(np.arange(len(items)), L)
    j = np.arange(L.sum()) - np.repeat(np.cumsum(L) - L, L)
    return pos, j, np.repeat(s, L) + j, L


def item_times(n, variant, speed):
    """Start time and duration of each of a part's n items under `variant`."""
    W = WAVES_PER_XCD
    if variant == "one-round":
        wave = np.arange(n) % W
        k = np.arange(n) // W
        return k * speed[wave], speed[wave]
    if variant == "interleaved":
        NW = 2 * W
        wave = np.arange(n) % NW
        k = np.arange(n) // NW
        cnt = np.bincount(wave, minlength=NW)
        start = np.zeros(NW)
        start[W:] = cnt[:W] * speed[:W]  # round-2 wave starts when its slot's round-1 wave ends
        return start[wave] + k * speed[wave], speed[wave]
    if variant == "halves":
        h = n // 2
        w1, k1 = np.arange(h) % W, np.arange(h) // W
        fin = np.bincount(w1, minlength=W) * speed[:W]
        w2, k2 = np.arange(n - h) % W, np.arange(n - h) // W
        t = np.concatenate([k1 * speed[w1], fin[w2] + k2 * speed[W + w2]])
        d = np.concatenate([speed[w1], speed[W + w2]])
        return t, d
    raise ValueError(variant)


def xcd_stream(items, idx, offsets, variant, speed):
    t_item, d_item = item_times(len(items), variant, speed)
    pos, j, lk, L = lookups(items, offsets)
    order = np.argsort(t_item[pos] + d_item[pos] * (j / L[pos]), kind="stable")
    l0, l1 = row_lines((items // B)[pos][order], idx[lk][order])
    two = l1 != l0
    out = np.empty(len(l0) + int(two.sum()), np.uint64)
    start = np.cumsum(1 + two) - (1 + two)
    out[start] = l0
    out[start[two] + 1] = l1[two]
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--batches", type=int, default=1)
    ap.add_argument("--spread", type=float, nargs="+", default=[1.0, 0.8])
    ap.add_argument("--variants", nargs="+", default=["interleaved", "halves", "one-round"])
    args = ap.parse_args()
    lib = _lib()
    I = T * B
    for bi in range(args.batches):
        idx, offsets = make_batch(7919 * bi + 1)
        pos, _, lk, _ = lookups(np.arange(I), offsets)
        l0, l1 = row_lines((np.arange(I) // B)[pos], idx[lk])
        every = np.concatenate([l0, l1[l1 != l0]])
        print(f"batch {bi}: {len(idx)} lookups, {len(every)} row-line touches, "
              f"compulsory {len(np.unique(every))} lines, index lines {len(idx) * 4 // LINE}", flush=True)
        per_xcd = 0
        for x in range(XCDS):
            part = np.arange(I * x // XCDS, I * (x + 1) // XCDS)
            per_xcd += len(np.unique(xcd_stream(part, idx, offsets, "one-round", np.ones(2 * WAVES_PER_XCD))))
        print(f"  per-XCD distinct lines (sum over XCDs) {per_xcd}", flush=True)
        rng = np.random.default_rng(5)
        for variant in args.variants:
            for spread in args.spread:
                misses = 0
                for x in range(XCDS):
                    part = np.arange(I * x // XCDS, I * (x + 1) // XCDS)
                    speed = rng.uniform(spread, 1.0, 2 * WAVES_PER_XCD) if spread < 1.0 else np.ones(2 * WAVES_PER_XCD)
                    st = np.ascontiguousarray(xcd_stream(part, idx, offsets, variant, speed))
                    misses += lib.lru_misses(st.ctypes.data, len(st), SETS, WAYS, 1)
                print(f"  {variant:12s} speed spread [{spread:.2f}, 1]: LRU misses {misses}", flush=True)


if __name__ == "__main__":
    main()
