"""Synthetic workloads of the five benchmark configurations (the op's inputs, built
directly in device memory with torch generators).

  0  1 x 100k rows, D128 INT8, B512, L=20 fixed, uniform int64 indices, SUM, fp32 out
  1  26 x 1M, D128 INT8, B2048, L~Poisson(30) clip [1,100], Zipf(1.05), int32, SUM, fp16 out
  2  26 x 4M, D128 INT4, B8192, L~Poisson(30) clip [1,100], Zipf(1.05), int32, SUM, fp16 out
  3  64 tables, rows logU[100k,5M], D in {32,64,128,256}, {FP16,INT8,INT4,INT2} @ {.1,.3,.4,.2},
     B16384, L~U[0,64] (empty bags), fp32 per-sample weights U(0,1), Zipf(1.1), int32, MEAN, fp32 out
  4  200 x 10M, D128 INT4, B32768, L~Poisson(40) clip [1,128], Zipf(1.2) + 5% uniform, int64,
     SUM, fp16 out (~160 GB of padded rows)

Zipf ranks are drawn by inverse CDF over the table's rows and mapped to rows by a
random permutation per table, so hot rows are scattered over the table.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Dict, List, Optional

import numpy as np
import torch

from .sparse_types import PoolingMode, SparseType, unpadded_row_bytes
from .tbe_module import IntNBitTableBatchedEmbeddingBagsCodegen

HBM_PEAK_BYTES_PER_S = 8.0e12


@dataclasses.dataclass
class ConfigSpec:
    cid: int
    tables: List[tuple]          # (E, D, SparseType)
    B: int
    bag_len: str                 # "fixed:L", "poisson:mean:lo:hi", "uniform:lo:hi"
    zipf_alpha: Optional[float]  # None = uniform indices
    uniform_tail: float
    index_dtype: torch.dtype
    pooling: PoolingMode
    out_ty: SparseType
    weighted: bool
    description: str


def config_spec(cid: int, scale_rows: float = 1.0) -> ConfigSpec:
    """Spec of configuration `cid`; scale_rows shrinks table heights (for CPU tests)."""
    def rows(n):
        return max(16, int(n * scale_rows))

    if cid == 0:
        return ConfigSpec(0, [(rows(100_000), 128, SparseType.INT8)], 512, "fixed:20", None, 0.0,
                          torch.int64, PoolingMode.SUM, SparseType.FP32, False,
                          "1x100k D128 INT8 B512 L20 SUM fp32")
    if cid == 1:
        return ConfigSpec(1, [(rows(1_000_000), 128, SparseType.INT8)] * 26, 2048,
                          "poisson:30:1:100", 1.05, 0.0, torch.int32, PoolingMode.SUM,
                          SparseType.FP16, False, "26x1M D128 INT8 B2048 Poisson30 Zipf1.05 SUM fp16")
    if cid == 2:
        return ConfigSpec(2, [(rows(4_000_000), 128, SparseType.INT4)] * 26, 8192,
                          "poisson:30:1:100", 1.05, 0.0, torch.int32, PoolingMode.SUM,
                          SparseType.FP16, False, "26x4M D128 INT4 B8192 Poisson30 Zipf1.05 SUM fp16")
    if cid == 3:
        rs = np.random.RandomState(0x7BE0 + 3)
        tys = [SparseType.FP16, SparseType.INT8, SparseType.INT4, SparseType.INT2]
        tabs = []
        for _ in range(64):
            E = int(math.exp(rs.uniform(math.log(100_000), math.log(5_000_000))))
            D = int(rs.choice([32, 64, 128, 256]))
            ty = tys[int(rs.choice(4, p=[0.1, 0.3, 0.4, 0.2]))]
            tabs.append((rows(E), D, ty))
        return ConfigSpec(3, tabs, 16384, "uniform:0:64", 1.1, 0.0, torch.int32, PoolingMode.MEAN,
                          SparseType.FP32, True, "64 mixed tables B16384 U[0,64] Zipf1.1 psw MEAN fp32")
    if cid == 4:
        return ConfigSpec(4, [(rows(10_000_000), 128, SparseType.INT4)] * 200, 32768,
                          "poisson:40:1:128", 1.2, 0.05, torch.int64, PoolingMode.SUM,
                          SparseType.FP16, False, "200x10M D128 INT4 B32768 Poisson40 Zipf1.2+5% SUM fp16")
    raise ValueError(f"unknown config {cid}")


def _bag_lengths(spec: ConfigSpec, T: int, g: torch.Generator, device) -> torch.Tensor:
    kind, *a = spec.bag_len.split(":")
    n = T * spec.B
    if kind == "fixed":
        return torch.full((n,), int(a[0]), dtype=torch.int64, device=device)
    if kind == "poisson":
        mean, lo, hi = float(a[0]), int(a[1]), int(a[2])
        lam = torch.full((n,), mean, dtype=torch.float32, device=device)
        return torch.poisson(lam, generator=g).to(torch.int64).clamp_(lo, hi)
    if kind == "uniform":
        lo, hi = int(a[0]), int(a[1])
        return torch.randint(lo, hi + 1, (n,), dtype=torch.int64, device=device, generator=g)
    raise ValueError(spec.bag_len)


_cdf_cache: Dict[tuple, torch.Tensor] = {}


def _zipf_cdf(n: int, alpha: float, device) -> torch.Tensor:
    key = (n, alpha, str(device))
    c = _cdf_cache.get(key)
    if c is None:
        w = torch.arange(1, n + 1, dtype=torch.float64, device=device).pow_(-alpha)
        c = torch.cumsum(w, 0)
        c /= c[-1].clone()
        _cdf_cache.clear()  # keep at most one (large) table
        _cdf_cache[key] = c
    return c


def _table_perm(n_rows: int, perm_seed: int, device) -> torch.Tensor:
    """Rank -> row map of one table: fixed by the table's seed, so every batch drawn
    from the table sees the same hot rows."""
    g = torch.Generator(device=device)
    g.manual_seed(perm_seed)
    return torch.randperm(n_rows, device=device, generator=g)


def sample_rows(n_rows: int, count: int, alpha: Optional[float], tail: float,
                g: torch.Generator, device, perm_seed: int = 0) -> torch.Tensor:
    """`count` row ids of one table: Zipf(alpha) ranks scattered by the table's fixed
    permutation (seeded by `perm_seed`, with a `tail` fraction drawn uniformly), or
    uniform when alpha is None."""
    if count == 0:
        return torch.empty(0, dtype=torch.int64, device=device)
    if alpha is None:
        return torch.randint(0, n_rows, (count,), dtype=torch.int64, device=device, generator=g)
    u = torch.rand(count, dtype=torch.float64, device=device, generator=g)
    ranks = torch.searchsorted(_zipf_cdf(n_rows, alpha, device), u).clamp_(max=n_rows - 1)
    rows = _table_perm(n_rows, perm_seed, device)[ranks]
    if tail > 0:
        pick = torch.rand(count, device=device, generator=g) < tail
        uni = torch.randint(0, n_rows, (count,), dtype=torch.int64, device=device, generator=g)
        rows = torch.where(pick, uni, rows)
    return rows


@dataclasses.dataclass
class Batch:
    """One batch of the op's sparse inputs."""
    indices: torch.Tensor
    offsets: torch.Tensor
    per_sample_weights: Optional[torch.Tensor]
    lengths: torch.Tensor          # int64 [T*B]


@dataclasses.dataclass
class Workload:
    spec: ConfigSpec
    module: IntNBitTableBatchedEmbeddingBagsCodegen
    batches: List[Batch]           # batch 0 first; all drawn from the same distributions

    @property
    def indices(self) -> torch.Tensor:
        return self.batches[0].indices

    @property
    def offsets(self) -> torch.Tensor:
        return self.batches[0].offsets

    @property
    def per_sample_weights(self) -> Optional[torch.Tensor]:
        return self.batches[0].per_sample_weights

    @property
    def lengths(self) -> torch.Tensor:
        return self.batches[0].lengths

    def num_indices_of(self, i: int = 0) -> int:
        return int(self.batches[i].indices.numel())

    @property
    def num_indices(self) -> int:
        return self.num_indices_of(0)

    @property
    def num_bags(self) -> int:
        return int(self.offsets.numel() - 1)

    def algorithmic_bytes(self, i: int = 0) -> int:
        """Bytes one call on batch i must move at minimum: every lookup's unpadded row,
        the indices, offsets, per-sample weights and the output."""
        bt = self.batches[i]
        T = len(self.module.specs)
        per_table = bt.lengths.view(T, -1).sum(dim=1).cpu().tolist()
        rows = sum(int(c) * unpadded_row_bytes(ty, D)
                   for c, (_, D, ty) in zip(per_table, self.module.specs))
        isz = bt.indices.element_size()
        out_sz = {0: 4, 1: 2, 5: 2}[self.module.output_dtype]
        b = rows + bt.indices.numel() * isz + bt.offsets.numel() * isz
        if bt.per_sample_weights is not None:
            b += 4 * bt.indices.numel()
        b += self.spec.B * self.module.total_D * out_sz
        return b

    def run(self, i: int = 0) -> torch.Tensor:
        bt = self.batches[i]
        return self.module(bt.indices, bt.offsets, bt.per_sample_weights)


def make_batch(spec: ConfigSpec, seed: int, device) -> Batch:
    """Bag lengths, indices (and weights) of one batch; table t's Zipf permutation is
    seeded by (config, t) alone, so batches of one config share their hot rows."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    T = len(spec.tables)
    lengths = _bag_lengths(spec, T, g, device)
    per_table = lengths.view(T, spec.B).sum(dim=1).cpu().tolist()
    parts = [sample_rows(E, int(c), spec.zipf_alpha, spec.uniform_tail, g, device,
                         perm_seed=(0x7BE0 + spec.cid) * 1000 + t)
             for t, ((E, _, _), c) in enumerate(zip(spec.tables, per_table))]
    indices = torch.cat(parts).to(spec.index_dtype)
    offsets = torch.zeros(T * spec.B + 1, dtype=torch.int64, device=device)
    torch.cumsum(lengths, 0, out=offsets[1:])
    offsets = offsets.to(spec.index_dtype)
    psw = (torch.rand(indices.numel(), device=device, generator=g) if spec.weighted else None)
    return Batch(indices, offsets, psw, lengths)


def mean_bag_len(rule: str) -> float:
    """Mean bag length of a bag-length rule (the Poisson mean, unclipped)."""
    kind, *a = rule.split(":")
    if kind in ("fixed", "poisson"):
        return float(a[0])
    if kind == "uniform":
        return (float(a[0]) + float(a[1])) / 2
    raise ValueError(rule)


def make_workload(cid: int, device="cuda", seed: Optional[int] = None, scale_rows: float = 1.0,
                  batch: Optional[int] = None, table_limit: Optional[int] = None,
                  num_batches: int = 1, bag_len: Optional[str] = None) -> Workload:
    """Tables of configuration `cid` (random weights) and `num_batches` batches of
    indices drawn from the configuration's distributions (distinct seeds).  bag_len
    replaces the bag-length rule and scales the batch so the mean number of lookups
    per call stays the configuration's."""
    spec = config_spec(cid, scale_rows)
    if bag_len is not None:
        B = max(1, round(spec.B * mean_bag_len(spec.bag_len) / mean_bag_len(bag_len)))
        spec = dataclasses.replace(spec, bag_len=bag_len, B=B)
    if batch is not None:
        spec = dataclasses.replace(spec, B=batch)
    if table_limit is not None:
        spec = dataclasses.replace(spec, tables=spec.tables[:table_limit])
    seed = 0x7BE0 + cid if seed is None else seed
    device = torch.device(device)
    mod = IntNBitTableBatchedEmbeddingBagsCodegen(spec.tables, device=device, pooling_mode=spec.pooling,
                                                  output_dtype=spec.out_ty, indices_dtype=spec.index_dtype)
    mod.fill_random_weights(seed)
    batches = [make_batch(spec, seed + 1 + 7919 * i, device) for i in range(num_batches)]
    return Workload(spec, mod, batches)
