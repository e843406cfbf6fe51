"""Benchmark of the quantized TBE inference forward on one MI355X.

Workload (the INT4 26-table DLRM shape the metric is quoted on):
26 tables x 4M rows, D=128, INT4 rowwise (80-byte padded rows), B=8192,
bag length Poisson(30) clipped to [1,100], Zipf(1.05) indices (ranks scattered by a
random permutation per table), int32 indices/offsets, SUM pooling, fp16 output
[8192, 3328].  A "step" is one call of
torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function over that batch,
with every input resident in HBM before the timed region starts.

Timing: one pair of HIP events on the launch stream around the timed calls (GPU time per
call = span / calls) and the host wall clock around the same loop (`ms_per_step`).
The timed loop rotates over --batches (default 4) distinct batches drawn from the
same distributions (every table keeps its Zipf rank -> row map), all resident in
HBM before timing, so each call meets the cache state a stream of fresh requests
leaves; the same batch replayed back to back and a cache-scrubbed call are reported
beside it (`replay_same_batch`, `cold_cache`).

Prints ONE JSON line.  `value` = pooled lookups per second; `roofline` prices the
kernel's algorithmic bytes (unpadded rows of every lookup + indices + offsets +
output) per launch against the 8 TB/s HBM peak; `cpu_baseline` times the C oracle
(OpenMP) on a bounded sample of the same workload on this host's cores, reading the
whole tables from host memory; `cpu_baseline_library` times torch's FBGEMM CPU
kernels (torch.ops.quantized.embedding_bag_*_rowwise_offsets) on the same sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=2, help="benchmark configuration id (0-4)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target wall time of the CPU leg")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache measurement")
    ap.add_argument("--no-replay", action="store_true", help="skip the same-batch replay measurement")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay measurement")
    ap.add_argument("--batches", type=int, default=4,
                    help="distinct batches generated before timing and rotated in the timed loop")
    ap.add_argument("--flags", type=int, default=0, help="TBE_FLAG_* tuning switches (C-ABI path)")
    ap.add_argument("--bag-len", default=None,
                    help="replace the configuration's bag-length rule (e.g. fixed:33); the batch is scaled so "
                         "the call keeps the configuration's mean number of lookups (a study of the kernel, "
                         "not a benchmark configuration)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a plain 1 GiB device copy instead (calibrates rocprof FETCH/WRITE_SIZE)")
    ap.add_argument("--traffic", default=None,
                    help="HBM traffic per launch measured with rocprofv3 --pmc (JSON); default: "
                         "profiles/tbe_cfg<config>_traffic.json when it exists")
    ap.add_argument("--op", default="tbe",
                    choices=["tbe", "tbe_nobag", "tbe_large_tables", "permute_pooled_embs",
                             "block_bucketize_sparse_features"],
                    help="tbe: the headline TBE forward; tbe_nobag: the same op with pooling_mode NONE on "
                         "config 2's tables and indices; tbe_large_tables: config 2's bags on 4 tables "
                         "of 60 M INT4 rows (4.47 GiB each, past 32-bit byte offsets) beside the same "
                         "lookups on 50 M-row tables; permute_pooled_embs: the pooled-output "
                         "permutation on config 4's output shape; block_bucketize_sparse_features: the "
                         "reference's stress case (16 features x 8192 samples, 128-512 indices, my_size 16)")
    return ap.parse_args()


def bench_permute(args, pkg, dev):
    """permute_pooled_embs on the pooled output of config 4 ([32768, 200 x 128] fp16):
    a strided column copy, priced as 2 * B * total_D * 2 bytes per call."""
    import torch
    import __graft_entry__ as graft

    B, T, D = 32768, 200, 128
    g = torch.Generator(device=dev)
    g.manual_seed(0x7BE4)
    x = torch.randn(B, T * D, device=dev, generator=g).to(torch.float16)
    perm = torch.randperm(T, device=dev, generator=g)
    off = torch.arange(0, (T + 1) * D, D, dtype=torch.int64, device=dev)
    inv = off.clone()
    inv_perm = torch.argsort(perm)
    step = lambda: torch.ops.fbgemm.permute_pooled_embs(x, off, perm, inv, inv_perm)  # noqa: E731
    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in evs:
        a.record(stream)
        step()
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = sorted(a.elapsed_time(b) for a, b in evs)
    mean_ms = sum(ms) / len(ms)
    nbytes = 2 * B * T * D * 2
    achieved = nbytes / (mean_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        oracle = graft.load_oracle()
        rows = 2048
        xs = x[:rows].cpu().view(torch.int16).numpy()
        offs, perms, invs = off.cpu().numpy(), perm.cpu().numpy(), inv.cpu().numpy()
        reps, c0 = 0, time.perf_counter()
        while time.perf_counter() - c0 < args.cpu_seconds and reps < 1000:
            oracle.permute_pooled_embs(xs, offs, perms, invs)
            reps += 1
        el = time.perf_counter() - c0
        cpu = {"value": 2 * rows * T * D * 2 * reps / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"{rows} of {B} rows, {reps} reps in {el:.1f}s, oracle/tbe_oracle.c (1 thread)"}
    out = {"metric": "permute_pooled_embs achieved HBM GB/s, 1 GPU", "value": achieved, "unit": "GB/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3 / args.steps,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
           "data": "synthetic (seeded, generated on device)",
           "config": {"workload": "permute_pooled_embs of config 4's pooled output", "batch": B,
                      "features": T, "D": D, "dtype": "fp16"},
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBPS, "traffic": None},
           "kernel_ms": mean_ms, "kernel_ms_median": ms[len(ms) // 2], "bytes_per_step": nbytes,
           "cpu_baseline": cpu}
    print(json.dumps(out), flush=True)


def bench_nobag(args, pkg, dev):
    """pooling_mode NONE (row a9 of the scope, N:44-340) on config 2's tables and
    indices: every lookup writes its dequantised row, out [N, 128] fp16.  Priced as
    N x (68 B row + 4 B index + 256 B output)."""
    import torch
    from fbgemm_ascend_amd.workloads import make_workload

    wl = make_workload(2, device=dev)
    m = wl.module
    op = torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function

    def step():
        return op(dev_weights=m.weights_dev, uvm_weights=m.weights_uvm, weights_placements=m.weights_placements,
                  weights_offsets=m.weights_offsets, weights_tys=m.weights_tys, D_offsets=m.D_offsets,
                  total_D=m.total_D, max_int2_D=m.max_int2_D, max_int4_D=m.max_int4_D, max_int8_D=m.max_int8_D,
                  max_float16_D=m.max_float16_D, max_float32_D=m.max_float32_D, indices=wl.indices,
                  offsets=wl.offsets, pooling_mode=2, indice_weights=None, output_dtype=m.output_dtype,
                  lxu_cache_weights=None, lxu_cache_locations=None, row_alignment=m.row_alignment,
                  max_float8_D=m.max_float8_D, fp8_exponent_bits=m.fp8_exponent_bits,
                  fp8_exponent_bias=m.fp8_exponent_bias)
    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in evs:
        a.record(stream)
        step()
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = sorted(a.elapsed_time(b) for a, b in evs)
    mean_ms = sum(ms) / len(ms)
    N = wl.num_indices
    nbytes = N * (68 + wl.indices.element_size() + 128 * 2)
    achieved = nbytes / (mean_ms * 1e-3) / 1e9
    # the same rows read and an [N, 128] fp16 output written, no arithmetic
    calib = gather_calibration(wl, stream, lambda order, fn: time_calls(stream, order, fn), [0] * args.steps,
                               mean_ms, [nbytes], out_bytes=N * 128 * 2)
    out = {"metric": "TBE nobag lookups/s, 1 GPU", "value": N / (mean_ms * 1e-3), "unit": "lookups/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3 / args.steps,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int4",
           "data": "synthetic (seeded, generated on device)",
           "config": {"workload": "config 2 tables and indices, pooling_mode NONE", "lookups": N, "D": 128,
                      "output": "fp16"},
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBPS, "traffic": None},
           "kernel_ms": mean_ms, "kernel_ms_median": ms[len(ms) // 2], "bytes_per_step": nbytes,
           "gather_calibration": calib, "cpu_baseline": None}
    print(json.dumps(out), flush=True)


def bench_large_tables(args, pkg, dev):
    """Tables past 32-bit byte offsets (a9/a2 of the scope on a 288 GB GPU): config 2's
    bag lengths and Zipf(1.05) rows on 4 INT4 D=128 tables of 60 M rows (4.47 GiB each,
    64-bit row addresses), SUM and NONE, timed beside the same lookups on 4 tables of 50 M
    rows (3.73 GiB, 32-bit offsets).  Batches rotate as in the headline."""
    import dataclasses
    import torch
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen
    from fbgemm_ascend_amd.workloads import config_spec, make_batch

    base = config_spec(2)
    stream = torch.cuda.current_stream(dev)
    res = {}
    for E in (60_000_000, 50_000_000):
        spec = dataclasses.replace(base, tables=[(E, 128, base.tables[0][2])] * 4)
        m = IntNBitTableBatchedEmbeddingBagsCodegen(spec.tables, device=dev, pooling_mode=spec.pooling,
                                                    output_dtype=spec.out_ty, indices_dtype=spec.index_dtype)
        m.fill_random_weights(0x7BE0 + 2)
        bs = [make_batch(spec, 0x7BE0 + 3 + 7919 * i, dev) for i in range(max(1, args.batches))]
        order = [i % len(bs) for i in range(args.steps)]
        for pm in (0, 2):
            m.pooling_mode = pkg.PoolingMode(pm)
            for i in range(args.warmup):
                b = bs[i % len(bs)]
                m(b.indices, b.offsets, b.per_sample_weights)
            ms, wall = time_calls(stream, order, lambda i: m(bs[i].indices, bs[i].offsets, bs[i].per_sample_weights))
            res[(E, pm)] = (ms, wall)
        n = sum(b.indices.numel() for b in bs) / len(bs)
        del m, bs
        torch.cuda.empty_cache()
    ms, wall = res[(60_000_000, 0)]
    out = {"metric": "TBE lookups/s on tables past 4 GiB, 1 GPU", "value": n / (ms * 1e-3), "unit": "lookups/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3 / args.steps,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int4",
           "data": "synthetic (seeded, generated on device)",
           "config": {"workload": "4 x 60M INT4 D128 (4.47 GiB per table), config 2 bags B8192 Poisson30 "
                                  "Zipf1.05, SUM fp16", "lookups": n},
           "kernel_ms": ms, "nobag_kernel_ms": res[(60_000_000, 2)][0],
           "below_4gib": {"tables": "4 x 50M INT4 D128 (3.73 GiB)", "kernel_ms": res[(50_000_000, 0)][0],
                          "nobag_kernel_ms": res[(50_000_000, 2)][0]},
           "cpu_baseline": None, "roofline": None}
    print(json.dumps(out), flush=True)


def time_calls(stream, order, fn):
    """fn(i) for every i of `order` between one pair of HIP events on `stream`; returns
    (GPU ms per call, wall s)."""
    import torch
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a.record(stream)
    for i in order:
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / len(order), time.perf_counter() - t0


def row_addresses(wl, i: int):
    """Byte address of every lookup's row (header first) in batch i, int64 [N] on the
    device; computed outside any timed region."""
    import torch
    m, bt = wl.module, wl.batches[i]
    dev = bt.indices.device
    T, B = len(m.specs), wl.spec.B
    per_table = bt.lengths.view(T, B).sum(dim=1)
    table = torch.repeat_interleave(torch.arange(T, device=dev), per_table)
    wo = m.weights_offsets.to(dev, torch.int64)
    stride = torch.as_tensor([int(x) for x in m.row_strides], dtype=torch.int64, device=dev)
    return (m.weights_dev.data_ptr() + wo[table] + bt.indices.to(torch.int64) * stride[table]).contiguous()


def gather_calibration(wl, stream, timed, order, op_ms, alg, out_bytes=None):
    """The same batches through measure/libtbe_floor.so's tbe_gather_floor: every lookup's
    header word and payload words gathered (the lines the operator fetches) by persistent
    waves that do nothing else (64-lookup chunks, the next chunk's rows in flight), and
    about the operator's output bytes written.  Its time is a floor of the operator's
    memory work on this workload; `op_over_floor` is the operator's time over it
    (`timed(order, fn)` returns GPU ms per call and wall seconds; `op_ms` is the
    operator's ms per call measured the same way).  None when the library is not built
    or the tables are not INT rows of one payload size up to 32 words."""
    import ctypes
    import torch
    from fbgemm_ascend_amd.sparse_types import SparseType, unpadded_row_bytes

    path = os.path.join(ROOT, "measure", "libtbe_floor.so")
    m = wl.module
    sizes = {unpadded_row_bytes(ty, D) for (_, D, ty) in m.specs}
    int_rows = all(ty in (SparseType.INT8, SparseType.INT4, SparseType.INT2) for (_, _, ty) in m.specs)
    if not os.path.exists(path) or len(sizes) != 1 or not int_rows:
        return None
    payload_words = (sizes.pop() - 4) // 4
    if payload_words > 32:
        return None
    lib = ctypes.CDLL(path)
    lib.tbe_gather_floor.restype = ctypes.c_int
    addrs = [row_addresses(wl, i) for i in range(len(wl.batches))]
    n_max = max(a.numel() for a in addrs)
    out_sz = {0: 4, 1: 2, 5: 2}[m.output_dtype]
    obytes = wl.spec.B * m.total_D * out_sz if out_bytes is None else out_bytes
    out_words = max(1, round(obytes / max(1, wl.num_indices) / 4))
    out = torch.empty(max(1, n_max * out_words), dtype=torch.int32, device=addrs[0].device)
    fallback = m.weights_dev.data_ptr()
    P = ctypes.c_void_p

    def run(i):
        a = addrs[i]
        rc = lib.tbe_gather_floor(P(a.data_ptr()), ctypes.c_int64(a.numel()), ctypes.c_uint64(fallback),
                                  ctypes.c_int32(payload_words), P(out.data_ptr()), ctypes.c_int32(out_words),
                                  P(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"tbe_gather_floor failed ({rc})")

    for i in range(len(wl.batches)):
        run(i)
    floor_ms, _ = timed(order, fn=run)
    total_alg = sum(alg[i] for i in order)
    return {"kernel_ms": floor_ms, "frac": total_alg / (floor_ms * len(order) * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "op_over_floor": None if op_ms is None else op_ms / floor_ms, "out_words_per_lookup": out_words}


def cold_cache_times(calls, K: int, alg, stream, n: int):
    """The op with nothing of its tables in the L2 or the memory-side cache: before each
    call a 512 MiB scrub (larger than the 32 MB of L2 and the 256 MB memory-side cache)
    evicts them.  Timed without an event pair around each call: one event pair around n
    (scrub, call) pairs and one around the n scrubs alone; the call's time is the
    difference over n.  Two scrubs: `cold_cache` reads the buffer (a max reduction), so
    the caches hold clean scrub lines; `cold_cache_dirty` writes it (a fill), so the call
    also pays for writing back the dirty scrub lines it evicts."""
    import torch
    scrub = torch.empty(512 * 2 ** 20 // 4, dtype=torch.int32, device=stream.device)
    scrub.fill_(1)

    def span(fn):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for i in range(n):
            fn(i)
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b)

    out = []
    for kind in ("read", "write"):
        if kind == "read":
            def s(i):
                return torch.amax(scrub)
        else:
            def s(i):
                scrub.fill_(i & 0x7F)

        def pair(i, s=s):
            s(i)
            calls[i % K]()

        span(pair)  # warm-up of both kernels
        ms = (span(pair) - span(s)) / n
        alg_mean = sum(alg[i % K] for i in range(n)) / n
        out.append({"kernel_ms": ms, "frac": alg_mean / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, "scrub": kind})
    del scrub
    return out[0], out[1]


def graph_replay(calls, K: int, stream, per_graph: int = 20, replays: int = 10):
    """The op captured in a HIP graph (torch.cuda.CUDAGraph): `per_graph` calls rotating the
    K batches, warmed up eagerly on the capture stream first, then replayed; GPU ms per call
    between one event pair around the replays.  Launch-bound configurations (config 0) show
    what graph replay saves per call.  None if the capture fails."""
    import torch
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    try:
        with torch.cuda.stream(cap):
            for i in range(per_graph):
                calls[i % K]()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            for i in range(per_graph):
                calls[i % K]()
        torch.cuda.synchronize()
    except RuntimeError as e:
        return {"error": str(e)[:200]}
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(replays):
        g.replay()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (replays * per_graph)
    del g
    return {"ms_per_call": ms, "calls_per_graph": per_graph}


def _cpu_threads():
    """Host threads of the CPU legs: the process's CPU affinity, capped by OMP_NUM_THREADS
    when it is set (the GPU boxes set it to their per-GPU CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# tables up to this size are copied to the host whole; beyond it the CPU legs take the
# first tables that fit in _HOST_SUBSET_BYTES (config 4: 10 of its 200 tables) and say so
_HOST_TABLE_LIMIT = 32 << 30
_HOST_SUBSET_BYTES = 8 << 30


def _sample_bags(wl, nsamp, k=None):
    """Indices/offsets/weights of the first `nsamp` samples of each of the first k tables (all
    by default; host arrays, original row ids), in the op's table-major bag order."""
    import numpy as np
    T = len(wl.module.specs) if k is None else k
    B = wl.spec.B
    off = wl.offsets.cpu().numpy().astype(np.int64)
    idx = wl.indices.cpu().numpy()
    psw = wl.per_sample_weights.cpu().numpy() if wl.per_sample_weights is not None else None
    parts, wparts, new_off = [], [], [0]
    for t in range(T):
        lo, hi = off[t * B], off[t * B + nsamp]
        parts.append(idx[lo:hi])
        if psw is not None:
            wparts.append(psw[lo:hi])
        new_off.extend((off[t * B + 1:t * B + nsamp + 1] - lo + new_off[-1]).tolist())
    s_idx = np.concatenate(parts)
    s_off = np.asarray(new_off, dtype=idx.dtype)
    s_psw = np.concatenate(wparts) if psw is not None else None
    return s_idx, s_off, s_psw


def cpu_baseline(wl, target_s: float):
    """Time the C oracle (OpenMP) on a bounded sample of the workload: the whole batch when it
    holds at most 2 M lookups, else the first B/8 samples of every table, reading rows from
    a host copy of the whole tables (of the first tables that fit in _HOST_SUBSET_BYTES when
    all of them exceed _HOST_TABLE_LIMIT: config 4, labelled as a subset)."""
    import numpy as np
    import __graft_entry__ as graft

    oracle = graft.load_oracle()
    cores = _cpu_threads()
    m = wl.module
    B = wl.spec.B
    T = len(m.specs)
    # the whole batch when it is small (per-call overheads would dominate a slice of it)
    nsamp = B if wl.num_indices <= (2 << 20) else max(1, B // 8)
    pm = int(m.pooling_mode)
    bits, bias = m.fp8_exponent_bits, m.fp8_exponent_bias
    wo = m.weights_offsets.cpu().numpy()
    ends = wo + np.array([E * int(st) for (E, _, _), st in zip(m.specs, m.row_strides)], dtype=np.int64)
    # tables are laid out in order: keep the first k whose rows end within the host copy limit
    k = T if int(ends.max()) <= _HOST_TABLE_LIMIT else max(1, int(np.searchsorted(ends, _HOST_SUBSET_BYTES, "right")))
    weights = m.weights_dev[:int(ends[:k].max())].cpu().numpy()
    s_idx, s_off, s_psw = _sample_bags(wl, nsamp, k)
    prob = dict(weights=weights, weights_offsets=wo[:k], weights_tys=m.weights_tys.cpu().numpy()[:k],
                D_offsets=m.D_offsets.cpu().numpy()[:k + 1], indices=s_idx, offsets=s_off, psw=s_psw)
    layout = ("whole tables in host memory" if k == T else
              f"first {k} of {T} tables (whole, host-resident; all {T} exceed the host copy limit)")
    n_lookups = int(prob["offsets"][-1])

    def run():
        oracle.forward(prob["weights"], prob["weights_offsets"], prob["weights_tys"], prob["D_offsets"],
                       prob["indices"], prob["offsets"], pm, prob["psw"], m.output_dtype,
                       fp8_exponent_bits=bits, fp8_exponent_bias=bias, num_threads=cores)

    run()  # page in
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s or reps >= 100000:
            break
    res = {"value": n_lookups * reps / el, "unit": "pooled lookups/s", "cores": cores, "kind": "port",
           "sample": f"first {nsamp} of {B} samples x {k} tables ({n_lookups} lookups), {layout}, "
                     f"{reps} reps in {el:.1f}s, oracle/tbe_oracle.c OpenMP fp32 on {cores} threads "
                     f"(process affinity capped by OMP_NUM_THREADS, the box's per-GPU CPU share)",
           "cpu_model": _cpu_model()}
    return res, library_baseline(wl, prob, k, cores, target_s)


def library_baseline(wl, prob, k: int, cores: int, target_s: float):
    """torch.ops.quantized.embedding_bag_{byte,4bit,2bit}_rowwise_offsets (FBGEMM's CPU kernels
    shipped with torch), one call per INT8/INT4/INT2 table of the oracle's sample (the first k
    tables), whole tables repacked to the scale/bias-last row layout those kernels read, with
    the per-sample weights when the workload has them.  Tables of other row types are left
    out (and counted out of the lookups); None if there is no INT table.  Those kernels sum
    (MEAN is the same sum, scaled afterwards) and return fp32."""
    import numpy as np
    import torch

    m = wl.module
    fns = {2: torch.ops.quantized.embedding_bag_byte_rowwise_offsets,
           3: torch.ops.quantized.embedding_bag_4bit_rowwise_offsets,
           4: torch.ops.quantized.embedding_bag_2bit_rowwise_offsets}
    w = prob["weights"]
    wo = prob["weights_offsets"]
    Bs = (len(prob["offsets"]) - 1) // k
    off = prob["offsets"].astype(np.int64)
    idx = prob["indices"].astype(np.int64)
    psw = prob["psw"]
    calls, n_lookups, used = [], 0, set()
    for t in range(k):
        E, D, ty = m.specs[t]
        ty = int(ty)
        if ty not in fns:
            continue
        payload = D * {2: 8, 3: 4, 4: 2}[ty] // 8
        stride = int(m.row_strides[t])
        rows = w[wo[t]:wo[t] + E * stride].reshape(E, stride)
        if ty == 2:  # fp32 scale and bias after the codes
            sb = np.empty((E, 2), dtype=np.float32)
            sb[:, 0] = rows[:, 0:2].copy().view(np.float16)[:, 0]
            sb[:, 1] = rows[:, 2:4].copy().view(np.float16)[:, 0]
            lib = np.concatenate([rows[:, 4:4 + payload], sb.view(np.uint8).reshape(E, 8)], 1)
        else:        # fp16 scale and bias after the codes
            lib = np.concatenate([rows[:, 4:4 + payload], rows[:, 0:4]], 1)
        lo, hi = off[t * Bs], off[(t + 1) * Bs]
        pw = torch.from_numpy(np.ascontiguousarray(psw[lo:hi])) if psw is not None else None
        calls.append((fns[ty], torch.from_numpy(np.ascontiguousarray(lib)), torch.from_numpy(idx[lo:hi]),
                      torch.from_numpy(off[t * Bs:(t + 1) * Bs + 1] - lo), pw))
        n_lookups += int(hi - lo)
        used.add({2: "byte", 3: "4bit", 4: "2bit"}[ty])
    if not calls:
        return None
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        def run():
            for fn, tab, i, o, pw in calls:
                fn(tab, i, o, False, 0, False, pw, None, True)
        run()
        reps, t0 = 0, time.perf_counter()
        while True:
            run()
            reps += 1
            el = time.perf_counter() - t0
            if el >= target_s or reps >= 100000:
                break
    finally:
        torch.set_num_threads(prev)
    left_out = k - len(calls)
    return {"value": n_lookups * reps / el, "unit": "pooled lookups/s", "cores": cores, "kind": "library",
            "sample": f"the oracle's sample, {len(calls)} INT tables ({n_lookups} lookups"
                      + (f"; {left_out} tables of other row types left out" if left_out else "")
                      + f"), whole tables repacked, torch.ops.quantized.embedding_bag_"
                      f"{'/'.join(sorted(used))}_rowwise_offsets per table"
                      + (" with per-sample weights" if psw is not None else "")
                      + f", fp32 out, {reps} reps in {el:.1f}s, torch.set_num_threads({cores})",
            "cpu_model": _cpu_model()}


def bench_bucketize(args, pkg, dev):
    """block_bucketize_sparse_features on the reference's i64_stress perf case, priced at the
    op's unavoidable bytes: indices read once and written once, lengths read, new_lengths written."""
    import torch
    import __graft_entry__ as graft

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from _bucketize_cases import CASES, gen_case

    case = [c for c in CASES if c.name == "i64_stress"][0]
    # three seeded inputs, rotated call by call: a call does not find its indices in
    # the memory-side cache because the previous call read the same ones
    inputs = []
    for seed in (0x7BE7, 0x7BE6, 0x7BE5):  # 0x7BE5's arrays stay for the sizes and the CPU leg
        lengths, indices, block_sizes, _ = gen_case(case, seed)
        inputs.append(tuple(torch.from_numpy(a).to(dev) for a in (lengths, indices, block_sizes)))
    op = torch.ops.fbgemm.block_bucketize_sparse_features
    step = lambda i: op(inputs[i % 3][0], inputs[i % 3][1], False, False, inputs[i % 3][2], case.my_size)  # noqa: E731
    for i in range(args.warmup):
        step(i)
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        step(i)
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = sorted(a.elapsed_time(b) for a, b in evs)
    per_call_mean = sum(ms) / len(ms)
    # one event pair around all calls (an event pair around each call adds its own gap)
    mean_ms, _ = time_calls(stream, range(args.steps), step)
    N, L = indices.size, lengths.size
    nbytes = 2 * N * indices.itemsize + L * lengths.itemsize + case.my_size * L * lengths.itemsize
    cpu = None
    if not args.no_cpu_baseline:
        oracle = graft.load_oracle()
        rows = L // 16
        n_s = int(lengths[:rows].sum())
        reps, c0 = 0, time.perf_counter()
        while time.perf_counter() - c0 < args.cpu_seconds and reps < 1000:
            oracle.block_bucketize_sparse_features(lengths[:rows], indices[:n_s], False, False, block_sizes,
                                                   case.my_size)
            reps += 1
        el = time.perf_counter() - c0
        cpu = {"value": n_s * reps / el, "unit": "indices/s", "cores": 1, "kind": "port",
               "sample": f"first {rows} of {L} rows ({n_s} indices), {reps} reps in {el:.1f}s, "
                         "oracle/tbe_oracle.c (1 thread)"}
    achieved = nbytes / (mean_ms * 1e-3) / 1e9
    out = {"metric": "block_bucketize_sparse_features indices/s, 1 GPU", "value": N / (mean_ms * 1e-3),
           "unit": "indices/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": wall * 1e3 / args.steps, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "int64", "data": "synthetic (seeded; 3 inputs rotated)",
           "config": {"workload": "reference perf case i64_stress", "features": case.num_features,
                      "batch": case.batch_size, "lengths": [case.min_length, case.max_length],
                      "my_size": case.my_size, "num_indices": int(N)},
           "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBPS, "traffic": None},
           "kernel_ms": mean_ms, "kernel_ms_per_call_events": {"mean": per_call_mean, "median": ms[len(ms) // 2]},
           "bytes_per_step": nbytes,
           "cpu_baseline": cpu}
    print(json.dumps(out), flush=True)


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the path shards table-wise across GPUs by design but no multi-GPU run is provided.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__ as graft
    pkg = graft.load_package()
    from fbgemm_ascend_amd.workloads import make_workload

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.op == "tbe_nobag":
        bench_nobag(args, pkg, dev)
        return
    if args.op == "tbe_large_tables":
        bench_large_tables(args, pkg, dev)
        return
    if args.op == "permute_pooled_embs":
        bench_permute(args, pkg, dev)
        return
    if args.op == "block_bucketize_sparse_features":
        bench_bucketize(args, pkg, dev)
        return
    if args.copy_calibration:
        src = torch.randint(0, 255, (2 ** 30,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.warmup + args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel(), "copy_bytes_written": dst.numel(),
                          "calls": args.warmup + args.steps}), flush=True)
        return
    wl = make_workload(args.config, device=dev, num_batches=max(1, args.batches), bag_len=args.bag_len)
    m = wl.module
    K = len(wl.batches)
    torch.cuda.synchronize()

    if args.flags:
        # C-ABI path with tuning switches: plan, upload and output allocation happen once here
        calls = [pkg.capi.prepare_forward(m.weights_dev, m.weights_offsets, m.weights_tys, m.D_offsets,
                                          bt.indices, bt.offsets, int(m.pooling_mode), bt.per_sample_weights,
                                          m.output_dtype, flags=args.flags) for bt in wl.batches]
    else:
        calls = [(lambda i=i: wl.run(i)) for i in range(K)]
    lookups = [wl.num_indices_of(i) for i in range(K)]
    alg = [wl.algorithmic_bytes(i) for i in range(K)]
    stream = torch.cuda.current_stream(dev)

    def timed(order, fn=None):
        """HIP events around every call on the launch stream; returns (per-call ms, wall s)."""
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in order]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for (a, b), i in zip(evs, order):
            a.record(stream)
            if fn is None:
                calls[i]()
            else:
                fn(i)
            b.record(stream)
        torch.cuda.synchronize()
        return [a.elapsed_time(b) for a, b in evs], time.perf_counter() - t0

    def timed_span(order, fn=None):
        """One HIP event before and one after the calls, on the launch stream (no event
        between calls, which would add its own gap to every call); returns (GPU ms per
        call, wall s)."""
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        a.record(stream)
        for i in order:
            if fn is None:
                calls[i]()
            else:
                fn(i)
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / len(order), time.perf_counter() - t0

    order = [s % K for s in range(args.steps)]

    # The secondary measurements run first, so that the headline is timed with the GPU
    # at the clocks of continuous work (after ~2 s idle a call takes ~8 % longer for
    # its first ~100 calls): cold cache, the gather floor, the same batch replayed and
    # the HIP graph; the calls of the last three also write back what the scrubs left.
    cold = cold_dirty = None
    if not args.no_cold:
        cold, cold_dirty = cold_cache_times(calls, K, alg, stream, min(args.steps, 20))
    calib = gather_calibration(wl, stream, timed_span, order, None, alg)
    # the same batch replayed back to back (L2 and MALL hold the previous call's rows)
    replay_kernel_ms = None
    if not args.no_replay:
        replay_kernel_ms, _ = timed_span([0] * args.steps)
    graph = None if (args.flags or args.no_graph) else graph_replay(calls, K, stream)

    for s in range(args.warmup):
        calls[s % K]()
    torch.cuda.synchronize()

    # headline: a stream of distinct batches from the same distributions (batch s % K)
    kernel_ms, wall = timed_span(order)
    ms_per_step = wall * 1e3 / args.steps
    total_lookups = sum(lookups[i] for i in order)
    total_alg = sum(alg[i] for i in order)
    achieved = total_alg / (kernel_ms * args.steps * 1e-3) / 1e9
    # the same calls with an event pair around each one (per-call spread; each pair adds a gap)
    per_call_ms, _ = timed(order)
    if calib is not None:
        calib["op_over_floor"] = kernel_ms / calib["kernel_ms"]

    traffic = None
    tpath = args.traffic or os.path.join(ROOT, "profiles", f"tbe_cfg{args.config}_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            t = json.load(f)
        if t.get("config") == args.config and t.get("batches") == K:
            traffic = t.get("hbm_bytes_per_launch")

    def frac(ms, nbytes):
        return nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS

    res = {
        "metric": "pooled lookups/sec + achieved HBM GB/s (% roofline), INT4/INT8 TBE fwd, 1 GPU",
        "value": total_lookups / wall,
        "unit": "pooled lookups/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {2: "int8", 3: "int4"}.get(int(m.specs[0][2]), "mixed") if args.config != 3 else "mixed",
        "data": f"synthetic (seeded, generated on device); {K} distinct batches from the same "
                "distributions, rotated (step s uses batch s % K)",
        "config": {"workload": f"config{args.config}: {wl.spec.description}" +
                               (f" with bag_len {args.bag_len} (study, B={wl.spec.B})" if args.bag_len else ""),
                   "tables": len(m.specs), "rows_per_table": m.specs[0][0] if args.config != 3 else "mixed",
                   "D": m.specs[0][1] if args.config != 3 else "mixed", "batch": wl.spec.B,
                   "bag_len": wl.spec.bag_len, "zipf_alpha": wl.spec.zipf_alpha,
                   "index_dtype": str(wl.indices.dtype).replace("torch.", ""),
                   "pooling": wl.spec.pooling.name, "output": {0: "fp32", 1: "fp16", 5: "bf16"}[m.output_dtype],
                   "batches": K, "lookups_per_step": total_lookups / args.steps, "bags_per_step": wl.num_bags},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic},
        "kernel_ms": kernel_ms,
        "kernel_ms_per_call_events": {"mean": sum(per_call_ms) / len(per_call_ms),
                                      "median": sorted(per_call_ms)[len(per_call_ms) // 2]},
        "algorithmic_bytes_per_step": total_alg / args.steps,
        "bags_per_s": wl.num_bags * args.steps / wall,
        "replay_same_batch": ({"kernel_ms": replay_kernel_ms, "frac": frac(replay_kernel_ms, alg[0])}
                              if replay_kernel_ms is not None else None),
        "cold_cache": cold,
        "cold_cache_dirty": cold_dirty,
        "gather_calibration": calib,
        "graph_replay": graph,
    }
    res["cpu_baseline"], res["cpu_baseline_library"] = (None, None)
    if not args.no_cpu_baseline:
        res["cpu_baseline"], res["cpu_baseline_library"] = cpu_baseline(wl, args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
