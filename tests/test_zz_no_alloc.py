"""GPU: tbe_block_bucketize_sparse_features_noalloc (no allocation, static scratch)
gives exactly the outputs of tbe_block_bucketize_sparse_features (workspace
argument), through the C ABI, on two calls in a row, the second with a smaller
input (the first given lengths, the second offsets), for register-cursor (my_size <= 64) and memory-cursor (my_size > 64)
bucket counts; a call that needs more scratch than the library holds is rejected."""
import numpy as np
import pytest
import torch

from _bucketize_cases import CASES, Case, gen_bucketize_pos, gen_case

pytestmark = pytest.mark.gpu

BY_NAME = {c.name: c for c in CASES}
WIDE = Case("i64_rank100", 6, 512, 0, 96, 4, 8, 100, np.int64)
WIDE_SMALL = Case("i32_rank70", 3, 64, 0, 40, 2, 6, 70, np.int32)


def _run(gpu, case, seed, noalloc, weights, bucketize_pos, sequence, pos, pass_offsets=True):
    from fbgemm_ascend_amd import capi
    lengths, indices, block_sizes, w = gen_case(case, seed, weights)
    d = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    plist = [d(p) for p in gen_bucketize_pos(block_sizes, case.my_size, seed)] if pos else None
    outs, new_off = capi.block_bucketize_sparse_features(
        d(lengths), d(indices), bucketize_pos, sequence, d(block_sizes), case.my_size, weights=d(w),
        block_bucketize_pos=plist, noalloc=noalloc, pass_offsets=pass_offsets)
    torch.cuda.synchronize()
    return [None if o is None else o.cpu() for o in outs] + [new_off.cpu()]


PAIRS = [("i64_stress", "i32_pow2_basic"), ("i64_rank64", "i64_nonpow2_rank5"), ("WIDE", "WIDE_SMALL"),
         ("i32_many_features", "i32_mysize1")]


@pytest.mark.parametrize("big,small", PAIRS)
@pytest.mark.parametrize("weights,bucketize_pos,sequence,pos", [(False, False, False, False),
                                                                (True, True, True, False),
                                                                (True, False, True, True)])
def test_noalloc_matches_workspace_entry(pkg, gpu, big, small, weights, bucketize_pos, sequence, pos):
    names = ["new_lengths", "new_indices", "new_weights", "new_pos", "unbucketize_permute", "new_offsets"]
    cases = {"WIDE": WIDE, "WIDE_SMALL": WIDE_SMALL, **BY_NAME}
    for step, name in enumerate((big, small)):
        case = cases[name]
        seed = 100 + step
        print(f"[gpu] noalloc call {step + 1}: {name} my_size={case.my_size} w={weights} pos={bucketize_pos} "
              f"seq={sequence} poslist={pos}", flush=True)
        # the first call hands over the lengths (the library forms the offsets in its
        # scratch), the second their cumsum
        got = _run(gpu, case, seed, True, weights, bucketize_pos, sequence, pos, pass_offsets=step == 1)
        want = _run(gpu, case, seed, False, weights, bucketize_pos, sequence, pos)
        for n, g, e in zip(names, got, want):
            assert (g is None) == (e is None), n
            if e is not None:
                assert torch.equal(g, e), f"{name}: {n} differs"


def test_noalloc_rejects_oversized_calls(pkg, gpu):
    from fbgemm_ascend_amd import capi
    my, L = 2000, 5000  # 40 MB of write cursors > the 32 MiB scratch
    lengths = torch.ones(L, dtype=torch.int32, device=gpu)
    indices = torch.arange(L, dtype=torch.int32, device=gpu)
    bs = torch.full((1,), 4, dtype=torch.int32, device=gpu)
    with pytest.raises(capi.TbeError, match="scratch"):
        capi.block_bucketize_sparse_features(lengths, indices, False, False, bs, my, noalloc=True)
    # the same call fits the workspace entry point
    capi.block_bucketize_sparse_features(lengths, indices, False, False, bs, my)


def test_noalloc_under_graph_capture(pkg, gpu):
    """The callers this entry point is for: a HIP graph captures one call (no allocation
    by the library inside the capture) and every replay, with new indices copied into
    the captured input, equals the workspace entry point's eager result."""
    from fbgemm_ascend_amd import capi
    case = BY_NAME["i64_pow2_basic"]
    lengths, indices, block_sizes, _ = gen_case(case, 5)
    L = torch.as_tensor(lengths, device=gpu)
    I = torch.as_tensor(indices, device=gpu)
    bs = torch.as_tensor(block_sizes, device=gpu)

    def run(noalloc):
        return capi.block_bucketize_sparse_features(L, I, True, True, bs, case.my_size, noalloc=noalloc)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            run(True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs_g, off_g = run(True)
    rng = np.random.default_rng(17)
    limit = int(block_sizes.max()) * case.my_size
    for rep in range(3):
        I.copy_(torch.as_tensor(rng.integers(0, limit, indices.size).astype(indices.dtype), device=gpu))
        want, want_off = run(False)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(off_g, want_off), f"replay {rep}: new_offsets"
        for k, (a, b) in enumerate(zip(outs_g, want)):
            assert (a is None) == (b is None), (rep, k)
            if a is not None:
                assert torch.equal(a, b), f"replay {rep}, output {k}"


def test_noalloc_calls_on_two_streams_are_ordered(pkg, gpu):
    """Calls on two streams, launched back to back with no host synchronisation, share
    the GPU's scratch (my_size > 64: the write cursors live there); each call waits for
    the previous one on the GPU, so both equal the workspace entry point's results."""
    from fbgemm_ascend_amd import capi
    names = ["new_lengths", "new_indices", "new_weights", "new_pos", "unbucketize_permute"]
    ins = []
    for seed in (31, 32):
        lengths, indices, block_sizes, w = gen_case(WIDE, seed, True)
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
        ins.append((d(lengths), d(indices), d(block_sizes), d(w)))
    want = [capi.block_bucketize_sparse_features(L, I, True, True, bs, WIDE.my_size, weights=w)
            for L, I, bs, w in ins]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"[gpu] noalloc on two streams, round {rep}", flush=True)
        got = []
        for (L, I, bs, w), st in zip(ins, streams):
            with torch.cuda.stream(st):
                got.append(capi.block_bucketize_sparse_features(L, I, True, True, bs, WIDE.my_size, weights=w,
                                                                noalloc=True, sync=False))
        torch.cuda.synchronize()
        for k, ((go, goff), (wo, woff)) in enumerate(zip(got, want)):
            assert torch.equal(goff, woff), f"round {rep}, call {k}: new_offsets"
            for n, a, b in zip(names, go, wo):
                assert torch.equal(a, b), f"round {rep}, call {k}: {n}"


_CAPTURE_FIRST = r"""
import sys
import numpy as np
import torch
sys.path[:0] = [sys.argv[1], sys.argv[1] + "/tests"]
import __graft_entry__ as graft
graft.load_package()
from fbgemm_ascend_amd import capi
from _bucketize_cases import CASES, gen_case
case = {c.name: c for c in CASES}["i64_pow2_basic"]
lengths, indices, block_sizes, _ = gen_case(case, 5)
L = torch.as_tensor(lengths, device="cuda:0")
I = torch.as_tensor(indices, device="cuda:0")
bs = torch.as_tensor(block_sizes, device="cuda:0")
torch.cuda.synchronize()
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):  # the process's first call of the entry point
    outs, off = capi.block_bucketize_sparse_features(L, I, True, True, bs, case.my_size, noalloc=True)
for rep in range(3):
    g.replay()
    torch.cuda.synchronize()
    want, want_off = capi.block_bucketize_sparse_features(L, I, True, True, bs, case.my_size)
    assert torch.equal(off, want_off), f"replay {rep}: new_offsets"
    for a, b in zip(outs, want):
        assert (a is None) == (b is None)
        assert a is None or torch.equal(a, b), f"replay {rep}"
print("capture-first OK", flush=True)
"""


def test_noalloc_first_call_under_capture(pkg, gpu, tmp_path):
    """A process whose first call of the entry point is made under HIP graph capture:
    the per-GPU set-up (scratch address, ordering event) happens inside the capture,
    and the replays equal the workspace entry point (fresh process, so no earlier call
    has done the set-up)."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "capture_first.py"
    script.write_text(_CAPTURE_FIRST)
    print("[gpu] noalloc first call under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, str(script), root], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "capture-first OK" in r.stdout
