"""The operators under HIP graph capture (torch.cuda.CUDAGraph): the TBE forward,
permute_pooled_embs and block_bucketize_sparse_features; and the TBE forward called
concurrently from several caller streams and host threads.

A serving loop captures the lookup once and replays it; the TBE forward forks its
table groups onto library streams and joins them back with events, which must come
along into the capture.  Each case warms the op up eagerly (plan cached, library
streams created), captures one call, then replays the graph several times with new
inputs copied into the captured buffers and eager work of the program in between;
every replay must equal the eager result bit for bit (the same kernels run).
"""
import pytest
import torch

from test_gpu_parity import _random_case

pytestmark = pytest.mark.gpu

FP32, FP16, INT8, INT4, INT2, BF16, FP8 = 0, 1, 2, 3, 4, 5, 6


def _mixed_module(pkg, gpu, pm, out_ty, B=96, seed=11):
    """Tables of four row types and widths: several table groups, so the group streams run."""
    from fbgemm_ascend_amd import IntNBitTableBatchedEmbeddingBagsCodegen, SparseType
    specs = [(5000, 64, SparseType.INT4), (3000, 128, SparseType.INT8), (2000, 32, SparseType.FP16),
             (4000, 256, SparseType.INT2), (1000, 128, SparseType.INT4), (6000, 64, SparseType.FP8)]
    if pm == 2:
        specs = [(E, 64, ty) for (E, _, ty) in specs]
    m = IntNBitTableBatchedEmbeddingBagsCodegen(specs, device=gpu, pooling_mode=pm, output_dtype=out_ty)
    m.fill_random_weights(seed)
    return m


def _inputs(m, gpu, B, seed, weighted):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    T = len(m.specs)
    lens = torch.randint(0, 40, (T * B,), device=gpu, generator=g)
    off = torch.zeros(T * B + 1, dtype=torch.int64, device=gpu)
    torch.cumsum(lens, 0, out=off[1:])
    offs = off.tolist()
    idx = torch.cat([torch.randint(0, E, (offs[(t + 1) * B] - offs[t * B],), device=gpu, generator=g)
                     for t, (E, _, _) in enumerate(m.specs)])
    psw = torch.rand(idx.numel(), device=gpu, generator=g) if weighted else None
    return idx.to(torch.int32), off.to(torch.int32), psw


@pytest.mark.parametrize("pm,weighted,out_ty", [(0, False, FP16), (1, True, FP32), (2, False, BF16)])
def test_tbe_forward_graph_replays(pkg, gpu, pm, weighted, out_ty):
    m = _mixed_module(pkg, gpu, pm, out_ty)
    B = 96
    # inputs of equal sizes for every replay: same bag lengths, new rows and weights
    idx0, off0, psw0 = _inputs(m, gpu, B, 1, weighted)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            m(idx0, off0, psw0)  # warm-up on the capture stream: plan and library streams exist
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warmed-up stream: its library streams exist
        out_g = m(idx0, off0, psw0)
    gen = torch.Generator(device=gpu)
    for rep in range(4):
        gen.manual_seed(100 + rep)
        E_min = min(E for (E, _, _) in m.specs)
        new_idx = torch.randint(0, E_min, idx0.shape, device=gpu, generator=gen).to(idx0.dtype)
        idx0.copy_(new_idx)
        if psw0 is not None:
            psw0.copy_(torch.rand(psw0.shape, device=gpu, generator=gen))
        want = m(idx0, off0, psw0)  # eager, on the current stream
        junk = torch.randn(1 << 20, device=gpu).sum()  # other eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, want), f"replay {rep}: max diff {(out_g.float() - want.float()).abs().max()}"
        del junk


def test_single_group_graph_replays(pkg, gpu):
    """One table group: the forward runs on the caller's stream alone."""
    m, idx, off, psw = _random_case(pkg, gpu, 5, 3, INT4, 0, False, torch.int32, FP16, B=64, L=50)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            m(idx, off, psw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warmed-up stream: its library streams exist
        out_g = m(idx, off, psw)
    E_min = min(E for (E, _, _) in m.specs)
    for rep in range(3):
        idx.copy_(torch.randint(0, E_min, idx.shape, device=gpu).to(idx.dtype))
        want = m(idx, off, psw)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, want), f"replay {rep}"


def test_permute_pooled_embs_graph_replays(pkg, gpu):
    B, T, D = 64, 12, 16
    x = torch.randn(B, T * D, device=gpu)
    perm = torch.randperm(T, device=gpu)
    off = torch.arange(0, (T + 1) * D, D, dtype=torch.int64, device=gpu)
    inv_perm = torch.argsort(perm)
    op = torch.ops.fbgemm.permute_pooled_embs
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            op(x, off, perm, off, inv_perm)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warmed-up stream: its library streams exist
        y = op(x, off, perm, off, inv_perm)
    for rep in range(3):
        x.copy_(torch.randn_like(x))
        want = op(x, off, perm, off, inv_perm)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {rep}"


def test_concurrent_caller_streams_and_threads(pkg, gpu):
    """Two modules of different layouts called alternately on two caller streams, and from
    two host threads: each caller stream gets its own library streams and each layout its
    own cached plan, so every output equals the same call made alone."""
    import threading
    ma = _mixed_module(pkg, gpu, 0, FP16, seed=21)
    mb = _mixed_module(pkg, gpu, 1, FP32, seed=22)
    ia, oa, pa = _inputs(ma, gpu, 80, 3, False)
    ib, ob, pb = _inputs(mb, gpu, 80, 4, True)
    want_a = ma(ia, oa, pa)
    want_b = mb(ib, ob, pb)
    torch.cuda.synchronize()
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    outs_a, outs_b = [], []
    for _ in range(8):  # interleaved enqueue on two streams
        with torch.cuda.stream(sa):
            outs_a.append(ma(ia, oa, pa))
        with torch.cuda.stream(sb):
            outs_b.append(mb(ib, ob, pb))
    torch.cuda.synchronize()
    assert all(torch.equal(o, want_a) for o in outs_a)
    assert all(torch.equal(o, want_b) for o in outs_b)

    errors = []

    def worker(m, idx, off, psw, want, n):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                got = [m(idx, off, psw) for _ in range(n)]
            s.synchronize()
            if not all(torch.equal(o, want) for o in got):
                errors.append("mismatch")
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    th = [threading.Thread(target=worker, args=(ma, ia, oa, pa, want_a, 10)),
          threading.Thread(target=worker, args=(mb, ib, ob, pb, want_b, 10))]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=120)
    assert not errors, errors


@pytest.mark.parametrize("sequence,weighted", [(False, False), (True, True)])
def test_block_bucketize_graph_replays(pkg, gpu, sequence, weighted):
    """block_bucketize_sparse_features captured once (its offsets scan, count, scan and
    scatter kernels) and replayed with new indices and weights of the same lengths."""
    import numpy as np
    from _bucketize_cases import CASES, gen_case
    case = next(c for c in CASES if c.name == "i64_pow2_basic")
    lengths, indices, block_sizes, w = gen_case(case, 7, weights=weighted)[:4]
    L = torch.as_tensor(lengths, device=gpu)
    I = torch.as_tensor(indices, device=gpu)
    bs = torch.as_tensor(block_sizes, device=gpu)
    W = torch.as_tensor(w, device=gpu) if weighted else None
    op = torch.ops.fbgemm.block_bucketize_sparse_features

    def run():
        return op(L, I, False, sequence, bs, case.my_size, W)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs_g = run()
    rng = np.random.default_rng(99)
    for rep in range(3):
        limit = int(block_sizes.max()) * case.my_size
        I.copy_(torch.as_tensor(rng.integers(0, limit, indices.size).astype(indices.dtype), device=gpu))
        if W is not None:
            W.copy_(torch.rand(W.shape, device=gpu))
        want = run()  # eager
        junk = torch.randn(1 << 20, device=gpu).sum()  # other eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for k, (a, b) in enumerate(zip(outs_g, want)):
            assert (a is None) == (b is None), (rep, k)
            if a is not None:
                assert torch.equal(a, b), f"replay {rep}, output {k}"
        del junk
