"""GPU parity of permute_pooled_embs: the HIP kernel (through the C ABI and
through torch.ops.fbgemm / torch.ops.mxrec) against the CPU oracle, bit-exact,
on the reference test's grid (reference bench/pooled_embedding/
permute_pooled_embs/test_permute_pooled_embs.py:61-203: T in [1, 40], B up to
16384, aligned dims {16..1024} and unaligned dims [1, 1024], fp32/fp16/bf16)
and the module tests of permute_pooled_embedding_test.py:59-81."""
import numpy as np
import pytest
import torch

from test_pooled_ops import lists

pytestmark = pytest.mark.gpu

INT_VIEW = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}


def _case(T, B, dims_kind, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    if dims_kind == "aligned":
        choices = torch.tensor([16, 32, 64, 128, 256, 512, 1024])
        dims = choices[torch.randint(0, 7, (T,), generator=g)].tolist()
    else:
        dims = torch.randint(1, 1025, (T,), generator=g).tolist()
    permute = torch.randperm(T, generator=g).tolist()
    x = torch.randn(B, sum(dims), generator=g).to(dtype)
    return dims, permute, x


def _run_and_check(oracle, gpu, dims, permute, x, via):
    off, perm, inv, inv_perm = lists(dims, permute)
    want = oracle.permute_pooled_embs(x.view(INT_VIEW[x.dtype]).numpy(), off, perm, inv)
    xd = x.to(gpu)
    lists_d = [torch.from_numpy(a).to(gpu) for a in (off, perm, inv, inv_perm)]
    print(f"[gpu] permute_pooled_embs via={via} B={x.shape[0]} D={x.shape[1]} T={len(dims)} {x.dtype}", flush=True)
    if via == "capi":
        from fbgemm_ascend_amd import capi
        out = capi.permute_pooled_embs(xd, *lists_d[:3])
    elif via == "mxrec":
        out = torch.ops.mxrec.permute_pooled_embs(xd, *lists_d)
    else:
        out = torch.ops.fbgemm.permute_pooled_embs(xd, *lists_d)
    torch.cuda.synchronize()
    got = out.cpu().view(INT_VIEW[x.dtype]).numpy()
    assert np.array_equal(got, want)


CASES = [(T, B) for T in (1, 4, 17, 40) for B in (1, 32, 1000, 2049)] + [(8, 16384), (3, 16384)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dims_kind", ["aligned", "unaligned"])
@pytest.mark.parametrize("T,B", CASES)
def test_permute_matches_oracle(pkg, oracle, gpu, dtype, dims_kind, T, B):
    dims, permute, x = _case(T, B, dims_kind, dtype, seed=T * 100003 + B)
    _run_and_check(oracle, gpu, dims, permute, x, via="fbgemm")


@pytest.mark.parametrize("via", ["capi", "mxrec", "fbgemm"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_permute_every_entry_point(pkg, oracle, gpu, via, dtype):
    dims, permute, x = _case(13, 777, "unaligned", dtype, seed=7)
    _run_and_check(oracle, gpu, dims, permute, x, via=via)


def test_permute_three_dim_and_invalid_segment(pkg, oracle, gpu):
    off, perm, inv, inv_perm = lists([2, 1, 3], [1, 2, 0])
    x = torch.randn(5, 6, 4)
    out = torch.ops.fbgemm.permute_pooled_embs(x.to(gpu), *(torch.from_numpy(a).to(gpu) for a in (off, perm, inv, inv_perm)))
    assert np.array_equal(out.cpu().numpy(), oracle.permute_pooled_embs(x.numpy(), off, perm, inv))
    bad = np.array([1, 7, 0], dtype=np.int64)
    from fbgemm_ascend_amd import capi
    x2 = torch.arange(1, 13, dtype=torch.float32).reshape(2, 6)
    o = torch.full_like(x2, -1.0).to(gpu)
    capi.permute_pooled_embs(x2.to(gpu), *(torch.from_numpy(a).to(gpu) for a in (off, bad, inv)), out=o)
    torch.cuda.synchronize()
    want = oracle.permute_pooled_embs(x2.numpy(), off, bad, inv, out=np.full((2, 6), -1.0, np.float32))
    assert np.array_equal(o.cpu().numpy(), want)


def test_module_reference_permutation(pkg, gpu):
    # permute_pooled_embedding_test.py:59-66
    m = pkg.PermutePooledEmbeddings([2, 3, 1, 4], [3, 0, 2, 1], device=gpu)
    x = torch.tensor([list(range(10))], dtype=torch.float32, device=gpu)
    assert m(x).view(10).tolist() == [6, 7, 8, 9, 0, 1, 5, 2, 3, 4]


def test_module_autograd(pkg, gpu):
    # permute_pooled_embedding_test.py:68-81: grads of fc1 permuted equal input_sum * fc2.weight
    torch.manual_seed(0)
    fc1 = torch.nn.Linear(1, 10, bias=False).to(gpu)
    fc2 = torch.nn.Linear(10, 1, bias=False).to(gpu)
    perm = pkg.PermutePooledEmbeddings([2, 3, 1, 4], [3, 0, 2, 1], device=gpu)
    x = torch.randn(2, 1, device=gpu)
    out = fc2(perm(fc1(x)))
    out.sum().backward()
    res = perm(fc1.weight.grad.view(1, 10))
    torch.testing.assert_close(res, x.sum() * fc2.weight, rtol=1e-3, atol=1e-3)
