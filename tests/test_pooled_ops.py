"""permute_pooled_embs: the CPU oracle pinned against the reference's known answers
and against torch.index_select (the reference's own host algorithm,
src/pooled_embedding_ops/permute_pooled_embs/permute_pooled_embs.cpp:83-98), plus
host-side checks of the C ABI and the op registration (no GPU needed)."""
import numpy as np
import pytest
import torch

DT = {"f32": np.float32, "f16": np.float16, "bf16": None}


def lists(dims, permute):
    off = np.concatenate([[0], np.cumsum(dims)]).astype(np.int64)
    perm = np.asarray(permute, dtype=np.int64)
    inv_dims = np.asarray(dims, dtype=np.int64)[perm]
    inv = np.concatenate([[0], np.cumsum(inv_dims)]).astype(np.int64)
    inv_perm = np.empty_like(perm)
    inv_perm[perm] = np.arange(len(perm))
    return off, perm, inv, inv_perm


def index_select_reference(x: torch.Tensor, off, perm):
    """PA:83-98: list the source columns of every output segment, then index_select dim 1."""
    cols = []
    for p in perm:
        cols += list(range(int(off[p]), int(off[p + 1])))
    return x.index_select(1, torch.tensor(cols, dtype=torch.int64))


def test_docstring_example(oracle):
    # reference permute_pooled_embedding_modules.py docstring: dims [4, 4, 8], permute [2, 0, 1]
    off, perm, inv, _ = lists([4, 4, 8], [2, 0, 1])
    x = np.arange(48, dtype=np.float32).reshape(3, 16)
    want = np.array([list(range(8, 16)) + list(range(0, 8))]) + np.array([[0], [16], [32]])
    assert np.array_equal(oracle.permute_pooled_embs(x, off, perm, inv), want.astype(np.float32))


def test_reference_net_permutation(oracle):
    # reference permute_pooled_embedding_test.py:59-66 with Net's dims [2, 3, 1, 4], permute [3, 0, 2, 1]
    off, perm, inv, _ = lists([2, 3, 1, 4], [3, 0, 2, 1])
    x = np.arange(10, dtype=np.float32).reshape(1, 10)
    got = oracle.permute_pooled_embs(x, off, perm, inv)
    assert got.reshape(10).tolist() == [6, 7, 8, 9, 0, 1, 5, 2, 3, 4]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("aligned", [True, False])
@pytest.mark.parametrize("seed", range(4))
def test_oracle_matches_index_select(oracle, dtype, aligned, seed):
    g = torch.Generator().manual_seed(100 + seed)
    T = int(torch.randint(1, 41, (1,), generator=g))
    B = int(torch.randint(1, 65, (1,), generator=g))
    if aligned:
        choices = torch.tensor([16, 32, 64, 128, 256, 512, 1024])
        dims = choices[torch.randint(0, 7, (T,), generator=g)].tolist()
    else:
        dims = torch.randint(1, 1025, (T,), generator=g).tolist()
    permute = torch.randperm(T, generator=g).tolist()
    off, perm, inv, _ = lists(dims, permute)
    x = torch.randn(B, sum(dims), generator=g).to(dtype)
    want = index_select_reference(x, off, perm)
    bits = x.view(torch.int16 if dtype != torch.float32 else torch.int32).numpy()
    got = oracle.permute_pooled_embs(bits, off, perm, inv)
    assert np.array_equal(got, want.view(torch.int16 if dtype != torch.float32 else torch.int32).numpy())


def test_oracle_three_dim_input(oracle):
    off, perm, inv, _ = lists([2, 1, 3], [1, 2, 0])
    x = torch.randn(5, 6, 4)
    want = index_select_reference(x, off, perm)
    assert np.array_equal(oracle.permute_pooled_embs(x.numpy(), off, perm, inv), want.numpy())


def test_oracle_invalid_permutation_zero_fills(oracle):
    off, perm, inv, _ = lists([2, 2], [1, 0])
    perm = np.array([5, 0], dtype=np.int64)  # 5 is outside [0, T)
    x = np.arange(8, dtype=np.float32).reshape(2, 4) + 1
    got = oracle.permute_pooled_embs(x, off, perm, inv)
    assert np.array_equal(got, np.array([[0, 0, 1, 2], [0, 0, 5, 6]], dtype=np.float32))


def test_schemas_registered(pkg):
    for qual in ("fbgemm::permute_pooled_embs", "mxrec::permute_pooled_embs"):
        schema = torch._C._dispatch_find_schema_or_throw(qual, "")
        assert schema is not None


def test_cpu_tensors_have_no_fallback(pkg):
    off, perm, inv, inv_perm = (torch.from_numpy(a) for a in lists([2, 2], [1, 0]))
    with pytest.raises((RuntimeError, NotImplementedError)):
        torch.ops.fbgemm.permute_pooled_embs(torch.zeros(2, 4), off, perm, inv, inv_perm)


def test_c_abi_rejects_bad_args_without_gpu(pkg):
    import ctypes
    c = pkg.capi
    a = c.TbePermutePooledArgs()
    a.B, a.total_D, a.inner, a.elem_size, a.T = 2, 4, 1, 3, 2
    rc = c.lib().tbe_permute_pooled_embs(ctypes.byref(a), None)
    assert rc != 0 and "float32, float16, or bfloat16" in c.last_error()
    a.elem_size, a.T = 4, 0
    rc = c.lib().tbe_permute_pooled_embs(ctypes.byref(a), None)
    assert rc != 0 and "permute_list" in c.last_error()
