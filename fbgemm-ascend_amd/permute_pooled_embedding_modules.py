"""PermutePooledEmbeddings: permutes the feature blocks of a pooled embedding output.

Same constructor and call signature as fbgemm_gpu's module that the reference's
tests use (reference bench/pooled_embedding/permute_pooled_embs/
permute_pooled_embedding_modules.py and common.py:12-17): `permute[i]` is the
feature moved to position i.  The forward is torch.ops.fbgemm.permute_pooled_embs
on HIP tensors; the backward applies the inverse permutation with the same op.
"""
from __future__ import annotations

from itertools import accumulate
from typing import List, Optional

import torch


class _PermuteFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pooled_embs, offset_dim_list, permute, inv_offset_dim_list, inv_permute):
        ctx.save_for_backward(offset_dim_list, permute, inv_offset_dim_list, inv_permute)
        return torch.ops.fbgemm.permute_pooled_embs(pooled_embs, offset_dim_list, permute,
                                                    inv_offset_dim_list, inv_permute)

    @staticmethod
    def backward(ctx, grad):
        offset_dim_list, permute, inv_offset_dim_list, inv_permute = ctx.saved_tensors
        # the output's feature i came from feature permute[i]: route it back
        g = torch.ops.fbgemm.permute_pooled_embs(grad.contiguous(), inv_offset_dim_list, inv_permute,
                                                 offset_dim_list, permute)
        return g, None, None, None, None


class PermutePooledEmbeddings:
    def __init__(self, embs_dims: List[int], permute: List[int],
                 device: Optional[torch.device] = None) -> None:
        self._offset_dim_list = torch.tensor([0] + list(accumulate(embs_dims)), device=device,
                                             dtype=torch.int64)
        self._permute = torch.tensor(permute, device=device, dtype=torch.int64)
        inv_permute = [0] * len(permute)
        for i, p in enumerate(permute):
            inv_permute[p] = i
        self._inv_permute = torch.tensor(inv_permute, device=device, dtype=torch.int64)
        inv_embs_dims = [embs_dims[i] for i in permute]
        self._inv_offset_dim_list = torch.tensor([0] + list(accumulate(inv_embs_dims)), device=device,
                                                 dtype=torch.int64)

    def __call__(self, pooled_embs: torch.Tensor) -> torch.Tensor:
        dev = pooled_embs.device
        return _PermuteFn.apply(pooled_embs, self._offset_dim_list.to(dev), self._permute.to(dev),
                                self._inv_offset_dim_list.to(dev), self._inv_permute.to(dev))
