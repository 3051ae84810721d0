"""The MoE layer's stages around the combine, single GPU (the callers on either side of the path).

Mirrors ``MoEFeedForward`` (src/fastmoe/models/tiny_model.py:42-420) at world size 1 -- where
every exchange of the reference short-circuits (:168-175, :314-315) -- with the combine fed the
ragged per-expert list instead of a ``torch.cat`` of it:

  gate_and_sort    (:79-164)  router -> top-k -> fp32 softmax -> ``permute_tokens`` (HIP sort +
                              gather); returns the reference's 6-tuple
  compute_experts  (:282-294) each expert on its own rows; returns the list of per-expert outputs
                              (the reference concatenates them, :294 -- the copy the grouped
                              combine exists to avoid)
  unpermute        (:396-409) FAST: ``grouped_weighted_scatter_add`` over the per-expert list;
                              STANDARD: the reference's torch formulation (mul + index_add_),
                              kept as the comparison implementation the selector names -- FAST
                              never falls back to it
  MoEFeedForward   the layer wiring these stages (router + experts as in :66-77)

The router GEMM, top-k, softmax and the expert MLPs are torch library calls, as in the reference.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from .consts import MoEImplementation
from .dispatch import PermutedTokens, permute_tokens
from .ops import _apply, _GroupedCombinePermuted, grouped_weighted_scatter_add

__all__ = ["MoEFeedForward", "compute_experts", "gate_and_sort", "unpermute"]


def gate_and_sort(x: torch.Tensor, router: nn.Module, top_k: int, num_experts: int):
    """Routing and permutation of tiny_model.py:79-164 at world size 1.

    Returns ``(permuted_data, rank_counts, expert_counts_by_rank, reverse_map_indices,
    sorted_weights, (B, T))`` like the reference (:160-166): ``rank_counts`` = [T*k] (:158),
    ``expert_counts_by_rank`` = counts viewed [1, E] (:157).
    """
    B, T, D = x.shape
    x_flat = x.reshape(-1, D)
    logits = router(x_flat)
    topk_weights, topk_indices = torch.topk(logits, top_k, dim=-1)
    topk_weights = F.softmax(topk_weights, dim=-1, dtype=torch.float32).type_as(x)
    p = permute_tokens(x_flat, topk_indices, topk_weights, num_experts)
    rank_counts = torch.tensor([p.permuted_data.shape[0]], device=x.device, dtype=torch.long)
    return _Routed((p.permuted_data, rank_counts, p.expert_counts.view(1, num_experts),
                    p.reverse_map_indices, p.sorted_weights, (B, T)), p)


class _Routed(tuple):
    """gate_and_sort's 6-tuple (tiny_model.py:160-166) that also carries the permutation."""

    def __new__(cls, items, permutation):
        self = super().__new__(cls, items)
        self.permutation = permutation
        return self


def compute_experts(experts: Sequence[nn.Module], recv_data: torch.Tensor,
                    tokens_per_expert: Sequence[int]) -> List[torch.Tensor]:
    """Each expert on its own rows (tiny_model.py:282-291); the per-expert outputs stay separate
    allocations (no :294 cat).  An expert with no rows yields an empty [0, D] tensor."""
    chunks = recv_data.split(list(tokens_per_expert), dim=0)
    out = []
    for chunk, expert in zip(chunks, experts):
        if chunk.shape[0] > 0:
            out.append(expert(chunk))
        else:
            out.append(torch.empty(0, recv_data.shape[1], device=recv_data.device,
                                   dtype=recv_data.dtype))
    return out


def unpermute(x_out: Union[torch.Tensor, Sequence[torch.Tensor]], reverse_map_indices: torch.Tensor,
              sorted_weights: torch.Tensor, original_shape, implementation=MoEImplementation.FAST,
              permutation: Optional[PermutedTokens] = None):
    """Combine of tiny_model.py:396-409.  ``x_out`` is the packed [T*k, D] tensor (as the
    reference passes it) or the list of per-expert outputs (no concatenation).  Given the
    ``permutation`` that produced ``reverse_map_indices``, the FAST combine builds its plan from
    the permutation's slot map (one kernel) instead of inverting the scatter index."""
    B, T = original_shape
    parts = list(x_out) if isinstance(x_out, (list, tuple)) else [x_out]
    D = parts[0].shape[1]
    impl = MoEImplementation(implementation)
    if impl == MoEImplementation.FAST:
        if permutation is not None:
            k = permutation.slot_pos.numel() // (B * T) if B * T else 0
            out = _apply(_GroupedCombinePermuted, (permutation.slot_pos, k), reverse_map_indices,
                         sorted_weights, (B * T, D), *parts)
        else:
            out = grouped_weighted_scatter_add(parts, reverse_map_indices, sorted_weights,
                                               (B * T, D))
        return out.view(B, T, D)
    if impl == MoEImplementation.STANDARD:
        packed = parts[0] if len(parts) == 1 else torch.cat(parts, dim=0)
        weighted = packed * sorted_weights.unsqueeze(-1)
        out = torch.zeros(B * T, D, device=packed.device, dtype=weighted.dtype)
        out.index_add_(0, reverse_map_indices, weighted)
        return out.view(B, T, D)
    raise NotImplementedError(impl)


class MoEFeedForward(nn.Module):
    """MoE feed-forward layer of tiny_model.py:42-77 on one GPU: router, E experts
    (Linear -> GELU -> Linear), HIP permutation, per-expert compute, grouped combine."""

    def __init__(self, dim: int, ff_dim: int, num_experts: int, top_k: int,
                 implementation=MoEImplementation.FAST) -> None:
        super().__init__()
        self.dim = dim
        self.num_experts = num_experts
        self.top_k = top_k
        self.implementation = MoEImplementation(implementation)
        self.router = nn.Linear(dim, num_experts, bias=False)
        self.experts = nn.ModuleList(
            [nn.Sequential(nn.Linear(dim, ff_dim, bias=False), nn.GELU(),
                           nn.Linear(ff_dim, dim, bias=False)) for _ in range(num_experts)])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        routed = gate_and_sort(x, self.router, self.top_k, self.num_experts)
        permuted, _, counts_by_rank, rev, weights, shape = routed
        # the split sizes go to the host, as in the reference (recv_splits .tolist(), :197-207)
        tokens_per_expert = counts_by_rank.view(-1).tolist()
        outs = compute_experts(self.experts, permuted, tokens_per_expert)
        if self.implementation == MoEImplementation.FAST:
            return unpermute(outs, rev, weights, shape, self.implementation,
                             permutation=routed.permutation)
        return unpermute(torch.cat(outs, 0), rev, weights, shape, self.implementation)
