"""The reference's CPU combine written with torch CPU ops -- TEST INFRASTRUCTURE ONLY.

These functions restate, step for step, what the reference runs on the CPU; they are the checker
for ``cref`` and the timed CPU baseline of bench.py (kind "port").  Never imported by the product.
"""
from __future__ import annotations

from typing import Sequence

import torch


def fwd_fallback(expert_tensors: Sequence[torch.Tensor], indices: torch.Tensor,
                 weights: torch.Tensor, out_shape, out: torch.Tensor | None = None) -> torch.Tensor:
    """src/fastmoe/kernels/ops.py:373-384: per-expert ``index_add_`` of ``t * w[:, None]`` into an
    output of ``weights.dtype`` (or into ``out``, accumulating)."""
    if out is None:
        out = torch.zeros(out_shape, device=indices.device, dtype=weights.dtype)
    offset = 0
    for t in expert_tensors:
        k = t.shape[0]
        if k > 0:
            idx_chunk = indices[offset: offset + k]
            w_chunk = weights[offset: offset + k]
            out.index_add_(0, idx_chunk, t * w_chunk.unsqueeze(-1))
        offset += k
    return out


def fwd_cat(expert_tensors: Sequence[torch.Tensor], indices: torch.Tensor, weights: torch.Tensor,
            out_shape) -> torch.Tensor:
    """src/fastmoe/benchmarks/run_on_cloud.py:17-20 (the "standard" combine): cat -> * w ->
    ``index_add_`` into fp32 zeros."""
    combined = torch.cat(list(expert_tensors), dim=0)
    weighted = combined * weights.unsqueeze(-1)
    out = torch.zeros(out_shape, device=combined.device, dtype=weighted.dtype)
    out.index_add_(0, indices, weighted)
    return out


def bwd_grad_x(grad_out: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor,
               sizes: Sequence[int], x_dtype: torch.dtype):
    """src/fastmoe/kernels/ops.py:344-353 followed by autograd's cast of each gradient to the
    expert tensor's dtype."""
    gathered = grad_out.index_select(0, indices)
    weighted = gathered * weights.unsqueeze(-1)
    return [g.to(x_dtype) for g in torch.split(weighted, list(sizes))]


def bwd_grad_w_fp64(expert_tensors: Sequence[torch.Tensor], indices: torch.Tensor,
                    weights: torch.Tensor, grad_out: torch.Tensor, T: int) -> torch.Tensor:
    """Gate gradient the reference omits on the GPU (ops.py:358-359) but its CPU path yields via
    autograd: d/dw of sum(grad_out * fwd_cat(...)), evaluated in float64."""
    w64 = weights.detach().double().requires_grad_(True)
    x64 = torch.cat([t.detach().double() for t in expert_tensors], 0)
    out = torch.zeros((T, x64.shape[1]), dtype=torch.float64)
    out = out.index_add(0, indices, x64 * w64.unsqueeze(-1))
    out.backward(grad_out.double())
    return w64.grad.detach()


def fwd_bwd_step(expert_tensors: Sequence[torch.Tensor], indices: torch.Tensor,
                 weights: torch.Tensor, grad_out: torch.Tensor, T: int):
    """One forward + backward of the reference's CPU path (the CPU baseline of bench.py):
    fwd_cat, grad_X per ops.py:344-353, grad_w as the fp32 row dot product."""
    out = fwd_cat(expert_tensors, indices, weights, (T, expert_tensors[0].shape[1]))
    sizes = [t.shape[0] for t in expert_tensors]
    gx = bwd_grad_x(grad_out, indices, weights, sizes, expert_tensors[0].dtype)
    gathered = grad_out.index_select(0, indices).float()
    gw = (gathered * torch.cat(list(expert_tensors), 0).float()).sum(-1)
    return out, gx, gw
