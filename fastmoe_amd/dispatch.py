"""Dispatch-side permutation of the MoE layer on gfx950 kernels: the producer of the combine.

Mirrors the sort-and-gather half of ``MoEFeedForward.gate_and_sort``
(src/fastmoe/models/tiny_model.py:108-138)::

    sort_indices        = argsort(topk_indices.view(-1))               (:112)
    reverse_map_indices = arange(T).repeat_interleave(k)[sort_indices] (:121-125)
    sorted_weights      = topk_weights.view(-1)[sort_indices]          (:128)
    permuted_data       = x_flat[reverse_map_indices]                  (:133)
    expert_counts       = bincount(sorted expert ids, minlength=E)     (:138)

computed by ``fmoe_permute_build`` (rank / scan / fill kernels) and ``fmoe_permute_gather`` (one
workgroup per token copies its row into its k packed rows).  The packed order is the stable one:
within an expert, slots keep ascending order.  The reference's argsort is unstable, so it leaves
the order of equal ids unspecified; ``torch.argsort(..., stable=True)`` gives exactly this order.

The backward is autograd-complete:
* grad of ``permuted_data`` -> grad of ``x_flat``. Each token sums its k packed rows in ascending
  row order, in fp32, rounded once. This is the deterministic combine of this package with unit
  gates: ``reverse_map_indices`` is its scatter index.
* grad of ``sorted_weights`` -> grad of ``topk_weights``, by the inverse permutation
  (``fmoe_permute_gate_grad``).
There is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

from typing import NamedTuple, Optional

import torch

from . import _abi
from .ops import (_FLOAT_CODES, _INDEX_CODES, _check_experts, _launch_fwd,
                  _metadata_and_plan_from_slots, _on_device, _refuse_autograd_capture,
                  _require_cuda, _span, _stream_handle, _validate_default,
                  prepare_metadata_and_plan)

__all__ = ["PermutedTokens", "permute_tokens"]


class PermutedTokens(NamedTuple):
    """Outputs of :func:`permute_tokens` (names of tiny_model.py:160-166)."""

    permuted_data: torch.Tensor        # [T*k, D], rows grouped by expert
    expert_counts: torch.Tensor        # int64 [E]
    reverse_map_indices: torch.Tensor  # int64 [T*k], token of each packed row
    sorted_weights: torch.Tensor       # [T*k], gate of each packed row
    expert_offsets: torch.Tensor       # int64 [E + 1], first packed row of each expert
    slot_pos: torch.Tensor             # int32 [T*k], packed row of slot t*k + j


# Unit gates of the backward combine: one grow-only buffer of ones per device, handed out as
# prefixes, built outside any graph a caller captures after its warm-up steps instead of a fill
# kernel in every backward.  A captured graph keeps the raw address of the prefix it was given
# (a pointer passed through the C ABI holds no reference), so no buffer is ever released: when a
# larger one replaces it, the old one moves to _RETIRED for the life of the process.  Sizes at
# least double, so the retired buffers together hold fewer elements than the live one.
_ONES: dict = {}
_RETIRED: list = []


def _unit_gates(n: int, dev: torch.device) -> torch.Tensor:
    ones = _ONES.get(dev)
    if ones is None or ones.numel() < n:
        if ones is not None:
            _RETIRED.append(ones)
        size = max(n, 2 * ones.numel() if ones is not None else 0, 1024)
        ones = _ONES[dev] = torch.ones(size, dtype=torch.float32, device=dev)
    return ones[:n]


def _unit_gate_combine(rows: torch.Tensor, rev: torch.Tensor, slot_pos: torch.Tensor,
                       num_tokens: int, top_k: int) -> torch.Tensor:
    """out[t] = sum of rows[g] with rev[g] == t, in ascending g, fp32, rounded once.

    Token t's rows are the packed rows of its slots, slot_pos[t * k + j], so the plan comes from
    the slot map (one thread per slot) when k <= 64; the forward orders each token's rows by g, so
    the sum is the same as from the plan of rev."""
    out = torch.empty((num_tokens, rows.shape[1]), dtype=rows.dtype, device=rows.device)
    if rows.shape[0] == 0:
        return out.zero_()
    ones = _unit_gates(rows.shape[0], rows.device)
    if top_k <= 64 and rows.shape[0] == num_tokens * top_k:
        meta, plan = _metadata_and_plan_from_slots(_check_experts([rows]), slot_pos, ones,
                                                   num_tokens, top_k)
    else:
        meta, plan = prepare_metadata_and_plan([rows], rev, ones, num_tokens, validate=False)
    _launch_fwd(meta, _abi.MODE_DET, plan, None, None, out, accumulate=False)
    return out


class _TokenPermute(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x_flat, topk_weights, topk_indices, num_experts, validate):
        lib = _abi.lib()
        T, D = x_flat.shape
        k = topk_indices.shape[1]
        E = int(num_experts)
        dev = x_flat.device
        ids = topk_indices.reshape(-1).contiguous()
        gates = topk_weights.reshape(-1).contiguous()
        N = T * k
        counts = torch.empty(E, dtype=torch.int64, device=dev)
        offsets = torch.empty(E + 1, dtype=torch.int64, device=dev)
        rev = torch.empty(N, dtype=torch.int64, device=dev)
        sorted_w = torch.empty(N, dtype=gates.dtype, device=dev)
        slot_pos = torch.empty(N, dtype=torch.int32, device=dev)
        status = torch.empty(1, dtype=torch.int32, device=dev)
        nbytes = lib.fmoe_permute_workspace_bytes(N, E)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        out = torch.empty((N, D), dtype=x_flat.dtype, device=dev)
        es = x_flat.element_size()
        with _on_device(dev):
            with _span("permute_build"):
                rc = lib.fmoe_permute_build(
                    ids.data_ptr(), _INDEX_CODES[ids.dtype], gates.data_ptr(),
                    _FLOAT_CODES[gates.dtype], T, k, E, counts.data_ptr(), offsets.data_ptr(),
                    rev.data_ptr(), sorted_w.data_ptr(), slot_pos.data_ptr(), status.data_ptr(),
                    ws.data_ptr(), _stream_handle(dev))
            _abi.check(rc, "fmoe_permute_build")
            if N and D:
                with _span("permute_gather"):
                    rc = lib.fmoe_permute_gather(
                        slot_pos.data_ptr(), T, k, D * es, x_flat.data_ptr(),
                        (x_flat.stride(0) if T > 1 else D) * es, out.data_ptr(),
                        _stream_handle(dev))
                _abi.check(rc, "fmoe_permute_gather")
        if validate:
            bad = int(status[0])
            if bad:
                raise IndexError(f"fastmoe_amd: {bad} expert ids lie outside [0, {E})")
        ctx.save_for_backward(rev, slot_pos)
        ctx.num_tokens = T
        ctx.top_k = k
        ctx.mark_non_differentiable(counts, rev, offsets, slot_pos)
        return out, sorted_w, counts, rev, offsets, slot_pos

    @staticmethod
    def backward(ctx, g_out, g_sorted_w, _g_counts, _g_rev, _g_off, _g_pos):
        rev, slot_pos = ctx.saved_tensors
        _refuse_autograd_capture("the permutation's backward", rev)
        T, k = ctx.num_tokens, ctx.top_k
        grad_x = grad_w = None
        if ctx.needs_input_grad[0] and g_out is not None:
            grad_x = _unit_gate_combine(g_out.contiguous(), rev, slot_pos, T, k)
        if ctx.needs_input_grad[1] and g_sorted_w is not None:
            gs = g_sorted_w.contiguous()
            grad_w = torch.empty(T * k, dtype=gs.dtype, device=gs.device)
            with _on_device(gs.device), _span("permute_gate_grad"):
                rc = _abi.lib().fmoe_permute_gate_grad(
                    slot_pos.data_ptr(), T * k, gs.data_ptr(), _FLOAT_CODES[gs.dtype],
                    grad_w.data_ptr(), _stream_handle(gs.device))
            _abi.check(rc, "fmoe_permute_gate_grad")
            grad_w = grad_w.view(T, k)
        return grad_x, grad_w, None, None, None


def permute_tokens(x_flat: torch.Tensor, topk_indices: torch.Tensor, topk_weights: torch.Tensor,
                   num_experts: int, *, validate: Optional[bool] = None) -> PermutedTokens:
    """Group the T*k routing slots by expert and gather the token rows into that order.

    ``x_flat`` [T, D] (unit column stride), ``topk_indices`` [T, k] int64/int32 expert ids,
    ``topk_weights`` [T, k] gates.  Returns :class:`PermutedTokens`.  Differentiable in ``x_flat``
    and ``topk_weights``.  Ids outside [0, num_experts) go after every expert's rows (not counted
    in ``expert_counts``); ``validate=True`` raises IndexError for them (one synchronisation).
    """
    _require_cuda(x_flat, "x_flat")
    _require_cuda(topk_indices, "topk_indices")
    _require_cuda(topk_weights, "topk_weights")
    if x_flat.dim() != 2:
        raise ValueError(f"fastmoe_amd: x_flat must be [T, D], got {tuple(x_flat.shape)}")
    T, D = x_flat.shape
    if topk_indices.dim() != 2 or topk_indices.shape[0] != T:
        raise ValueError(f"fastmoe_amd: topk_indices must be [{T}, k], got "
                         f"{tuple(topk_indices.shape)}")
    if topk_weights.shape != topk_indices.shape:
        raise ValueError("fastmoe_amd: topk_weights and topk_indices differ in shape")
    if topk_indices.dtype not in _INDEX_CODES:
        raise TypeError(f"fastmoe_amd: topk_indices must be int64 or int32, got {topk_indices.dtype}")
    if topk_weights.dtype not in _FLOAT_CODES or x_flat.dtype not in _FLOAT_CODES:
        raise TypeError("fastmoe_amd: unsupported x / gate dtype")
    if D > 1 and x_flat.stride(1) != 1:
        raise ValueError("fastmoe_amd: x_flat must have unit column stride")
    if not (1 <= int(num_experts) <= 4096):
        raise ValueError(f"fastmoe_amd: num_experts must be in [1, 4096], got {num_experts}")
    if len({x_flat.device, topk_indices.device, topk_weights.device}) != 1:
        raise ValueError("fastmoe_amd: x_flat, topk_indices and topk_weights must share a device")
    if torch.is_grad_enabled():
        _refuse_autograd_capture("the autograd permutation", x_flat,
                                 x_flat.requires_grad or topk_weights.requires_grad)
    out, sorted_w, counts, rev, offsets, slot_pos = _TokenPermute.apply(
        x_flat, topk_weights, topk_indices, int(num_experts), _validate_default(validate))
    return PermutedTokens(out, counts, rev, sorted_w, offsets, slot_pos)
