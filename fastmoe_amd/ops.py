"""Grouped pointer-indirection MoE combine: the operator API of fastmoe on gfx950 kernels.

Drop-in for ``fastmoe.kernels.ops`` (src/fastmoe/kernels/ops.py): the same public names,
argument meaning and return values --

    grouped_weighted_scatter_add(expert_tensors, indices, weights, out_shape, out=None,
                                 metadata=None)                        (ops.py:365-394)
    weighted_scatter_add(src, indices, weights, out_shape, out=None)   (ops.py:397-398)
    prepare_grouped_metadata(expert_tensors, device)                   (ops.py:200-271)
    GroupedWeightedScatterAdd.apply(indices, weights, out_shape, *expert_tensors)
                                                                       (ops.py:316-359)

    out[indices[g], :] += weights[g] * cat(expert_tensors)[g, :]

computed without concatenating: a device pointer table addresses every expert's own buffer.  All
work runs in ``libfastmoe_amd.so`` (HIP, gfx950) through its C ABI on the caller's current
stream; nothing here computes on the CPU, and there is no fallback: CPU tensors and a missing
library raise.

Differences from the reference, each deliberate:
  * CPU tensors raise instead of running torch's ``index_add_`` (ops.py:373-384).  That CPU
    algorithm lives in ``oracle/`` as the test checker.
  * The backward also returns the gate gradient when ``weights.requires_grad`` (the reference
    returns None, ops.py:358-359).
  * ``mode`` selects the forward kernel: "det" (default; token-major, fixed-order, bit-identical
    run to run), "atomic" (hardware fp32 atomics in packed-row order, like the reference's Triton
    kernel; a bf16/f16 output is accumulated in fp32 and rounded once) or "atomic_packed" (a
    bf16/f16 output takes packed 16-bit atomics directly, rounding at every add, as the Triton
    kernel does with a bf16 output).  ``FASTMOE_COMBINE_MODE`` sets the default when the module
    is imported.
  * Scatter indices outside [0, T) are dropped by the forward and get zero gradient instead of
    faulting; ``validate=True`` (or ``FASTMOE_VALIDATE=1``) raises IndexError for them at the cost
    of one device->host synchronisation.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
from typing import Optional, Sequence

import torch

from . import _abi

__all__ = [
    "GroupedMetadata",
    "GroupedWeightedScatterAdd",
    "build_plan",
    "build_plan_from_slots",
    "grouped_weighted_scatter_add",
    "prepare_grouped_metadata",
    "prepare_metadata_and_plan",
    "prepare_metadata_and_plan_from_slots",
    "weighted_scatter_add",
]

# Optional per-launch timer (bench.py installs one): an object with span(name) returning a
# context manager that brackets the C-ABI launch on the current stream.
_TIMER = None


_HOST = []


def _host():
    """The host helper module ``fastmoe_amd._host`` (built with the library); raises if missing."""
    if not _HOST:
        try:
            from . import _host as mod
        except ImportError as exc:
            raise _abi.FastMoEError(
                "fastmoe_amd: the host helper module fastmoe_amd._host is not built "
                "(run python -m fastmoe_amd.build)") from exc
        _HOST.append(mod)
    return _HOST[0]


def _span(name: str):
    timer = _TIMER
    return contextlib.nullcontext() if timer is None else timer.span(name)


_FLOAT_CODES = {torch.float32: _abi.F32, torch.bfloat16: _abi.BF16, torch.float16: _abi.F16}
_INDEX_CODES = {torch.int64: _abi.I64, torch.int32: _abi.I32}
_MODES = {"det": _abi.MODE_DET, "atomic": _abi.MODE_ATOMIC,
          "atomic_packed": _abi.MODE_ATOMIC_PACKED}

# Defaults of ``mode`` and ``validate``, read from the environment once, at import.
_DEFAULT_MODE = os.environ.get("FASTMOE_COMBINE_MODE", "det")
_DEFAULT_VALIDATE = os.environ.get("FASTMOE_VALIDATE", "0") not in ("", "0")


def _mode_code(mode: Optional[str]) -> int:
    name = (mode or _DEFAULT_MODE).lower()
    if name not in _MODES:
        raise ValueError(f"fastmoe_amd: unknown combine mode {name!r} "
                         f"(expected one of {sorted(_MODES)})")
    return _MODES[name]


def _validate_default(validate: Optional[bool]) -> bool:
    return _DEFAULT_VALIDATE if validate is None else bool(validate)


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch._C._cuda_getDevice()


def _stream_handle(device: torch.device) -> int:
    """The raw handle of ``device``'s current stream (every launch goes on it)."""
    return torch._C._cuda_getCurrentRawStream(_device_index(device))


def _on_device(device: torch.device):
    """``torch.cuda.device(device)``, or nothing when it is already the current device."""
    if torch._C._cuda_getDevice() == _device_index(device):
        return contextlib.nullcontext()
    return torch.cuda.device(device)


class _DeviceProbe:
    """Duck-types the ``is_cuda``/``device`` of a tensor for a bare device argument."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.is_cuda = self.device.type == "cuda"


def _require_cuda(t, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"fastmoe_amd: {what} is on {t.device}; the combine runs only on the GPU "
            "(the reference's CPU index_add_ path is the test oracle, not a product path)"
        )


class GroupedMetadata(tuple):
    """Device metadata of a list of ragged expert buffers.

    Unpacks like the reference's 5-tuple ``(ptr_table, chunk_sizes, expert_offsets, max_rows,
    num_experts)`` (ops.py:271) so code that passes it back as ``metadata=`` keeps working
    (run_on_cloud.py:67-81).  It also keeps references to the expert tensors, so the raw addresses
    in ``ptr_table`` stay valid as long as the metadata lives (a freed-and-reused buffer cannot be
    read through a stale table).
    """

    def __new__(cls, ptr_table, chunk_sizes, offsets_full, max_rows, num_experts, **extra):
        self = super().__new__(
            cls, (ptr_table, chunk_sizes, offsets_full[:num_experts], max_rows, num_experts)
        )
        ex = extra["experts"]
        self.offsets_full = offsets_full  # int64[E + 1], offsets_full[E] == N
        self.max_rows_device = extra["max_rows_device"]
        self.tensors = tuple(ex.tensors)
        self.sizes = tuple(ex.sizes)
        self.ptrs = tuple(ex.ptrs)
        self.table = bytes(ex.table)  # the packed (addresses, rows) this metadata describes
        self.hidden = ex.hidden
        self.dtype = ex.dtype
        self.device = ex.device
        self.num_rows = ex.rows
        return self

    # the reference tuple's fields by name
    ptr_table = property(lambda self: self[0])
    chunk_sizes = property(lambda self: self[1])
    expert_offsets = property(lambda self: self[2])
    max_rows = property(lambda self: self[3])
    num_experts = property(lambda self: self[4])

    def matches(self, expert_tensors: Sequence[torch.Tensor]) -> bool:
        """True if this metadata describes exactly these buffers: same addresses, rows, dtype,
        device and hidden size, each row-contiguous (a strided view of the same memory does not
        match)."""
        if len(expert_tensors) != len(self.ptrs):
            return False
        try:
            ex = _check_experts(expert_tensors)
        except (ValueError, TypeError, RuntimeError):
            return False
        return (ex.dtype == self.dtype and ex.device == self.device and ex.hidden == self.hidden
                and ex.table == self.table)


class _Experts:
    """Validated expert buffers (``_check_experts``): dtype, device, hidden size, total and largest
    row count, and ``table``, a bytearray of the E data addresses then the E row counts (int64),
    which the C ABI takes as its two host tables."""

    __slots__ = ("tensors", "dtype", "device", "hidden", "rows", "max_rows", "table", "num",
                 "versions")

    def __init__(self, tensors, dtype, device, hidden, rows, max_rows, table, versions):
        self.tensors, self.dtype, self.device, self.hidden = tensors, dtype, device, hidden
        self.rows, self.max_rows, self.table = rows, max_rows, table
        self.num = len(table) // 16
        self.versions = versions  # sum of the autograd version counters, if asked for

    @property
    def ptrs(self) -> list:
        return memoryview(self.table).cast("q")[: self.num].tolist()

    @property
    def sizes(self) -> list:
        return memoryview(self.table).cast("q")[self.num:].tolist()

    def host_tables(self) -> tuple:
        """(addresses, rows) as ctypes int64 arrays over ``table`` (they keep it alive)."""
        E = self.num
        return ((ctypes.c_int64 * E).from_buffer(self.table),
                (ctypes.c_int64 * E).from_buffer(self.table, 8 * E))


def _check_experts(expert_tensors: Sequence[torch.Tensor], versions: bool = False) -> _Experts:
    """Validate the expert buffers.

    Every buffer must be a 2-D [rows, D] tensor of one float dtype on one GPU, row-contiguous
    (``is_contiguous()`` on a 2-D tensor is exactly the layout the kernels address: strides (D, 1)
    for several rows, a unit column stride for one row, anything for no rows).  With hundreds of
    experts this runs on every call, so the per-tensor checks and the packing of the (address,
    rows) pairs run in C++ (``_host.experts``), which names the first offending buffer.
    """
    if len(expert_tensors) == 0:
        raise ValueError("fastmoe_amd: expert_tensors is empty")
    ref = expert_tensors[0]
    _require_cuda(ref, "expert_tensors[0]")
    if ref.dtype not in _FLOAT_CODES:
        raise TypeError(f"fastmoe_amd: unsupported expert dtype {ref.dtype}")
    hidden, rows, max_rows, table, vsum = _host().experts(expert_tensors, versions)
    return _Experts(expert_tensors, ref.dtype, ref.device, hidden, rows, max_rows, table, vsum)


_ELEM_BYTES = {torch.float32: 4, torch.bfloat16: 2, torch.float16: 2}


def _meta_layout(E: int, plan_bytes: int = 0):
    """One device workspace for the metadata arrays -- ptr_table int64[E], offsets int64[E + 1],
    chunk_sizes int32[E], max_rows int32[1] -- and, at the next 256-byte boundary, the plan of
    ``plan_bytes``: (byte offsets of offsets, chunk_sizes, max_rows, plan; total bytes).  torch's
    caching allocator returns 512-byte aligned blocks, so the plan is 256-byte aligned."""
    o_off = 8 * E
    o_chunk = o_off + 8 * (E + 1)
    o_max = o_chunk + 4 * E
    o_plan = (o_max + 4 + 255) & ~255
    return (o_off, o_chunk, o_max, o_plan), o_plan + plan_bytes


class _RawMeta:
    """Metadata (and optionally a plan) in one device workspace, as raw addresses for the C ABI;
    ``ws`` keeps the memory alive."""

    __slots__ = ("ws", "E", "offs", "ptr_table", "offsets", "chunk_sizes", "max_rows", "plan")

    def __init__(self, ex: _Experts, plan_bytes: int = 0):
        self.E = ex.num
        self.offs, total = _meta_layout(ex.num, plan_bytes)
        self.ws = torch.empty(total, dtype=torch.uint8, device=ex.device)
        base = self.ws.data_ptr()
        self.ptr_table = base
        self.offsets = base + self.offs[0]
        self.chunk_sizes = base + self.offs[1]
        self.max_rows = base + self.offs[2]
        self.plan = base + self.offs[3] if plan_bytes else None

    def plan_tensor(self) -> torch.Tensor:
        return self.ws[self.offs[3]:]

    def tensors(self):
        """(ptr_table, chunk_sizes, offsets, max_rows) as views of the workspace."""
        E, (o_off, o_chunk, o_max, _) = self.E, self.offs
        ws = self.ws
        return (ws[: 8 * E].view(torch.int64), ws[o_chunk: o_chunk + 4 * E].view(torch.int32),
                ws[o_off: o_off + 8 * (E + 1)].view(torch.int64),
                ws[o_max: o_max + 4].view(torch.int32))


def _new_metadata(ex: _Experts, m: _RawMeta) -> GroupedMetadata:
    ptr_table, chunk_sizes, offsets, max_rows_dev = m.tensors()
    return GroupedMetadata(ptr_table, chunk_sizes, offsets, ex.max_rows, ex.num,
                           max_rows_device=max_rows_dev, experts=ex)


def _plan_bytes(N: int, num_tokens: int) -> int:
    nbytes = _abi.lib().fmoe_plan_workspace_bytes(N, num_tokens)
    if nbytes <= 0:
        raise ValueError(f"fastmoe_amd: bad plan size N={N} T={num_tokens}")
    return nbytes


def _run_metadata(ex: _Experts, m: _RawMeta) -> None:
    """fmoe_build_metadata into ``m``."""
    ptrs, rows = ex.host_tables()
    dev = ex.device
    with _on_device(dev), _span("metadata"):
        rc = _abi.lib().fmoe_build_metadata(ptrs, rows, ex.num, m.ptr_table, m.chunk_sizes,
                                            m.offsets, m.max_rows, _stream_handle(dev))
    _abi.check(rc, "fmoe_build_metadata")


def _run_metadata_and_plan(ex: _Experts, m: _RawMeta, idx, w, num_tokens: int) -> None:
    """fmoe_build_metadata_and_plan into ``m``; idx and w already flat and checked."""
    ptrs, rows = ex.host_tables()
    dev = ex.device
    with _on_device(dev), _span("metadata_plan"):
        rc = _abi.lib().fmoe_build_metadata_and_plan(
            ptrs, rows, ex.num, m.ptr_table, m.chunk_sizes, m.offsets, m.max_rows,
            idx.data_ptr(), _INDEX_CODES[idx.dtype], w.data_ptr(), _FLOAT_CODES[w.dtype],
            num_tokens, ex.hidden * _ELEM_BYTES[ex.dtype], m.plan, _stream_handle(dev))
    _abi.check(rc, "fmoe_build_metadata_and_plan")


def _run_metadata_and_plan_from_slots(ex: _Experts, m: _RawMeta, slot_pos, w, num_tokens: int,
                                      top_k: int) -> None:
    """fmoe_build_metadata_and_plan_from_slots into ``m``; arguments already checked."""
    ptrs, rows = ex.host_tables()
    dev = ex.device
    with _on_device(dev), _span("metadata_plan"):
        rc = _abi.lib().fmoe_build_metadata_and_plan_from_slots(
            ptrs, rows, ex.num, m.ptr_table, m.chunk_sizes, m.offsets, m.max_rows,
            slot_pos.data_ptr(), num_tokens, top_k, w.data_ptr(), _FLOAT_CODES[w.dtype],
            ex.hidden * _ELEM_BYTES[ex.dtype], m.plan, _stream_handle(dev))
    _abi.check(rc, "fmoe_build_metadata_and_plan_from_slots")


def prepare_grouped_metadata(expert_tensors: Sequence[torch.Tensor], device=None) -> GroupedMetadata:
    """Pointer table, row counts, exclusive offsets and max_rows of the expert buffers.

    Mirrors prepare_grouped_metadata (src/fastmoe/kernels/ops.py:200-271).  The table is built on
    the device by one kernel launch whose arguments carry the (address, rows) pairs
    (``fmoe_build_metadata``): no host staging buffer and no synchronous copy.
    """
    ex = _check_experts(expert_tensors)
    if device is not None:
        _require_cuda(_DeviceProbe(device), "device")
    return _metadata(ex)


def _metadata(ex: _Experts) -> GroupedMetadata:
    m = _RawMeta(ex)
    _run_metadata(ex, m)
    return _new_metadata(ex, m)


def _routing_args(indices: torch.Tensor, weights: torch.Tensor, num_rows: int, dev):
    _require_cuda(indices, "indices")
    _require_cuda(weights, "weights")
    if indices.device != dev or weights.device != dev:
        raise ValueError("fastmoe_amd: indices/weights must be on the experts' device")
    if indices.dtype not in _INDEX_CODES:
        raise TypeError(f"fastmoe_amd: indices must be int64 or int32, got {indices.dtype}")
    if weights.dtype not in _FLOAT_CODES:
        raise TypeError(f"fastmoe_amd: unsupported weights dtype {weights.dtype}")
    if indices.numel() != num_rows or weights.numel() != num_rows:
        raise ValueError(
            f"fastmoe_amd: len(indices)={indices.numel()} and len(weights)={weights.numel()} must "
            f"equal the total expert rows {num_rows}"
        )
    return indices.reshape(-1).contiguous(), weights.reshape(-1).contiguous()


def _check_plan_status(plan: torch.Tensor, num_tokens: int) -> None:
    bad = int(plan_status(plan)[0])
    if bad:
        raise IndexError(f"fastmoe_amd: {bad} scatter indices lie outside [0, {num_tokens})")


def _build_plan_raw(ptr_table: int, offsets_full: int, E: int, N: int, row_bytes: int, idx, w,
                    num_tokens: int, dev) -> torch.Tensor:
    """fmoe_build_plan into a new workspace (returned); the metadata arrays given by address, idx
    and w already flat and checked."""
    ws = torch.empty(_plan_bytes(N, num_tokens), dtype=torch.uint8, device=dev)
    with _on_device(dev), _span("plan"):
        rc = _abi.lib().fmoe_build_plan(
            idx.data_ptr(), _INDEX_CODES[idx.dtype], w.data_ptr(), _FLOAT_CODES[w.dtype], N,
            num_tokens, ptr_table, offsets_full, E, row_bytes, ws.data_ptr(), _stream_handle(dev),
        )
    _abi.check(rc, "fmoe_build_plan")
    return ws


def build_plan(meta: GroupedMetadata, indices: torch.Tensor, weights: torch.Tensor,
               num_tokens: int, validate: Optional[bool] = None) -> torch.Tensor:
    """Token-major inverse of ``indices`` (``fmoe_build_plan``) as an opaque uint8 device tensor.

    The deterministic forward and the backward read it.  With ``validate`` it synchronises once
    and raises IndexError if any index lies outside [0, num_tokens).
    """
    N = meta.num_rows
    idx, w = _routing_args(indices, weights, N, meta.device)
    ws = _build_plan_raw(meta.ptr_table.data_ptr(), meta.offsets_full.data_ptr(), len(meta.sizes),
                         N, meta.hidden * _ELEM_BYTES[meta.dtype], idx, w, num_tokens, meta.device)
    if _validate_default(validate):
        _check_plan_status(ws, num_tokens)
    return ws


def prepare_metadata_and_plan(expert_tensors: Sequence[torch.Tensor], indices: torch.Tensor,
                              weights: torch.Tensor, num_tokens: int,
                              validate: Optional[bool] = None):
    """``prepare_grouped_metadata`` followed by ``build_plan`` in one C-ABI call
    (``fmoe_build_metadata_and_plan``: the plan's own launches write the metadata for up to 256
    experts); returns ``(metadata, plan)``, each exactly what the two calls return."""
    ex = _check_experts(expert_tensors)
    idx, w = _routing_args(indices, weights, ex.rows, ex.device)
    return _metadata_and_plan(ex, idx, w, num_tokens, validate)


def _metadata_and_plan(ex: _Experts, idx, w, num_tokens, validate):
    """idx and w already flat and checked (_routing_args)."""
    m = _RawMeta(ex, _plan_bytes(ex.rows, num_tokens))
    _run_metadata_and_plan(ex, m, idx, w, num_tokens)
    plan = m.plan_tensor()
    if _validate_default(validate):
        _check_plan_status(plan, num_tokens)
    return _new_metadata(ex, m), plan


def _check_slots(slot_pos, weights, N: int, num_tokens: int, top_k: int, dev):
    if N != num_tokens * top_k or not (1 <= top_k <= 64):
        raise ValueError(f"fastmoe_amd: a slot plan needs rows == T*k and k <= 64 "
                         f"(rows {N}, T {num_tokens}, k {top_k})")
    if slot_pos.dtype != torch.int32 or slot_pos.numel() != N or slot_pos.device != dev:
        raise ValueError("fastmoe_amd: slot_pos must be int32 [T*k] on the experts' device")
    w = weights.reshape(-1).contiguous()
    if w.dtype not in _FLOAT_CODES or w.numel() != N:
        raise ValueError("fastmoe_amd: weights must be a float [T*k] tensor")
    return slot_pos.contiguous(), w


def _build_plan_from_slots_raw(ptr_table: int, offsets_full: int, E: int, N: int, row_bytes: int,
                               slot_pos, w, num_tokens: int, top_k: int, dev) -> torch.Tensor:
    ws = torch.empty(_plan_bytes(N, num_tokens), dtype=torch.uint8, device=dev)
    with _on_device(dev), _span("plan"):
        rc = _abi.lib().fmoe_build_plan_from_slots(
            slot_pos.data_ptr(), num_tokens, top_k, w.data_ptr(), _FLOAT_CODES[w.dtype],
            ptr_table, offsets_full, E, N, row_bytes, ws.data_ptr(), _stream_handle(dev),
        )
    _abi.check(rc, "fmoe_build_plan_from_slots")
    return ws


def build_plan_from_slots(meta: GroupedMetadata, slot_pos: torch.Tensor, weights: torch.Tensor,
                          num_tokens: int, top_k: int) -> torch.Tensor:
    """The plan of a combine fed by the dispatch permutation (``fmoe_build_plan_from_slots``).

    ``slot_pos`` is the permutation's int32 slot -> packed-row map; token t's rows are
    ``slot_pos[t * top_k : (t + 1) * top_k]``.  Requires every slot to be a row of the combine
    (``meta.num_rows == num_tokens * top_k``) and ``top_k <= 64``.  Same layout as build_plan.
    """
    N = meta.num_rows
    sp, w = _check_slots(slot_pos, weights, N, num_tokens, top_k, meta.device)
    return _build_plan_from_slots_raw(meta.ptr_table.data_ptr(), meta.offsets_full.data_ptr(),
                                      len(meta.sizes), N, meta.hidden * _ELEM_BYTES[meta.dtype],
                                      sp, w, num_tokens, top_k, meta.device)


def prepare_metadata_and_plan_from_slots(expert_tensors: Sequence[torch.Tensor],
                                         slot_pos: torch.Tensor, weights: torch.Tensor,
                                         num_tokens: int, top_k: int):
    """``prepare_grouped_metadata`` followed by ``build_plan_from_slots`` in one C-ABI call
    (``fmoe_build_metadata_and_plan_from_slots``: one kernel launch for up to 256 experts);
    returns ``(metadata, plan)``."""
    return _metadata_and_plan_from_slots(_check_experts(expert_tensors), slot_pos, weights,
                                         num_tokens, top_k)


def _metadata_and_plan_from_slots(ex: _Experts, slot_pos, weights, num_tokens, top_k):
    sp, w = _check_slots(slot_pos, weights, ex.rows, num_tokens, top_k, ex.device)
    m = _RawMeta(ex, _plan_bytes(ex.rows, num_tokens))
    _run_metadata_and_plan_from_slots(ex, m, sp, w, num_tokens, top_k)
    return _new_metadata(ex, m), m.plan_tensor()


def invert_scatter_index(indices: torch.Tensor, num_tokens: int):
    """The token-major inverse of ``indices`` as a CSR (``fmoe_invert_scatter_index``).

    Returns ``(row_ptr, rows)``, int32 device tensors of T + 2 and N entries: token t's packed
    rows are ``rows[row_ptr[t]:row_ptr[t + 1]]`` in ascending order, and segment T holds the rows
    whose index lies outside [0, num_tokens).  Equal to a stable argsort of ``indices`` (with
    out-of-range indices mapped to T) and the exclusive prefix of its bincount.
    """
    lib = _abi.lib()
    _require_cuda(indices, "indices")
    if indices.dtype not in _INDEX_CODES:
        raise TypeError(f"fastmoe_amd: indices must be int64 or int32, got {indices.dtype}")
    if num_tokens < 1:
        raise ValueError(f"fastmoe_amd: num_tokens must be >= 1, got {num_tokens}")
    idx = indices.reshape(-1).contiguous()
    N, dev = idx.numel(), idx.device
    row_ptr = torch.empty(num_tokens + 2, dtype=torch.int32, device=dev)
    rows = torch.empty(N, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.fmoe_plan_workspace_bytes(N, num_tokens), dtype=torch.uint8, device=dev)
    with _on_device(dev), _span("invert_scatter_index"):
        rc = lib.fmoe_invert_scatter_index(
            idx.data_ptr(), _INDEX_CODES[idx.dtype], N, num_tokens, row_ptr.data_ptr(),
            rows.data_ptr(), ws.data_ptr(), _stream_handle(dev),
        )
    _abi.check(rc, "fmoe_invert_scatter_index")
    return row_ptr, rows


def plan_status(plan: torch.Tensor) -> torch.Tensor:
    """The plan's int32 status words [invalid_index_count, misaligned_flag, longest_segment]
    (a device view).  longest_segment counts the rows of the busiest token when the plan was built
    by the bucketed or radix plan or from a slot map, and is -1 for the one-launch and ranged
    plans, whose workgroups never see every segment in one place."""
    off = _abi.lib().fmoe_plan_status_offset()
    return plan[off: off + 12].view(torch.int32)


def _check_out(out: torch.Tensor, num_tokens_hint, hidden: int, dev) -> None:
    _require_cuda(out, "out")
    if out.device != dev:
        raise ValueError("fastmoe_amd: out must be on the experts' device")
    if out.dtype not in _FLOAT_CODES:
        raise TypeError(f"fastmoe_amd: unsupported out dtype {out.dtype}")
    if out.dim() != 2 or out.shape[1] != hidden:
        raise ValueError(f"fastmoe_amd: out must be [T, {hidden}], got {tuple(out.shape)}")
    if hidden > 1 and out.stride(1) != 1:
        raise ValueError("fastmoe_amd: out must have unit column stride")
    if out.shape[0] > 1 and out.stride(0) < hidden:
        raise ValueError("fastmoe_amd: out rows overlap")


def _launch_fwd_raw(mode: int, plan: Optional[int], idx: Optional[torch.Tensor],
                    w: Optional[torch.Tensor], ptr_table: int, offsets_full: int, E: int, N: int,
                    x_dtype: torch.dtype, out: torch.Tensor, accumulate: bool) -> None:
    """fmoe_combine_fwd; the plan and the metadata arrays given by address."""
    lib = _abi.lib()
    T, D = out.shape
    dev = out.device
    out_code = _FLOAT_CODES[out.dtype]
    ws, ws_bytes = None, 0
    if mode == _abi.MODE_ATOMIC and out_code != _abi.F32:
        # the fp32 accumulator of a 16-bit output (fmoe_combine_fwd_workspace_bytes)
        ws_bytes = lib.fmoe_combine_fwd_workspace_bytes(mode, T, D, out_code)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    name = "fwd_det" if mode == _abi.MODE_DET else "fwd_atomic"
    with _on_device(dev), _span(name):
        rc = lib.fmoe_combine_fwd(
            mode, plan,
            idx.data_ptr() if idx is not None else None,
            _INDEX_CODES[idx.dtype] if idx is not None else _abi.I64,
            w.data_ptr() if w is not None else None,
            _FLOAT_CODES[w.dtype] if w is not None else _abi.F32,
            ptr_table, offsets_full, E, N, T, D, _FLOAT_CODES[x_dtype], out.data_ptr(), out_code,
            out.stride(0) if T > 1 else D, 1 if accumulate else 0,
            ws.data_ptr() if ws is not None else None, ws_bytes, _stream_handle(dev),
        )
    _abi.check(rc, "fmoe_combine_fwd")


def _launch_fwd(meta: GroupedMetadata, mode: int, plan: Optional[torch.Tensor],
                idx: Optional[torch.Tensor], w: Optional[torch.Tensor], out: torch.Tensor,
                accumulate: bool) -> None:
    """fmoe_combine_fwd from a GroupedMetadata and a plan tensor."""
    _launch_fwd_raw(mode, plan.data_ptr() if plan is not None else None, idx, w,
                    meta.ptr_table.data_ptr(), meta.offsets_full.data_ptr(), len(meta.sizes),
                    meta.num_rows, meta.dtype, out, accumulate)


# The one-launch small path (fmoe_combine_fwd_small / fmoe_combine_bwd_small): deterministic calls
# of at most fmoe_combine_small_max_rows() rows over at most 256 experts, with no plan.  A training
# step is two launches instead of four (metadata + plan, forward, grad_X pass, grad_w pass), and a
# forward saves the plan's dependent launch.  Each forward wave scans the token id of every row, so
# the cost grows with T * N: it is taken while T * N <= _SMALL_SCAN_LIMIT (graph-replayed steps on
# one MI355X, planned -> small: fwd+bwd 17.6 -> 15.3 us at T=256, D=512, top-2, fp32 and 24.3 ->
# 18.9 us at T=64, D=7168, top-8, bf16; forward 19.0 -> 14.8 us at T=128, D=16384, top-8; past
# the limit, fwd+bwd 31.9 -> 33.7 us at T=256, D=7168, top-8).
_SMALL_MAX_EXPERTS = 256
_SMALL_SCAN_LIMIT = 1 << 17
_SMALL_MAX_ROWS: list = []


def _use_small(rows: int, num_tokens: int, num_experts: int) -> bool:
    choice = _abi.option("small")
    if choice == 1 or _abi.option("plan") != 0 or num_experts > _SMALL_MAX_EXPERTS or rows < 1:
        return False
    if not _SMALL_MAX_ROWS:
        _SMALL_MAX_ROWS.append(int(_abi.lib().fmoe_combine_small_max_rows()))
    if rows > _SMALL_MAX_ROWS[0]:
        return False
    return choice == 2 or rows * num_tokens <= _SMALL_SCAN_LIMIT


def _launch_fwd_small(tables, num_experts: int, idx: torch.Tensor, w: torch.Tensor,
                      x_dtype: torch.dtype, out: torch.Tensor, accumulate: bool) -> torch.Tensor:
    """fmoe_combine_fwd_small into ``out``; returns its status word (rows with an index outside
    [0, T)) on the device."""
    T, D = out.shape
    status = torch.empty(1, dtype=torch.int32, device=out.device)
    with _on_device(out.device), _span("fwd_small"):
        rc = _abi.lib().fmoe_combine_fwd_small(
            tables[0], tables[1], num_experts, idx.data_ptr(), _INDEX_CODES[idx.dtype],
            w.data_ptr(), _FLOAT_CODES[w.dtype], T, D, _FLOAT_CODES[x_dtype], out.data_ptr(),
            _FLOAT_CODES[out.dtype], out.stride(0) if T > 1 else D, 1 if accumulate else 0,
            status.data_ptr(), _stream_handle(out.device))
    _abi.check(rc, "fmoe_combine_fwd_small")
    return status


def _check_small_status(status: torch.Tensor, num_tokens: int) -> None:
    bad = int(status[0])
    if bad:
        raise IndexError(f"fastmoe_amd: {bad} scatter indices lie outside [0, {num_tokens})")


def _launch_grouped_kernel(expert_tensors, indices, weights, out, metadata=None, *, mode=None,
                           validate=None):
    """In-place combine into ``out`` (accumulates; mirrors ops.py:277-310)."""
    code = _mode_code(mode)
    T = out.shape[0]
    plan = None
    if isinstance(metadata, GroupedMetadata) and metadata.matches(expert_tensors):
        idx, w = _routing_args(indices, weights, metadata.num_rows, metadata.device)
    else:
        ex = _check_experts(expert_tensors)
        idx, w = _routing_args(indices, weights, ex.rows, ex.device)
        # The small path counts out-of-range indices in the same launch that accumulates into
        # ``out``; a validating call takes the planned path, which raises before any forward
        # launch, so ``out`` is left untouched when it raises.
        if (code == _abi.MODE_DET and not _validate_default(validate)
                and _use_small(ex.rows, T, ex.num)):
            _check_out(out, None, ex.hidden, ex.device)
            _launch_fwd_small(ex.host_tables(), ex.num, idx, w, ex.dtype, out, accumulate=True)
            return out
        if code == _abi.MODE_DET and ex.rows > 0:
            metadata, plan = _metadata_and_plan(ex, idx, w, T, validate)
        else:
            metadata = _metadata(ex)
    _check_out(out, None, metadata.hidden, metadata.device)
    if metadata.max_rows == 0:  # ops.py:286: nothing to add
        return out
    if code == _abi.MODE_DET:
        if plan is None:
            plan = build_plan(metadata, idx, w, T, validate)
        _launch_fwd(metadata, code, plan, None, None, out, accumulate=True)
    else:
        if _validate_default(validate):
            build_plan(metadata, idx, w, T, True)
        _launch_fwd(metadata, code, None, idx, w, out, accumulate=True)
    return out


def _combine_forward(ctx, mode: Optional[str], validate: Optional[bool], indices, weights,
                     out_shape, expert_tensors, w_grad: bool, slots=None):
    """Autograd forward.  ``w_grad``: the gate gradient will be asked for.  The backward then
    reads the expert buffers through the addresses in the plan (or the small path's tables), so
    the forward keeps the tensors on ``ctx`` with the sum of their version counters, and the
    backward refuses buffers modified in place since (torch's check of saved tensors).  They are
    not passed through ``save_for_backward``: unpacking hundreds of saved tensors in every
    backward costs more host time than the rest of the call (the reference saves only the index
    and gates, ops.py:326, and needs no expert data in its backward)."""
    ex = _check_experts(expert_tensors, w_grad)
    dtype, dev, hidden = ex.dtype, ex.device, ex.hidden
    shape = tuple(int(s) for s in out_shape)
    if len(shape) != 2 or shape[1] != hidden:
        raise ValueError(f"fastmoe_amd: out_shape {shape} must be [T, {hidden}]")
    T = shape[0]
    code = _mode_code(mode)
    rows = ex.rows
    idx, w = _routing_args(indices, weights, rows, dev)
    use_slots = slots is not None and rows == T * slots[1] and slots[1] <= 64
    meta = small = None
    if rows == 0:
        meta = _RawMeta(ex)
        _run_metadata(ex, meta)
        out = torch.zeros(shape, dtype=dtype, device=dev)
    elif code == _abi.MODE_DET and _use_small(rows, T, ex.num):
        # one launch, no plan; the backward is one launch too
        small = ex.host_tables()
        out = torch.empty(shape, dtype=dtype, device=dev)
        status = _launch_fwd_small(small, ex.num, idx, w, dtype, out, accumulate=False)
        if _validate_default(validate):
            _check_small_status(status, T)
    elif code == _abi.MODE_DET:
        # metadata and plan in one workspace and one call; every output row is written exactly
        # once (tokens without rows get zeros), so out needs no zero-fill
        meta = _RawMeta(ex, _plan_bytes(rows, T))
        if use_slots:
            sp, w = _check_slots(slots[0], w, rows, T, slots[1], dev)
            _run_metadata_and_plan_from_slots(ex, meta, sp, w, T, slots[1])
        else:
            _run_metadata_and_plan(ex, meta, idx, w, T)
            if _validate_default(validate):
                _check_plan_status(meta.plan_tensor(), T)
        out = torch.empty(shape, dtype=dtype, device=dev)
        _launch_fwd_raw(code, meta.plan, None, None, meta.ptr_table, meta.offsets, ex.num, rows,
                        dtype, out, accumulate=False)
    else:
        # the atomic forward reads no plan: the backward builds it if a gradient is asked for
        meta = _RawMeta(ex)
        _run_metadata(ex, meta)
        if _validate_default(validate):
            _check_plan_status(_build_plan_raw(meta.ptr_table, meta.offsets, ex.num, rows,
                                               hidden * _ELEM_BYTES[dtype], idx, w, T, dev), T)
        out = torch.empty(shape, dtype=dtype, device=dev)  # overwritten: the library clears it
        _launch_fwd_raw(code, None, idx, w, meta.ptr_table, meta.offsets, ex.num, rows, dtype,
                        out, accumulate=False)
    ctx.save_for_backward(idx, w)
    ctx.experts = tuple(expert_tensors) if w_grad else None
    ctx.x_version = ex.versions
    ctx.meta = meta    # metadata and plan workspace (None on the small path)
    ctx.small = small  # the small path's host tables
    ctx.slots = (slots[0], slots[1]) if use_slots else None
    ctx.sizes = ex.sizes
    ctx.hidden = hidden
    ctx.num_tokens = T
    ctx.x_dtype = dtype
    ctx.w_shape = weights.shape
    return out


def _combine_backward(ctx, grad_output, needs_w: bool, needs_x: Sequence[bool]):
    idx, w = ctx.saved_tensors
    sizes = ctx.sizes
    need_x = any(needs_x)
    N, T, D = idx.numel(), ctx.num_tokens, ctx.hidden
    dev = idx.device
    if not (needs_w or need_x):
        return None, [None] * len(sizes)
    if needs_w and ctx.experts is not None and _host().versions(ctx.experts) != ctx.x_version:
        raise RuntimeError(
            "fastmoe_amd: an expert tensor needed for the gate gradient has been modified by an "
            "inplace operation since the forward")
    if N == 0:
        gw = torch.zeros(ctx.w_shape, dtype=w.dtype, device=dev) if needs_w else None
        gx = [torch.zeros((n, D), dtype=ctx.x_dtype, device=dev) if need else None
              for n, need in zip(sizes, needs_x)]
        return gw, gx
    small = ctx.small
    meta = ctx.meta
    plan_ws = None
    if small is not None:
        plan = None
    elif meta.plan is not None:
        plan = meta.plan
    else:  # atomic forward: the plan now
        row_bytes = D * _ELEM_BYTES[ctx.x_dtype]
        if ctx.slots is not None:
            sp, ws_w = _check_slots(ctx.slots[0], w, N, T, ctx.slots[1], dev)
            plan_ws = _build_plan_from_slots_raw(meta.ptr_table, meta.offsets, meta.E, N,
                                                 row_bytes, sp, ws_w, T, ctx.slots[1], dev)
        else:
            plan_ws = _build_plan_raw(meta.ptr_table, meta.offsets, meta.E, N, row_bytes, idx, w,
                                      T, dev)
        plan = plan_ws.data_ptr()
    go = grad_output
    if go.dtype != ctx.x_dtype:
        go = go.to(ctx.x_dtype)
    if D > 1 and go.stride(1) != 1:
        go = go.contiguous()
    gx = torch.empty((N, D), dtype=ctx.x_dtype, device=dev) if need_x else None
    gw = torch.empty(N, dtype=w.dtype, device=dev) if needs_w else None
    lib = _abi.lib()
    stream = _stream_handle(dev)
    x_code, g_code, w_code = _FLOAT_CODES[ctx.x_dtype], _FLOAT_CODES[go.dtype], _FLOAT_CODES[w.dtype]
    g_stride = go.stride(0) if T > 1 else D
    gx_ptr = gx.data_ptr() if gx is not None else None
    gw_ptr = gw.data_ptr() if gw is not None else None
    with _on_device(dev):
        if small is not None:
            # both gradients (or either) in one launch, no plan
            with _span("bwd_small"):
                rc = lib.fmoe_combine_bwd_small(
                    small[0], small[1], len(sizes), idx.data_ptr(), _INDEX_CODES[idx.dtype],
                    w.data_ptr(), w_code, T, D, x_code, go.data_ptr(), g_code, g_stride, gx_ptr,
                    gw_ptr, w_code, stream)
            _abi.check(rc, "fmoe_combine_bwd_small")
        elif gx_ptr and gw_ptr and _TIMER is not None and not _abi.option("bwd_fused"):
            # Timed: the grad_X (write) and grad_w (read) passes, one call each -- the same two
            # launches fmoe_combine_bwd makes when given both outputs, issued separately so that
            # each gets its own span.
            for name, a, b in (("bwd_gx", gx_ptr, None), ("bwd_gw", None, gw_ptr)):
                with _span(name):
                    rc = lib.fmoe_combine_bwd(plan, N, T, D, x_code, go.data_ptr(), g_code,
                                              g_stride, a, b, w_code, stream)
                _abi.check(rc, "fmoe_combine_bwd")
        else:
            name = "bwd" if gx_ptr and gw_ptr else ("bwd_gx" if gx_ptr else "bwd_gw")
            with _span(name):
                rc = lib.fmoe_combine_bwd(plan, N, T, D, x_code, go.data_ptr(), g_code, g_stride,
                                          gx_ptr, gw_ptr, w_code, stream)
            _abi.check(rc, "fmoe_combine_bwd")
    if need_x:
        parts = torch.split(gx, sizes)
        grads_x = parts if all(needs_x) else [p if n else None for p, n in zip(parts, needs_x)]
    else:
        grads_x = [None] * len(sizes)
    return (gw.view(ctx.w_shape) if gw is not None else None), grads_x


def _apply(fn, *args):
    """``fn.apply(*args)`` (one place for every autograd entry of the combine), refused under HIP
    graph capture when it would record a backward (see _refuse_autograd_capture)."""
    probe = next(a for a in args if isinstance(a, torch.Tensor))
    if _capturing(probe) and torch.is_grad_enabled():
        _refuse_autograd_capture("the autograd combine", probe, _records_backward(args))
    return fn.apply(*args)


def _records_backward(args) -> bool:
    return any(isinstance(a, torch.Tensor) and a.requires_grad for a in args)


def _capturing(t: torch.Tensor) -> bool:
    """Whether ``t`` is a GPU tensor and the current stream is capturing a HIP graph."""
    return t.is_cuda and torch.cuda.is_current_stream_capturing()


def _refuse_autograd_capture(what: str, t: torch.Tensor, recording: bool = True) -> None:
    """Raise instead of recording an autograd step into a HIP graph.

    One capture of a whole autograd step (this forward and ``torch.autograd.grad``, whose backward
    runs on the autograd engine's device thread) inside ``torch.cuda.graph`` ended in a host
    segmentation fault in ``CUDAGraph.capture_end``, with no GPU fault, and no cause has been shown
    in this package's code.  Until one is, that capture is refused with this error rather than
    risked.  Captures that do not go through the engine stay supported and tested: the in-place
    call (``out=``, run_on_cloud.py:66-92) and the autograd forward under ``torch.no_grad()``.
    """
    if recording and _capturing(t):
        raise RuntimeError(
            f"fastmoe_amd: {what} under HIP graph capture is not supported (a captured autograd "
            "step once crashed the host in CUDAGraph.capture_end).  Capture the in-place call "
            "(grouped_weighted_scatter_add(..., out=..., metadata=...)) or run the autograd step "
            "eagerly.")


class GroupedWeightedScatterAdd(torch.autograd.Function):
    """Autograd bridge (mirrors src/fastmoe/kernels/ops.py:316-359).

    forward : out = zeros(out_shape, dtype=experts[0].dtype) + combine   (ops.py:317-331)
    backward: grad_X_e = split(grad_out[indices] * weights[:, None])     (ops.py:333-353)
              plus grad_weights[g] = <grad_out[indices[g]], X[g]>  when weights require grad.
    Both directions share one plan (token-major inverse of the indices), built in the forward
    (deterministic mode) or in the backward (atomic modes, whose forward does not read it).
    The forward kernel is chosen by ``FASTMOE_COMBINE_MODE`` ("det" by default).
    """

    @staticmethod
    def forward(ctx, indices, weights, out_shape, *expert_tensors):
        return _combine_forward(ctx, None, None, indices, weights, out_shape, expert_tensors,
                                ctx.needs_input_grad[1])

    @staticmethod
    def backward(ctx, grad_output):
        _refuse_autograd_capture("the combine's backward", grad_output)
        gw, gx = _combine_backward(ctx, grad_output, ctx.needs_input_grad[1],
                                   ctx.needs_input_grad[3:])
        return (None, gw, None, *gx)


class _GroupedCombineWithOptions(torch.autograd.Function):
    """Same as GroupedWeightedScatterAdd with an explicit (mode, validate) first argument."""

    @staticmethod
    def forward(ctx, options, indices, weights, out_shape, *expert_tensors):
        mode, validate = options
        return _combine_forward(ctx, mode, validate, indices, weights, out_shape, expert_tensors,
                                ctx.needs_input_grad[2])

    @staticmethod
    def backward(ctx, grad_output):
        _refuse_autograd_capture("the combine's backward", grad_output)
        gw, gx = _combine_backward(ctx, grad_output, ctx.needs_input_grad[2],
                                   ctx.needs_input_grad[4:])
        return (None, None, gw, None, *gx)


class _GroupedCombinePermuted(torch.autograd.Function):
    """GroupedWeightedScatterAdd for a scatter index produced by the dispatch permutation: the
    plan comes from the permutation's slot map (first argument: (slot_pos, top_k))."""

    @staticmethod
    def forward(ctx, slots, indices, weights, out_shape, *expert_tensors):
        return _combine_forward(ctx, None, None, indices, weights, out_shape, expert_tensors,
                                ctx.needs_input_grad[2], slots=slots)

    @staticmethod
    def backward(ctx, grad_output):
        _refuse_autograd_capture("the combine's backward", grad_output)
        gw, gx = _combine_backward(ctx, grad_output, ctx.needs_input_grad[2],
                                   ctx.needs_input_grad[4:])
        return (None, None, gw, None, *gx)


def grouped_weighted_scatter_add(expert_tensors, indices, weights, out_shape, out=None,
                                 metadata=None, *, mode=None, validate=None):
    """Public entry point (mirrors src/fastmoe/kernels/ops.py:365-394).

    * ``out`` given: accumulate into it in place, outside autograd (graph-capturable; ops.py:389).
    * otherwise: autograd path, returns a new ``[T, D]`` tensor in the experts' dtype (ops.py:394).
    CPU tensors raise (see the module docstring).
    """
    _require_cuda(indices, "indices")
    if out is not None:
        return _launch_grouped_kernel(expert_tensors, indices, weights, out, metadata=metadata,
                                      mode=mode, validate=validate)
    if mode is None and validate is None:
        return _apply(GroupedWeightedScatterAdd, indices, weights, out_shape, *expert_tensors)
    return _apply(_GroupedCombineWithOptions, (mode, validate), indices, weights, out_shape,
                  *expert_tensors)


def weighted_scatter_add(src, indices, weights, out_shape, out=None, *, mode=None, validate=None):
    """Single-tensor form (mirrors src/fastmoe/kernels/ops.py:397-398)."""
    return grouped_weighted_scatter_add([src], indices, weights, out_shape, out, mode=mode,
                                        validate=validate)
