"""The reference-side binding, run as a fastmoe maintainer would write it.

fastmoe is Python, so its FFI to this library is ctypes.  The functions below are the binding
that would replace the Triton launch (src/fastmoe/kernels/ops.py:277-310) and the torch backward
(ops.py:333-359) inside the reference's own module: a raw ``ctypes.CDLL`` of the library with the
argument types of ``include/fastmoe_amd.h``, torch tensors for every buffer, and no use of this
package's Python layer.  Each call's result is held to the C oracle (forward and grad_X bit for
bit, grad_w within 1e-6 of sum|terms|).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from fastmoe_amd import _abi
from tests.helpers import abs_dot, bits, oracle_bwd, oracle_fwd, to_np

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

# ---- the binding (ops.py of the reference would hold these lines; loaded on first use here, so
# that collecting this module needs no built library) -----------------------------------------
_L = None
_vp, _i64, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int


def _load():
    global _L
    _L = ctypes.CDLL(str(_abi.LIB_PATH))
    _L.fmoe_last_error.restype = ctypes.c_char_p
    _L.fmoe_plan_workspace_bytes.restype = _i64
    _L.fmoe_plan_workspace_bytes.argtypes = [_i64, _i64]
    _L.fmoe_build_metadata_and_plan.argtypes = [ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i64,
                                                _vp, _vp, _vp, _vp, _vp, _int, _vp, _int, _i64,
                                                _i64, _vp, _vp]
    _L.fmoe_combine_fwd.argtypes = [_int, _vp, _vp, _int, _vp, _int, _vp, _vp, _i64, _i64, _i64,
                                    _i64, _int, _vp, _int, _i64, _int, _vp, _i64, _vp]
    _L.fmoe_combine_bwd.argtypes = [_vp, _i64, _i64, _i64, _int, _vp, _int, _i64, _vp, _vp, _int,
                                    _vp]


_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int64: 3, torch.int32: 4}
DET = 0


def _ok(rc):
    if rc != 0:
        raise RuntimeError(_L.fmoe_last_error().decode())


def _plan(expert_tensors, indices, weights, T):
    dev, E = indices.device, len(expert_tensors)
    s = torch.cuda.current_stream(dev).cuda_stream
    rows = [t.shape[0] for t in expert_tensors]
    ptrs = [t.data_ptr() if n else 0 for t, n in zip(expert_tensors, rows)]
    ptr_table = torch.empty(E, dtype=torch.int64, device=dev)
    sizes = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int64, device=dev)
    max_rows = torch.empty(1, dtype=torch.int32, device=dev)
    N = sum(rows)
    ws = torch.empty(_L.fmoe_plan_workspace_bytes(N, T), dtype=torch.uint8, device=dev)
    row_bytes = expert_tensors[0].shape[1] * expert_tensors[0].element_size()
    _ok(_L.fmoe_build_metadata_and_plan((_i64 * E)(*ptrs), (_i64 * E)(*rows), E,
                                        ptr_table.data_ptr(), sizes.data_ptr(), offsets.data_ptr(),
                                        max_rows.data_ptr(), indices.data_ptr(),
                                        _CODE[indices.dtype], weights.data_ptr(),
                                        _CODE[weights.dtype], T, row_bytes, ws.data_ptr(), s))
    return ws, N


def _launch_grouped_kernel(expert_tensors, indices, weights, out, metadata=None):
    T, D = out.shape
    ws, N = _plan(expert_tensors, indices, weights, T)
    if N:
        _ok(_L.fmoe_combine_fwd(DET, ws.data_ptr(), None, 3, None, 0, None, None, 0, N, T, D,
                                _CODE[expert_tensors[0].dtype], out.data_ptr(), _CODE[out.dtype],
                                out.stride(0), 1, None, 0,
                                torch.cuda.current_stream().cuda_stream))
    return out, ws


def _backward(ws, N, T, D, x_dtype, weights, grad_output, expert_sizes):
    if D > 1 and grad_output.stride(1) != 1:  # rows are read with a unit column stride
        grad_output = grad_output.contiguous()
    gx = torch.empty((N, D), dtype=x_dtype, device=grad_output.device)
    gw = torch.empty(N, dtype=weights.dtype, device=grad_output.device)
    _ok(_L.fmoe_combine_bwd(ws.data_ptr(), N, T, D, _CODE[x_dtype], grad_output.data_ptr(),
                            _CODE[grad_output.dtype], grad_output.stride(0), gx.data_ptr(),
                            gw.data_ptr(), _CODE[gw.dtype], torch.cuda.current_stream().cuda_stream))
    return None, gw, None, *torch.split(gx, expert_sizes)
# ---- end of the binding ----------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_reference_binding_forward_and_backward(dtype):
    """The reference's in-place call (out.zero_() then _launch_grouped_kernel, the harness of
    run_on_cloud.py:66-92) and its backward, through the raw ctypes binding: top-4 routing of 96
    tokens over 16 experts (one of them empty), D = 520 (not a multiple of the 2048-column chunk),
    against the C oracle."""
    _load()
    gen = torch.Generator().manual_seed(17)
    T, E, k, D = 96, 16, 4, 520
    logits = torch.randn(T, E, generator=gen)
    logits[:, 5] = -1e9  # expert 5 gets no rows
    top = logits.topk(k, dim=1).indices.reshape(-1)
    order = torch.sort(top, stable=True).indices
    idx = (order // k).to(torch.int64)  # packed row -> token, expert-major
    counts = torch.bincount(top, minlength=E).tolist()
    w = torch.rand(T * k, generator=gen)
    experts = [torch.randn(n, D, generator=gen).to(dtype) for n in counts]
    go_cpu = torch.randn(T, D, generator=gen).to(dtype)

    xd = [x.to(DEV) for x in experts]
    idd, wd, go = idx.to(DEV), w.to(DEV), go_cpu.to(DEV)
    out = torch.empty(T, D, dtype=dtype, device=DEV)
    out.zero_()
    out, ws = _launch_grouped_kernel(xd, idd, wd, out)
    torch.cuda.synchronize()
    want, _, _ = oracle_fwd(experts, idx, w, T, dtype)
    np.testing.assert_array_equal(bits(out),
                                  want.view(np.uint32) if want.dtype == np.float32 else want)

    grads = _backward(ws, T * k, T, D, dtype, wd, go, counts)
    torch.cuda.synchronize()
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go_cpu)
    np.testing.assert_array_equal(np.concatenate([to_np(t) for t in grads[3:]]), want_gx)
    scale = abs_dot(experts, idx, go_cpu, T)
    assert np.all(np.abs(grads[1].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)
