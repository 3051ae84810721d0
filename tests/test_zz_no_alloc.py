"""fmoe_combine_fwd_noalloc (the allocation-free deterministic forward) against the entry points it
stands for, fmoe_build_metadata_and_plan + fmoe_combine_fwd(det), called through the C ABI.

The bar is bit equality (the same kernels on the same inputs), and the oracle on top.  Two calls
in a row, the second smaller, check that nothing left in the shared static buffer by the first call
leaks into the second.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from fastmoe_amd import _abi
from fastmoe_amd.workloads import Workload, make_experts, make_routing
from tests.helpers import bits, oracle_fwd

CODE = {torch.float32: _abi.F32, torch.bfloat16: _abi.BF16, torch.float16: _abi.F16}
ICODE = {torch.int64: _abi.I64, torch.int32: _abi.I32}
SCRATCH_BYTES = 16 << 20


def _case(T, D, E, k, dtype, seed, idx_dtype=torch.int64):
    wl = Workload(f"noalloc{seed}", T, D, E, k, dtype, seed, False)
    idx, w, counts = make_routing(wl)
    xs_cpu = make_experts(counts, D, dtype, "cpu", seed)
    dev = torch.device("cuda:0")
    return dict(T=T, D=D, xs_cpu=xs_cpu, idx_cpu=idx, w_cpu=w,
                xs=[x.to(dev) for x in xs_cpu], idx=idx.to(idx_dtype).to(dev), w=w.to(dev))


def _as_bits(a: np.ndarray) -> np.ndarray:
    """Oracle output as bit patterns (fp32 values -> uint32; 16-bit outputs are bits already)."""
    return a.view(np.uint32) if a.dtype == np.float32 else a


def _table(xs):
    E = len(xs)
    ptrs = (ctypes.c_int64 * E)(*[x.data_ptr() if x.shape[0] else 0 for x in xs])
    rows = (ctypes.c_int64 * E)(*[x.shape[0] for x in xs])
    return ptrs, rows, E


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _noalloc(c, out, accumulate):
    lib = _abi.lib()
    ptrs, rows, E = _table(c["xs"])
    rc = lib.fmoe_combine_fwd_noalloc(
        ptrs, rows, E, c["idx"].data_ptr(), ICODE[c["idx"].dtype], c["w"].data_ptr(),
        CODE[c["w"].dtype], c["T"], c["D"], CODE[c["xs"][0].dtype], out.data_ptr(),
        CODE[out.dtype], out.stride(0), accumulate, _stream())
    _abi.check(rc, "fmoe_combine_fwd_noalloc")


def _with_workspace(c, out, accumulate):
    """The existing entry points, with caller-allocated metadata arrays and plan workspace."""
    lib = _abi.lib()
    dev = out.device
    ptrs, rows, E = _table(c["xs"])
    N = sum(x.shape[0] for x in c["xs"])
    T, D = c["T"], c["D"]
    ptr_table = torch.empty(E, dtype=torch.int64, device=dev)
    chunk = torch.empty(E, dtype=torch.int32, device=dev)
    offs = torch.empty(E + 1, dtype=torch.int64, device=dev)
    mx = torch.empty(1, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.fmoe_plan_workspace_bytes(N, T), dtype=torch.uint8, device=dev)
    xdt = c["xs"][0].dtype
    rc = lib.fmoe_build_metadata_and_plan(
        ptrs, rows, E, ptr_table.data_ptr(), chunk.data_ptr(), offs.data_ptr(), mx.data_ptr(),
        c["idx"].data_ptr(), ICODE[c["idx"].dtype], c["w"].data_ptr(), CODE[c["w"].dtype], T,
        D * c["xs"][0].element_size(), ws.data_ptr(), _stream())
    _abi.check(rc, "fmoe_build_metadata_and_plan")
    rc = lib.fmoe_combine_fwd(_abi.MODE_DET, ws.data_ptr(), None, _abi.I64, None, _abi.F32,
                              ptr_table.data_ptr(), offs.data_ptr(), E, N, T, D, CODE[xdt],
                              out.data_ptr(), CODE[out.dtype], out.stride(0), accumulate, None, 0,
                              _stream())
    _abi.check(rc, "fmoe_combine_fwd")
    return ws  # kept alive until the caller synchronises


@pytest.mark.gpu
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_noalloc_equals_workspace_entry_points_two_calls_second_smaller(out_dtype):
    print(f"noalloc: two calls, out {out_dtype}", flush=True)
    big = _case(1024, 2048, 64, 6, torch.bfloat16, 11)
    small = _case(96, 520, 8, 2, torch.bfloat16, 12)  # D % 8 == 0, narrower rows, fewer experts
    dev = big["xs"][0].device
    want = []
    keep = []
    for c in (big, small):
        o = torch.full((c["T"], c["D"]), 7.0, dtype=out_dtype, device=dev)
        keep.append(_with_workspace(c, o, 0))
        want.append(o)
    got = []
    for c in (big, small):  # back to back on one stream: the second reuses the first's scratch
        o = torch.full((c["T"], c["D"]), -3.0, dtype=out_dtype, device=dev)
        _noalloc(c, o, 0)
        got.append(o)
    torch.cuda.synchronize()
    for c, g, wnt in zip((big, small), got, want):
        assert np.array_equal(bits(g), bits(wnt))
        exp, _, _ = oracle_fwd(c["xs_cpu"], c["idx_cpu"], c["w_cpu"], c["T"], out_dtype)
        assert np.array_equal(bits(g), _as_bits(exp))


@pytest.mark.gpu
def test_noalloc_ranged_plan_then_smaller_call():
    """72,000 rows (at least 2^16: the metadata and plan take the ranged plan's two launches, its
    partition and tables in the static buffer), then a call of 192 rows reusing that buffer; both
    equal the workspace entry points bit for bit and the oracle."""
    print("noalloc: ranged-plan call, then a smaller one", flush=True)
    big = _case(12000, 64, 64, 6, torch.bfloat16, 13)
    small = _case(96, 520, 8, 2, torch.bfloat16, 14)
    dev = big["xs"][0].device
    want, got, keep = [], [], []
    for c in (big, small):
        o = torch.zeros((c["T"], c["D"]), dtype=torch.bfloat16, device=dev)
        keep.append(_with_workspace(c, o, 0))
        want.append(o)
    for c in (big, small):
        o = torch.full((c["T"], c["D"]), 5.0, dtype=torch.bfloat16, device=dev)
        _noalloc(c, o, 0)
        got.append(o)
    torch.cuda.synchronize()
    for c, g, wnt in zip((big, small), got, want):
        assert np.array_equal(bits(g), bits(wnt))
        exp, _, _ = oracle_fwd(c["xs_cpu"], c["idx_cpu"], c["w_cpu"], c["T"], torch.bfloat16)
        assert np.array_equal(bits(g), _as_bits(exp))


@pytest.mark.gpu
def test_noalloc_accumulates_into_padded_out_with_int32_indices():
    print("noalloc: accumulate, padded fp32 out, int32 indices", flush=True)
    big = _case(700, 1000, 40, 4, torch.bfloat16, 13, torch.int32)
    small = _case(33, 1000, 5, 3, torch.bfloat16, 14, torch.int32)
    dev = big["xs"][0].device
    gen = torch.Generator(device=dev).manual_seed(5)
    for c in (big, small):
        base = torch.randn(c["T"], c["D"] + 24, device=dev, generator=gen)
        a = base.clone()[:, : c["D"]]
        b = base.clone()[:, : c["D"]]
        ws = _with_workspace(c, a, 1)
        _noalloc(c, b, 1)
        torch.cuda.synchronize()
        del ws
        assert np.array_equal(bits(a), bits(b))
        init = base[:, : c["D"]].contiguous().cpu().numpy()
        exp, _, _ = oracle_fwd(c["xs_cpu"], c["idx_cpu"], c["w_cpu"], c["T"], torch.float32,
                               acc_init=init)
        assert np.array_equal(bits(b), _as_bits(exp))


@pytest.mark.gpu
def test_noalloc_captured_in_a_graph_replays_like_the_oracle():
    """After one eager call on the device (which looks up the static buffer's address), the
    entry point is captured in a HIP graph.  Every replay overwrites ``out`` with the oracle's
    bits, also after an eager call of another size has reused the static buffer in between."""
    print("noalloc: captured once, replayed with eager calls between", flush=True)
    c = _case(512, 1024, 32, 6, torch.bfloat16, 15)
    other = _case(96, 520, 8, 2, torch.bfloat16, 16)
    dev = c["xs"][0].device
    exp, _, _ = oracle_fwd(c["xs_cpu"], c["idx_cpu"], c["w_cpu"], c["T"], torch.bfloat16)
    exp_other, _, _ = oracle_fwd(other["xs_cpu"], other["idx_cpu"], other["w_cpu"], other["T"],
                                 torch.bfloat16)
    out = torch.zeros((c["T"], c["D"]), dtype=torch.bfloat16, device=dev)
    _noalloc(c, out, 0)  # first call on the device, outside any capture
    torch.cuda.synchronize()
    assert np.array_equal(bits(out), _as_bits(exp))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            _noalloc(c, out, 0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        out.fill_(-1.0)
        o2 = torch.full((other["T"], other["D"]), 2.0, dtype=torch.bfloat16, device=dev)
        _noalloc(other, o2, 0)  # reuses the static buffer between replays
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), _as_bits(exp)), f"replay {i}"
        assert np.array_equal(bits(o2), _as_bits(exp_other))


def test_noalloc_rejects_sizes_beyond_the_static_buffer():
    """Host-side checks only: they return before any HIP call (no GPU needed)."""
    lib = _abi.lib()
    E = 4
    ptrs = (ctypes.c_int64 * E)(0x1000, 0x2000, 0x3000, 0x4000)
    n = 300_000  # 4 * 300k rows: ~38 MB of plan records, beyond the 16 MiB buffer
    rows = (ctypes.c_int64 * E)(n, n, n, n)
    dev = 0x10000  # never dereferenced
    rc = lib.fmoe_combine_fwd_noalloc(ptrs, rows, E, dev, _abi.I64, dev, _abi.F32, 1000, 64,
                                      _abi.F32, dev, _abi.F32, 64, 0, None)
    assert rc == _abi.ERANGE
    msg = lib.fmoe_last_error().decode()
    assert "static scratch" in msg and str(4 * n) in msg
    assert lib.fmoe_plan_workspace_bytes(4 * n, 1000) > SCRATCH_BYTES
    rc = lib.fmoe_combine_fwd_noalloc(ptrs, rows, 5000, dev, _abi.I64, dev, _abi.F32, 1000, 64,
                                      _abi.F32, dev, _abi.F32, 64, 0, None)
    assert rc == _abi.EINVAL
