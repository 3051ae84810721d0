"""GPU parity of the HIP combine against the C oracle (oracle/combine_ref.c).

Bars:
  * deterministic forward: bit-identical to the oracle, which adds the fp32-rounded products in
    ascending packed-row order like torch's CPU index_add_ (ops.py:373-384), then rounds once to
    the output dtype -- i.e. 0 ulp in fp32 and "<= 1 ulp after fp32 accumulation" in bf16/f16;
  * atomic forward: fp32 within 2 (n-1) * 2^-24 * sum|terms| of the oracle for n terms per
    output (two summation orders, each within (n-1) * 2^-24 * sum|terms| of the exact sum, the
    in-place initial value being a term); 16-bit outputs with
    packed 16-bit atomics round after every add, so within k * 2^-8 (bf16) / k * 2^-11 (f16) of
    sum|terms|;
  * grad_X: bit-identical (one fp32 product, one rounding, as ops.py:344-353 + autograd's cast);
  * grad_w: within 1e-6 * sum_d |grad_out * X| of the fp64 oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import fastmoe_amd
from fastmoe_amd import ops
from fastmoe_amd.workloads import WORKLOADS, Workload, make_experts, make_routing
from tests.helpers import (abs_dot, abs_sum, bits, oracle_bwd, oracle_fwd, packed_tol,
                           reorder_tol, to_np, within_one_ulp16)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# BASELINE configurations at sizes the CPU oracle finishes in about a second.
SCALED = {
    "plumbing": 256,    # full size
    "mid": 512,
    "gigachat": 256,
    "skewed": 1024,
    "detatomic": 1024,
    "published": 512,
}


def _inputs(name: str, T: int | None = None, dtype=None):
    wl = WORKLOADS[name]
    T = SCALED[name] if T is None else T
    idx, w, counts = make_routing(wl, T)
    experts = make_experts(counts, wl.D, dtype or wl.dtype, "cpu", wl.seed)
    return wl, T, idx, w, experts


def _to_dev(experts, idx, w):
    return [x.to(DEV) for x in experts], idx.to(DEV), w.to(DEV)


@pytest.mark.parametrize("name", list(SCALED))
def test_fwd_det_bitexact(name):
    wl, T, idx, w, experts = _inputs(name)
    xd, idd, wd = _to_dev(experts, idx, w)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), mode="det")
    torch.cuda.synchronize()
    assert out.dtype == wl.dtype and out.shape == (T, wl.D)
    want, _, bad = oracle_fwd(experts, idx, w, T, wl.dtype)
    assert bad == 0
    np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32 else want)


@pytest.mark.parametrize("order", [1, 2], ids=["row_chunks", "chunk_major"])
@pytest.mark.parametrize("mode", ["atomic", "atomic_packed"])
@pytest.mark.parametrize("name", list(SCALED))
def test_fwd_atomic_within_reordering(name, mode, order, kernel_options):
    """Atomic forwards against the oracle, in both grid orders (a row's column chunks side by
    side, and column-chunk-major).  fp32 outputs (both modes): within the gap of two fp32
    summation orders.  16-bit outputs: "atomic" accumulates in fp32 and rounds once, so within one
    ulp of the oracle's result (the sequential fp32 sum rounded once) plus that gap;
    "atomic_packed" rounds at every add, within the (n + 2) u sum|terms| rounding model."""
    kernel_options(fwd_atomic_order=order)
    wl, T, idx, w, experts = _inputs(name)
    xd, idd, wd = _to_dev(experts, idx, w)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), mode=mode)
    torch.cuda.synchronize()
    want, acc, _ = oracle_fwd(experts, idx, w, T, wl.dtype)
    scale = abs_sum(experts, idx, w, T)
    got = out.float().cpu().numpy()
    k = max(2, int(np.bincount(idx.numpy(), minlength=T).max()))
    if wl.dtype == torch.float32:
        assert np.all(np.abs(got - acc) <= reorder_tol(k, scale))
    elif mode == "atomic":
        want16 = torch.from_numpy(want.view(np.int16)).view(wl.dtype).float().numpy()
        assert np.all(within_one_ulp16(got, want16, wl.dtype, k, scale))
    else:
        want16 = torch.from_numpy(want.view(np.int16)).view(wl.dtype).float().numpy()
        assert np.all(np.abs(got - want16) <= packed_tol(k, scale, wl.dtype))


def test_fwd_fp32_atomic_vs_det_on_published_shape():
    """The reference's own bench shape (randint indices, fp32): det is bit-exact, atomic close."""
    wl, T, idx, w, experts = _inputs("published")
    xd, idd, wd = _to_dev(experts, idx, w)
    det = torch.zeros(T, wl.D, device=DEV)
    atom = torch.zeros(T, wl.D, device=DEV)
    fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), out=det, mode="det")
    fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), out=atom, mode="atomic")
    want, acc, _ = oracle_fwd(experts, idx, w, T, torch.float32)
    np.testing.assert_array_equal(bits(det), want.view(np.uint32))
    k = int(np.bincount(idx.numpy(), minlength=T).max())
    scale = abs_sum(experts, idx, w, T)
    assert np.all(np.abs(atom.cpu().numpy() - acc) <= reorder_tol(k, scale))


# Backward launch shapes: split grad_X / grad_w passes (default), the fused single pass, and the
# narrower column steps chosen for small D.
_BWD_VARIANTS = {
    "split": {},
    "fused": {"bwd_fused": 1},
    "split_u1": {"bwd_u": 1},
    "fused_u2": {"bwd_fused": 1, "bwd_u": 2},
}


def _set_bwd_variant(kernel_options, variant):
    kernel_options(**_BWD_VARIANTS[variant])


_PLAN_PATHS = {"tok": 3, "ranged": 4, "bucketed": 2, "radix": 1}  # values of the "plan" option
_NO_LONGEST = ("tok", "ranged")  # plans whose workgroups never see every segment


@pytest.mark.parametrize("variant", list(_BWD_VARIANTS))
@pytest.mark.parametrize("name", ["plumbing", "gigachat", "skewed"])
def test_bwd_grad_x_bitexact_grad_w_close(name, variant, kernel_options):
    _set_bwd_variant(kernel_options, variant)
    wl, T, idx, w, experts = _inputs(name)
    xd, idd, wd = _to_dev(experts, idx, w)
    xd = [x.requires_grad_(True) for x in xd]
    wd.requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D))
    gen = torch.Generator().manual_seed(wl.seed + 7)
    grad_out = torch.randn(T, wl.D, generator=gen).to(wl.dtype)
    grads = torch.autograd.grad(out, [wd, *xd], grad_out.to(DEV))
    gw, gxs = grads[0], grads[1:]
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, grad_out)
    got_gx = np.concatenate([to_np(g) for g in gxs], 0)
    np.testing.assert_array_equal(got_gx.view(np.uint32) if got_gx.dtype == np.float32 else got_gx,
                                  want_gx.view(np.uint32) if want_gx.dtype == np.float32 else want_gx)
    scale = abs_dot(experts, idx, grad_out, T)
    err = np.abs(gw.double().cpu().numpy() - want_gw)
    assert np.all(err <= 1e-6 * scale + 1e-30)
    assert gw.dtype == wd.dtype


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 16384), (torch.float32, 4104),
                                     (torch.float16, 8200)])
def test_bwd_grad_w_staged_equals_per_wave(dtype, D, kernel_options):
    """At U = 4 the grad_w pass shares grad_out through LDS for tokens of 1-8 rows and reads it
    per wave otherwise (longer segments, the out-of-range segment, or FMOE_GW_STAGED=0): both give
    the same bits, and both meet the oracle's 1e-6 bar.  Row lengths are not multiples of the LDS
    slice.  U = 4 is set: by row length the pass takes it only from 24 KiB rows."""
    rng = np.random.default_rng(17)
    T, E = 300, 37
    per_token = rng.integers(0, 13, T)          # 0..12 rows: both paths occur
    idx = np.repeat(np.arange(T), per_token)
    idx[:: 29] = T + 3                           # out of range: the per-wave zero path
    idx = torch.from_numpy(idx[rng.permutation(idx.size)])
    N = idx.numel()
    gen = torch.Generator().manual_seed(18)
    sizes = np.diff(np.concatenate([[0], np.sort(rng.integers(0, N + 1, E - 1)), [N]])).tolist()
    experts = [torch.randn(n, D, generator=gen).to(dtype) for n in sizes]
    w = torch.rand(N, generator=gen)
    go = torch.randn(T, D, generator=gen).to(dtype)
    xd, idd, wd = _to_dev(experts, idx, w)
    got = {}
    for staged in ("1", "0"):
        kernel_options(gw_staged=int(staged), bwd_u=4)
        wg = wd.clone().requires_grad_(True)
        out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wg, (T, D))
        (got[staged],) = torch.autograd.grad(out, [wg], go.to(DEV))
    np.testing.assert_array_equal(bits(got["1"]), bits(got["0"]))
    _, want_gw = oracle_bwd(experts, idx, w, T, go)
    scale = abs_dot(experts, idx, go, T)
    assert np.all(np.abs(got["1"].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


# (dtype, D): row lengths that are not multiples of the column step, and D % 8 != 0 (element
# accesses instead of 16-byte vectors).
_GX_EDGES = [(torch.bfloat16, 16384), (torch.bfloat16, 7000), (torch.float16, 8200),
             (torch.float32, 4104), (torch.bfloat16, 7001)]


@pytest.mark.parametrize("dtype,D", _GX_EDGES)
def test_bwd_grad_x_negative_gates_and_out_of_range_rows(dtype, D):
    """grad_X alone through the C ABI, bit for bit against the oracle, with gates of both signs
    (an out-of-range row's gradient is +0, not 0 * w = -0), out-of-range indices (the plan's last
    segment), tokens without rows and a grad_out row stride wider than D."""
    rng = np.random.default_rng(23 + D)
    T, E = 301, 29
    per_token = rng.integers(0, 11, T)
    idx = np.repeat(np.arange(T), per_token)
    idx[:: 31] = T + 3
    idx = torch.from_numpy(idx[rng.permutation(idx.size)])
    N = idx.numel()
    gen = torch.Generator().manual_seed(24)
    sizes = np.diff(np.concatenate([[0], np.sort(rng.integers(0, N + 1, E - 1)), [N]])).tolist()
    experts = [torch.randn(n, D, generator=gen).to(dtype) for n in sizes]
    w = torch.rand(N, generator=gen) - 0.5
    go_wide = torch.randn(T, D + 8, generator=gen).to(dtype)
    xd, idd, wd = _to_dev(experts, idx, w)
    meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
    plan = fastmoe_amd.build_plan(meta, idd, wd, T)
    god = go_wide.to(DEV)
    code = {torch.float32: fastmoe_amd._abi.F32, torch.bfloat16: fastmoe_amd._abi.BF16,
            torch.float16: fastmoe_amd._abi.F16}[dtype]
    gx = torch.full((N, D), float("nan"), dtype=dtype, device=DEV)
    rc = fastmoe_amd._abi.lib().fmoe_combine_bwd(
        plan.data_ptr(), N, T, D, code, god.data_ptr(), code, D + 8, gx.data_ptr(), None,
        fastmoe_amd._abi.F32, torch.cuda.current_stream().cuda_stream)
    fastmoe_amd._abi.check(rc, "fmoe_combine_bwd")
    torch.cuda.synchronize()
    want_gx, _ = oracle_bwd(experts, idx, w, T, go_wide[:, :D].contiguous())
    np.testing.assert_array_equal(bits(gx), want_gx.view(np.uint32) if want_gx.dtype == np.float32
                                  else want_gx)


@pytest.mark.parametrize("fused", ["0", "1"])
def test_bwd_abi_both_outputs_in_one_call(fused, kernel_options):
    """fmoe_combine_bwd given both outputs (the call a C-ABI binding makes): grad_X and grad_w
    from its two back-to-back passes (or the fused pass) equal the oracle."""
    kernel_options(bwd_fused=int(fused))
    wl, T, idx, w, experts = _inputs("gigachat")
    xd, idd, wd = _to_dev(experts, idx, w)
    meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
    plan = fastmoe_amd.build_plan(meta, idd, wd, T)
    N, D = idx.numel(), wl.D
    gen = torch.Generator().manual_seed(11)
    grad_out = torch.randn(T, D, generator=gen).to(wl.dtype)
    god = grad_out.to(DEV)
    gx = torch.full((N, D), float("nan"), dtype=wl.dtype, device=DEV)
    gw = torch.full((N,), float("nan"), dtype=torch.float32, device=DEV)
    lib = fastmoe_amd._abi.lib()
    rc = lib.fmoe_combine_bwd(plan.data_ptr(), N, T, D, fastmoe_amd._abi.BF16, god.data_ptr(),
                              fastmoe_amd._abi.BF16, D, gx.data_ptr(), gw.data_ptr(),
                              fastmoe_amd._abi.F32, torch.cuda.current_stream().cuda_stream)
    fastmoe_amd._abi.check(rc, "fmoe_combine_bwd")
    torch.cuda.synchronize()
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, grad_out)
    np.testing.assert_array_equal(to_np(gx), want_gx)
    scale = abs_dot(experts, idx, grad_out, T)
    assert np.all(np.abs(gw.double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


def test_bwd_without_gate_grad_and_without_expert_grad():
    wl, T, idx, w, experts = _inputs("plumbing")
    xd, idd, wd = _to_dev(experts, idx, w)
    grad_out = torch.randn(T, wl.D)
    # only experts
    xg = [x.clone().requires_grad_(True) for x in xd]
    out = fastmoe_amd.grouped_weighted_scatter_add(xg, idd, wd, (T, wl.D))
    gxs = torch.autograd.grad(out, xg, grad_out.to(DEV))
    want_gx, _ = oracle_bwd(experts, idx, w, T, grad_out)
    np.testing.assert_array_equal(np.concatenate([to_np(g) for g in gxs]).view(np.uint32),
                                  want_gx.view(np.uint32))
    # only the gate
    wg = wd.clone().requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wg, (T, wl.D))
    (gw,) = torch.autograd.grad(out, [wg], grad_out.to(DEV))
    _, want_gw = oracle_bwd(experts, idx, w, T, grad_out)
    scale = abs_dot(experts, idx, grad_out, T)
    assert np.all(np.abs(gw.double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


@pytest.mark.parametrize("form", ["row_broadcast", "sum"])
def test_bwd_broadcast_grad_out(form):
    """Broadcast gradients: one row expanded over the tokens (row stride 0, read in place by the
    backward) and the all-zero-stride gradient of out.sum().  Both equal the oracle on the
    materialised grad_out."""
    wl, T, idx, w, experts = _inputs("gigachat", T=64)
    xd, idd, wd = _to_dev(experts, idx, w)
    xd = [x.requires_grad_(True) for x in xd]
    wd.requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D))
    if form == "row_broadcast":
        row = torch.randn(1, wl.D, generator=torch.Generator().manual_seed(3)).to(wl.dtype)
        god = row.to(DEV).expand(T, wl.D)
        assert god.stride() == (0, 1)
        grads = torch.autograd.grad(out, [wd, *xd], god)
        grad_out = row.expand(T, wl.D).contiguous()
    else:
        grads = torch.autograd.grad(out.sum(), [wd, *xd])
        grad_out = torch.ones(T, wl.D, dtype=wl.dtype)
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, grad_out)
    got_gx = np.concatenate([to_np(g) for g in grads[1:]], 0)
    np.testing.assert_array_equal(got_gx, want_gx)
    scale = abs_dot(experts, idx, grad_out, T)
    assert np.all(np.abs(grads[0].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


def test_inplace_accumulates_into_out():
    """ops.py:389-390 contract: the kernel adds into the given out (here non-zero)."""
    wl, T, idx, w, experts = _inputs("mid", T=256)
    xd, idd, wd = _to_dev(experts, idx, w)
    init = torch.randn(T, wl.D, generator=torch.Generator().manual_seed(9))
    for mode in ("det", "atomic"):
        out = init.to(DEV).clone()
        meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
        ret = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), out=out,
                                                        metadata=meta, mode=mode)
        assert ret is out
        want, acc, _ = oracle_fwd(experts, idx, w, T, torch.float32, acc_init=init.numpy())
        if mode == "det":
            np.testing.assert_array_equal(bits(out), want.view(np.uint32))
        else:
            scale = abs_sum(experts, idx, w, T) + np.abs(init.numpy())
            k = int(np.bincount(idx.numpy(), minlength=T).max())
            assert np.all(np.abs(out.cpu().numpy() - acc) <= reorder_tol(k + 1, scale))


def test_det_repeatable_10x():
    wl, T, idx, w, experts = _inputs("detatomic", T=2048)
    xd, idd, wd = _to_dev(experts, idx, w)
    first = None
    for _ in range(10):
        out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), mode="det")
        b = bits(out)
        if first is None:
            first = b
        else:
            np.testing.assert_array_equal(b, first)


def test_grouping_invariance():
    """Any split of the packed rows into expert buffers gives the same bits (det)."""
    wl, T, idx, w, experts = _inputs("mid", T=128)
    cat = torch.cat(experts, 0)
    xd, idd, wd = _to_dev(experts, idx, w)
    a = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), mode="det")
    one = fastmoe_amd.weighted_scatter_add(cat.to(DEV), idd, wd, (T, wl.D), mode="det")
    parts = list(torch.split(cat, [1, 7, 0, 100, cat.shape[0] - 108]))
    b = fastmoe_amd.grouped_weighted_scatter_add([p.contiguous().to(DEV) for p in parts], idd, wd,
                                                 (T, wl.D), mode="det")
    np.testing.assert_array_equal(bits(a), bits(one))
    np.testing.assert_array_equal(bits(a), bits(b))


def test_linearity_in_w():
    wl, T, idx, w, experts = _inputs("plumbing")
    xd, idd, wd = _to_dev(experts, idx, w)
    a = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D))
    b = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd * 2, (T, wl.D))
    np.testing.assert_array_equal(bits(a * 2), bits(b))


def test_edge_empty_experts_and_tokens():
    D = 64
    T = 10
    sizes = [0, 3, 0, 0, 5, 0]
    gen = torch.Generator().manual_seed(3)
    experts = [torch.randn(n, D, generator=gen) for n in sizes]
    idx = torch.tensor([0, 2, 2, 9, 4, 0, 2, 7])
    w = torch.rand(8, generator=gen)
    xd, idd, wd = _to_dev(experts, idx, w)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D))
    want, _, _ = oracle_fwd(experts, idx, w, T, torch.float32)
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))
    assert torch.all(out[[1, 3, 5, 6, 8]] == 0)


def test_edge_all_experts_empty():
    D = 16
    experts = [torch.empty(0, D, device=DEV) for _ in range(4)]
    idx = torch.empty(0, dtype=torch.long, device=DEV)
    w = torch.empty(0, device=DEV, requires_grad=True)
    xs = [x.requires_grad_(True) for x in experts]
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (5, D))
    assert out.shape == (5, D) and torch.all(out == 0)
    o2 = torch.ones(5, D, device=DEV)
    fastmoe_amd.grouped_weighted_scatter_add(experts, idx, w.detach(), (5, D), out=o2)
    assert torch.all(o2 == 1)
    g = torch.autograd.grad(out, [w, *xs], torch.ones(5, D, device=DEV))
    assert g[0].shape == (0,)


def test_edge_large_segments_randint():
    """Many rows per token (segments > 64) take the plan's long-segment ordering pass."""
    D, T, N = 40, 3, 700
    gen = torch.Generator().manual_seed(11)
    experts = [torch.randn(n, D, generator=gen) for n in (300, 0, 400)]
    idx = torch.randint(0, T, (N,), generator=gen)
    w = torch.rand(N, generator=gen)
    xd, idd, wd = _to_dev(experts, idx, w)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), mode="det")
    want, _, _ = oracle_fwd(experts, idx, w, T, torch.float32)
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))
    xg = [x.clone().requires_grad_(True) for x in xd]
    wg = wd.clone().requires_grad_(True)
    go = torch.randn(T, D, generator=gen)
    out = fastmoe_amd.grouped_weighted_scatter_add(xg, idd, wg, (T, D))
    g = torch.autograd.grad(out, [wg, *xg], go.to(DEV))
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
    got_gx = np.concatenate([to_np(t) for t in g[1:] if t is not None])
    np.testing.assert_array_equal(got_gx.view(np.uint32), want_gx.view(np.uint32))
    scale = abs_dot(experts, idx, go, T)
    assert np.all(np.abs(g[0].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


@pytest.mark.parametrize("variant", ["split", "fused"])
def test_edge_invalid_indices_dropped_and_flagged(variant, kernel_options):
    _set_bwd_variant(kernel_options, variant)
    D, T = 32, 6
    gen = torch.Generator().manual_seed(5)
    experts = [torch.randn(4, D, generator=gen), torch.randn(3, D, generator=gen)]
    idx = torch.tensor([0, -1, 5, 6, 2, 100, 2])
    w = torch.rand(7, generator=gen)
    xd, idd, wd = _to_dev(experts, idx, w)
    for mode in ("det", "atomic"):
        out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), mode=mode)
        want, acc, bad = oracle_fwd(experts, idx, w, T, torch.float32)
        assert bad == 3
        if mode == "det":
            np.testing.assert_array_equal(bits(out), want.view(np.uint32))
        else:
            np.testing.assert_allclose(out.cpu().numpy(), acc, rtol=1e-6, atol=1e-6)
    meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
    plan = fastmoe_amd.build_plan(meta, idd, wd, T)
    assert int(ops.plan_status(plan)[0]) == 3
    with pytest.raises(IndexError):
        fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), validate=True)
    xg = [x.clone().requires_grad_(True) for x in xd]
    wg = wd.clone().requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xg, idd, wg, (T, D))
    go = torch.randn(T, D, generator=gen)
    g = torch.autograd.grad(out, [wg, *xg], go.to(DEV))
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
    got = np.concatenate([to_np(t) for t in g[1:]])
    np.testing.assert_array_equal(got.view(np.uint32), want_gx.view(np.uint32))
    assert np.all(g[0].cpu().numpy()[[1, 3, 5]] == 0)


@pytest.mark.parametrize("D", [100, 8, 1, 4096 + 8, 65536 + 8, 131072])
def test_edge_odd_hidden_sizes(D):
    """D not a multiple of the 16-byte vector (scalar path), partial column chunks, and wide rows
    (32 to 64 column chunks per token, rows of up to 512 KiB in fp32)."""
    T = 33
    gen = torch.Generator().manual_seed(D)
    sizes = [5, 17, 0, 11]
    for dtype in (torch.float32, torch.bfloat16):
        experts = [torch.randn(n, D, generator=gen).to(dtype) for n in sizes]
        idx = torch.randint(0, T, (sum(sizes),), generator=gen)
        w = torch.rand(sum(sizes), generator=gen)
        xd, idd, wd = _to_dev(experts, idx, w)
        out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), mode="det")
        want, _, _ = oracle_fwd(experts, idx, w, T, dtype)
        np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32 else want)
        xg = [x.clone().requires_grad_(True) for x in xd]
        wg = wd.clone().requires_grad_(True)
        out = fastmoe_amd.grouped_weighted_scatter_add(xg, idd, wg, (T, D))
        go = torch.randn(T, D, generator=gen).to(dtype)
        g = torch.autograd.grad(out, [wg, *xg], go.to(DEV))
        want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
        got = np.concatenate([to_np(t) for t in g[1:] if t is not None])
        np.testing.assert_array_equal(got, want_gx)
        scale = abs_dot(experts, idx, go, T)
        assert np.all(np.abs(g[0].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


def test_edge_misaligned_expert_buffers():
    """Expert buffers that start 2 bytes off a 16-byte boundary (views into a larger buffer)."""
    D, T = 64, 20
    gen = torch.Generator().manual_seed(21)
    sizes = [6, 9, 5]
    experts, views = [], []
    for n in sizes:
        big = torch.randn(n * D + 1, generator=gen).to(torch.bfloat16).to(DEV)
        v = big[1:].view(n, D)
        assert v.data_ptr() % 16 != 0
        views.append(v)
        experts.append(v.cpu())
    idx = torch.randint(0, T, (sum(sizes),), generator=gen)
    w = torch.rand(sum(sizes), generator=gen)
    idd, wd = idx.to(DEV), w.to(DEV)
    out = fastmoe_amd.grouped_weighted_scatter_add(views, idd, wd, (T, D), mode="det")
    want, _, _ = oracle_fwd(experts, idx, w, T, torch.bfloat16)
    np.testing.assert_array_equal(bits(out), want)
    meta = fastmoe_amd.prepare_grouped_metadata(views, DEV)
    plan = fastmoe_amd.build_plan(meta, idd, wd, T)
    assert int(ops.plan_status(plan)[1]) != 0
    atom = fastmoe_amd.grouped_weighted_scatter_add(views, idd, wd, (T, D), mode="atomic")
    _, acc, _ = oracle_fwd(experts, idx, w, T, torch.float32)
    scale = abs_sum(experts, idx, w, T)
    assert np.all(np.abs(atom.float().cpu().numpy() - acc) <= 8 * 2.0 ** -8 * scale + 1e-30)
    wg = wd.clone().requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(views, idd, wg, (T, D))
    go = torch.randn(T, D, generator=gen).to(torch.bfloat16)
    (gw,) = torch.autograd.grad(out, [wg], go.to(DEV))
    _, want_gw = oracle_bwd(experts, idx, w, T, go)
    scale = abs_dot(experts, idx, go, T)
    assert np.all(np.abs(gw.double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


@pytest.mark.parametrize("xdt,wdt,idt,odt", [
    (torch.float16, torch.float32, torch.int64, torch.float16),
    (torch.bfloat16, torch.bfloat16, torch.int32, torch.bfloat16),
    (torch.bfloat16, torch.float32, torch.int64, torch.float32),
    (torch.float32, torch.float32, torch.int32, torch.bfloat16),
])
def test_dtype_combinations(xdt, wdt, idt, odt):
    D, T = 256, 64
    gen = torch.Generator().manual_seed(2)
    sizes = [20, 0, 44, 64]
    experts = [torch.randn(n, D, generator=gen).to(xdt) for n in sizes]
    idx = torch.randint(0, T, (sum(sizes),), generator=gen)
    w = torch.rand(sum(sizes), generator=gen).to(wdt)
    xd = [x.to(DEV) for x in experts]
    out = torch.zeros(T, D, dtype=odt, device=DEV)
    fastmoe_amd.grouped_weighted_scatter_add(xd, idx.to(idt).to(DEV), w.to(DEV), (T, D), out=out,
                                             mode="det")
    want, _, _ = oracle_fwd(experts, idx, w, T, odt)
    np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32 else want)


def _plan_case(case: str):
    """(T, idx, w, experts, D) of a plan test case.  The fused plan gives each workgroup a slice
    of 2048 rows (fewer groups than rows / 2048 only above 256 groups), so N decides how many
    workgroups split a segment; N >= 65536 selects its 64-bit histogram."""
    gen = torch.Generator().manual_seed(17)
    if case in ("topk512", "long40"):
        wl, T, idx, w, experts = _inputs("skewed", T=512 if case == "topk512" else 40)
        if case == "long40":  # pile 200 extra rows onto tokens 0..2 through one more expert
            experts = experts + [torch.randn(200, wl.D, generator=gen).to(wl.dtype)]
            idx = torch.cat([idx, torch.randint(0, 3, (200,), generator=gen)])
            w = torch.cat([w, torch.rand(200, generator=gen)])
        return T, idx, w, experts, wl.D
    # randint routing over ragged experts of 8 fp32 columns
    T, N, hot = {"long_pieces_short": (50, 4096, 50),   # 2 groups, ~41-row pieces of 82-row segments
                 "long_pieces_long": (40, 10000, 3),    # 5 groups, pieces of ~650 rows
                 "wide_hist": (512, 70000, 512)}[case]  # 35 groups, 64-bit histogram words
    idx = torch.randint(0, hot, (N,), generator=gen)
    cuts = torch.sort(torch.randint(0, N + 1, (23,), generator=gen)).values.tolist()
    sizes = [b - a for a, b in zip([0] + cuts, cuts + [N])]
    experts = [torch.randn(n, 8, generator=gen) for n in sizes]
    return T, idx, torch.rand(N, generator=gen), experts, 8


@pytest.mark.parametrize("path", list(_PLAN_PATHS))
@pytest.mark.parametrize("case", ["topk512", "long40", "long_pieces_short", "long_pieces_long",
                                  "wide_hist"])
def test_plan_matches_oracle(case, path, kernel_options):
    """row_ptr, the records (source address, gate bits, g) and the status words equal the
    oracle's stable inverse, for the one-launch plan, the ranged plan (partition by token range,
    then a workgroup per range), the bucketed plan (two launches) and the radix plan (count +
    scan, then a stable radix sort by token bin): each writes every segment in ascending g,
    including when several workgroups each take a piece of one segment."""
    from oracle import cref

    kernel_options(plan=_PLAN_PATHS[path])
    T, idx, w, experts, D = _plan_case(case)
    xd, idd, wd = _to_dev(experts, idx, w)
    meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
    plan = fastmoe_amd.build_plan(meta, idd, wd, T)
    lib = fastmoe_amd._abi.lib()
    N = idx.numel()
    # the forced builder's limits hold here, so it is the one that ran (the status word's
    # longest-segment field below tells the builders apart)
    assert lib.fmoe_plan_path(N, T, len(experts)) == _PLAN_PATHS[path]
    rp_off = lib.fmoe_plan_row_ptr_offset(N, T)
    rec_off = lib.fmoe_plan_records_offset(N, T)
    row_ptr = plan[rp_off: rp_off + 4 * (T + 2)].view(torch.int32).cpu().numpy()
    rec = plan[rec_off: rec_off + 16 * N].view(torch.int64).view(N, 2).cpu()
    want_rp, want_g = cref.plan(idx.numpy(), T)
    np.testing.assert_array_equal(row_ptr, want_rp)
    g = (rec[:, 1] >> 32).numpy().astype(np.int32)
    seg_len = np.diff(want_rp)
    st = ops.plan_status(plan).cpu().numpy()
    misaligned = int((D * experts[0].element_size()) % 16 != 0)
    assert st[0] == 0 and st[1] == misaligned
    # the longest segment: recorded by the radix and bucketed plans; -1 from the one-launch and
    # ranged plans (no workgroup sees every segment)
    assert st[2] == (-1 if path in _NO_LONGEST else seg_len[:T].max())
    if case != "topk512":
        assert seg_len[:T].max() > 64
    np.testing.assert_array_equal(g, want_g)  # stable: every segment in ascending g
    wbits = (rec[:, 1] & 0xFFFFFFFF).numpy().astype(np.uint32)
    np.testing.assert_array_equal(wbits, w.numpy()[want_g].view(np.uint32))
    off, _ = cref.metadata(meta.sizes)
    e_of = np.searchsorted(off, want_g, side="right") - 1
    src = (np.array([meta.ptrs[e] for e in e_of], dtype=np.int64)
           + (want_g - off[e_of]) * D * experts[0].element_size())
    np.testing.assert_array_equal(rec[:, 0].numpy(), src)
    assert lib.fmoe_plan_workspace_bytes(N, T) == plan.numel()
    # and the forward that reads this plan is bit-exact
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), mode="det")
    want, _, _ = oracle_fwd(experts, idx, w, T, experts[0].dtype)
    np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32 else want)


@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("groups", [1, 7, 64, 256])
def test_plan_one_launch_any_group_count(groups, idx_dtype, kernel_options):
    """The one-launch plan is the oracle's stable inverse whatever the number of workgroups that
    split the token bins (option plan_groups): one workgroup for all bins, a count that leaves a
    ragged last range, and more workgroups than the automatic choice.  N = 5003 is neither even
    nor a multiple of 4, so the rows past the last whole 16-byte index vector take the tail
    path, for int64 (2 rows per vector) and int32 (4 rows per vector) indices; 3% of the indices
    are out of range."""
    from oracle import cref

    kernel_options(plan=_PLAN_PATHS["tok"], plan_groups=groups)
    gen = torch.Generator().manual_seed(61 + groups)
    T, N, D = 300, 5003, 8
    idx = torch.randint(0, T, (N,), generator=gen)
    bad = torch.rand(N, generator=gen) < 0.03
    idx = torch.where(bad, torch.full_like(idx, T + 5), idx).to(idx_dtype)
    w = torch.rand(N, generator=gen)
    cuts = torch.sort(torch.randint(0, N + 1, (15,), generator=gen)).values.tolist()
    sizes = [b - a for a, b in zip([0] + cuts, cuts + [N])]
    experts = [torch.randn(n, D, generator=gen) for n in sizes]
    xd, idd, wd = _to_dev(experts, idx, w)
    meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
    plan = fastmoe_amd.build_plan(meta, idd, wd, T)
    lib = fastmoe_amd._abi.lib()
    rp_off = lib.fmoe_plan_row_ptr_offset(N, T)
    rec_off = lib.fmoe_plan_records_offset(N, T)
    row_ptr = plan[rp_off: rp_off + 4 * (T + 2)].view(torch.int32).cpu().numpy()
    rec = plan[rec_off: rec_off + 16 * N].view(torch.int64).view(N, 2).cpu()
    want_rp, want_g = cref.plan(idx.to(torch.int64).numpy(), T)
    np.testing.assert_array_equal(row_ptr, want_rp)
    np.testing.assert_array_equal((rec[:, 1] >> 32).numpy().astype(np.int32), want_g)
    wbits = (rec[:, 1] & 0xFFFFFFFF).numpy().astype(np.uint32)
    np.testing.assert_array_equal(wbits, w.numpy()[want_g].view(np.uint32))
    st = ops.plan_status(plan).cpu().numpy()
    assert st[0] == int(bad.sum()) and st[1] == 0


@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("T,N,hot", [(16384, 131072, 0), (32768, 65536, 0), (1000, 100_003, 0),
                                     (70000, 200_000, 0), (4096, 50_000, 20_000),
                                     (131071, 1 << 20, 0), (262143, (1 << 21) + 3, 0),
                                     ((1 << 19) - 1, (1 << 22) - 5, 0)])
def test_plan_ranged_matches_oracle(T, N, hot, idx_dtype, kernel_options):
    """The ranged plan (k_plan_split partitions the rows by token range in 1024-row slices, then
    a workgroup per range orders its rows) is the oracle's stable inverse at the sizes it is
    chosen for: the skewed and detatomic shapes (bins per range 65 and 129, found by the
    multiply-shift division), a ragged last slice (N not a multiple of 1024), more token bins than
    256 ranges of 256 bins hold, int32 and int64 indices, 2% of them out of range on both sides;
    with `hot` rows piled onto token 7, that range's waves overflow their stashes and replay their
    rows; T + 1 = 2^17 bins over 2^20 rows (256 ranges of 512 bins, 1024 slices), 2^18 bins over
    2^21 rows (513 ranges) and 2^19 bins over 2^22 rows (the plan's limit: 1024 ranges of 512
    bins, 4096 slices).  The forward reading the plan is bit-exact."""
    from oracle import cref

    kernel_options(plan=_PLAN_PATHS["ranged"])
    gen = torch.Generator().manual_seed(T + N)
    D = 4
    idx = torch.randint(0, T, (N,), generator=gen)
    if hot:
        idx[torch.randperm(N, generator=gen)[:hot]] = 7
    bad = torch.rand(N, generator=gen) < 0.02
    idx = torch.where(bad, torch.where(torch.rand(N, generator=gen) < 0.5,
                                       torch.full_like(idx, T), torch.full_like(idx, -3)), idx)
    idx = idx.to(idx_dtype)
    w = torch.rand(N, generator=gen)
    cuts = torch.sort(torch.randint(0, N + 1, (31,), generator=gen)).values.tolist()
    sizes = [b - a for a, b in zip([0] + cuts, cuts + [N])]
    experts = [torch.randn(n, D, generator=gen) for n in sizes]
    xd, idd, wd = _to_dev(experts, idx, w)
    meta, plan = ops.prepare_metadata_and_plan(xd, idd, wd, T)
    lib = fastmoe_amd._abi.lib()
    rp = plan[lib.fmoe_plan_row_ptr_offset(N, T):][: 4 * (T + 2)].view(torch.int32).cpu().numpy()
    rec = plan[lib.fmoe_plan_records_offset(N, T):][: 16 * N].view(torch.int64).view(N, 2).cpu()
    want_rp, want_g = cref.plan(idx.to(torch.int64).numpy(), T)
    np.testing.assert_array_equal(rp, want_rp)
    np.testing.assert_array_equal((rec[:, 1] >> 32).numpy().astype(np.int32), want_g)
    wbits = (rec[:, 1] & 0xFFFFFFFF).numpy().astype(np.uint32)
    np.testing.assert_array_equal(wbits, w.numpy()[want_g].view(np.uint32))
    st = ops.plan_status(plan).cpu().numpy()
    assert st[0] == int(bad.sum()) and st[1] == 0 and st[2] == -1
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D))
    want, _, _ = oracle_fwd(experts, idx.to(torch.int64), w, T, torch.float32)
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))


@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("path,T,N,hot", [("tok", 500, 20_003, 12_000), ("tok", 1, 9_000, 0),
                                          ("ranged", 3000, 90_001, 50_000),
                                          ("ranged", 70_000, 140_000, 30_000)])
def test_plan_hot_token_matches_oracle(path, T, N, hot, idx_dtype, kernel_options):
    """A hot token (`hot` rows on token 7, or every row on the single token) makes its range's
    waves overflow their stashes: the one-launch plan then replays each wave's rows for the
    counts and the fill, the ranged plan counts the rows past the stash during its pass and
    replays them for the fill, with the rows' gates and experts looked up a batch at a time.
    256 experts, a fifth of them empty, so the expert search crosses runs of equal offsets.
    Row pointers, record order and gate bits equal the oracle's stable inverse and the forward
    reading the records (their source addresses) is bit-exact."""
    from oracle import cref

    kernel_options(plan=_PLAN_PATHS[path])
    gen = torch.Generator().manual_seed(T + N + hot)
    D = 4
    idx = torch.randint(0, T, (N,), generator=gen)
    if hot:
        idx[torch.randperm(N, generator=gen)[:hot]] = 7
    bad = torch.rand(N, generator=gen) < 0.01
    idx = torch.where(bad, torch.full_like(idx, T + 3), idx).to(idx_dtype)
    w = torch.rand(N, generator=gen)
    cuts = torch.sort(torch.randint(0, N + 1, (255,), generator=gen)).values
    sizes = [b - a for a, b in zip([0] + cuts.tolist(), cuts.tolist() + [N])]
    empty = torch.randperm(256, generator=gen)[:51].tolist()
    for e in empty:  # hand an expert's rows to its neighbour, leaving it empty
        n = (e + 1) % 256
        sizes[n] += sizes[e]
        sizes[e] = 0
    experts = [torch.randn(n, D, generator=gen) for n in sizes]
    xd, idd, wd = _to_dev(experts, idx, w)
    meta, plan = ops.prepare_metadata_and_plan(xd, idd, wd, T)
    lib = fastmoe_amd._abi.lib()
    assert lib.fmoe_plan_path(N, T, 256) == _PLAN_PATHS[path]
    rp = plan[lib.fmoe_plan_row_ptr_offset(N, T):][: 4 * (T + 2)].view(torch.int32).cpu().numpy()
    rec = plan[lib.fmoe_plan_records_offset(N, T):][: 16 * N].view(torch.int64).view(N, 2).cpu()
    want_rp, want_g = cref.plan(idx.to(torch.int64).numpy(), T)
    np.testing.assert_array_equal(rp, want_rp)
    np.testing.assert_array_equal((rec[:, 1] >> 32).numpy().astype(np.int32), want_g)
    wbits = (rec[:, 1] & 0xFFFFFFFF).numpy().astype(np.uint32)
    np.testing.assert_array_equal(wbits, w.numpy()[want_g].view(np.uint32))
    assert int(ops.plan_status(plan).cpu()[0]) == int(bad.sum())
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D))
    want, _, _ = oracle_fwd(experts, idx.to(torch.int64), w, T, torch.float32)
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))


def test_bwd_f16_grad_x_rounds_twice_like_the_reference():
    """f16 experts, fp32 gates: grad_X is the fp32 product rounded to fp32 and then to f16
    (index_select * w, then autograd's cast; ops.py:344-353).  The inputs include elements where
    rounding the exact product once to f16 gives another value, so a kernel that fuses the
    multiply and the conversion (one rounding) fails here."""
    gen = torch.Generator().manual_seed(47)
    T, D, k, E = 1000, 1024, 2, 64
    N = T * k
    idx = torch.arange(T).repeat_interleave(k)[torch.randperm(N, generator=gen)]
    w = torch.rand(N, generator=gen)
    sizes = [N // E] * (E - 1) + [N - (N // E) * (E - 1)]
    experts = [torch.randn(n, D, generator=gen).to(torch.float16) for n in sizes]
    go = torch.randn(T, D, generator=gen).to(torch.float16)
    # sensitivity: some products differ between one rounding and two
    prod = go.double().numpy()[idx.numpy()] * w.double().numpy()[:, None]
    once = prod.astype(np.float16)
    twice = prod.astype(np.float32).astype(np.float16)
    assert np.count_nonzero(once != twice) > 0
    xs = [x.to(DEV).requires_grad_(True) for x in experts]
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx.to(DEV), w.to(DEV), (T, D))
    grads = torch.autograd.grad(out, xs, go.to(DEV))
    want_gx, _ = oracle_bwd(experts, idx, w, T, go)
    np.testing.assert_array_equal(np.concatenate([to_np(g) for g in grads]), want_gx)
    np.testing.assert_array_equal(want_gx.view(np.float16), twice)  # the oracle rounds twice


@pytest.mark.parametrize("plan", list(_PLAN_PATHS))
def test_random_shapes_against_oracle(plan, kernel_options):
    """40 seeded random cases: tokens, experts (some empty), rows, D, every dtype combination,
    int32/int64 indices, and out-of-range indices mixed in; forward bits, grad_X bits and grad_w
    (1e-6 of sum|terms|) against the oracle, through the autograd path, with each of the
    four plans."""
    kernel_options(plan=_PLAN_PATHS[plan])
    rng = np.random.default_rng(2026)
    dts = [torch.float32, torch.bfloat16, torch.float16]
    for case in range(40):
        T = int(rng.choice([1, 2, 7, 64, 300, 1000, 2500]))
        E = int(rng.integers(1, 300))
        N = int(rng.integers(1, 6000))
        D = int(rng.choice([1, 7, 8, 64, 200, 1024]))
        xdt = dts[int(rng.integers(3))]
        wdt = [torch.float32, torch.bfloat16][int(rng.integers(2))]
        idt = [torch.int64, torch.int32][int(rng.integers(2))]
        gen = torch.Generator().manual_seed(case)
        cuts = np.sort(rng.integers(0, N + 1, E - 1))
        sizes = np.diff(np.concatenate([[0], cuts, [N]])).tolist()
        idx = torch.from_numpy(rng.integers(0, T, N)).to(idt)
        if case % 3 == 0:
            idx[:: int(rng.integers(5, 50))] = T + 1  # out of range
        w = torch.rand(N, generator=gen).to(wdt)
        experts = [torch.randn(n, D, generator=gen).to(xdt) for n in sizes]
        xs = [x.to(DEV).requires_grad_(True) for x in experts]
        wd = w.to(DEV).requires_grad_(True)
        out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx.to(DEV), wd, (T, D))
        go = torch.randn(T, D, generator=gen).to(xdt)
        if case % 5 == 3:    # grad_out rows with a padded stride (read in place)
            god = torch.zeros(T, D + 24, dtype=xdt, device=DEV)[:, :D]
            god.copy_(go.to(DEV))
        elif case % 5 == 4:  # a transposed grad_out (made contiguous by the backward)
            god = go.t().contiguous().to(DEV).t()
        else:
            god = go.to(DEV)
        grads = torch.autograd.grad(out, [wd, *xs], god)
        torch.cuda.synchronize()
        label = f"case {case}: T={T} E={E} N={N} D={D} {xdt} {wdt} {idt} go strides {god.stride()}"
        want, _, _ = oracle_fwd(experts, idx, w, T, xdt)
        np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32
                                      else want, err_msg=label)
        want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
        got_gx = np.concatenate([to_np(g).reshape(-1, D) for g in grads[1:]])
        np.testing.assert_array_equal(got_gx.view(want_gx.dtype), want_gx, err_msg=label)
        scale = abs_dot(experts, idx, go, T)
        err = np.abs(grads[0].double().cpu().numpy() - want_gw)
        # grad_w is stored in the gates' dtype: add its rounding (2^-8 for bf16)
        rtol = 1e-6 if wdt == torch.float32 else 2.0 ** -8
        assert np.all(err <= 1e-6 * scale + rtol * np.abs(want_gw) + 1e-30), label


@pytest.mark.parametrize("bwd", ["split", "fused"])
def test_random_misaligned_buffers_against_oracle(bwd, kernel_options):
    """16 seeded random cases whose buffers sit at arbitrary element offsets of shared pools:
    every expert (some empty) a contiguous view at a random offset, grad_out and an in-place out
    at odd offsets with padded row strides.  Forward (autograd and in place, det) bit-exact,
    grad_X bit-exact and grad_w within 1e-6 of sum|terms|, with the backward's two passes or its
    fused pass."""
    kernel_options(bwd_fused=1 if bwd == "fused" else 0)
    rng = np.random.default_rng(4242)
    dts = [torch.float32, torch.bfloat16, torch.float16]
    for case in range(16):
        T = int(rng.choice([1, 3, 64, 500]))
        E = int(rng.integers(1, 40))
        N = int(rng.integers(1, 3000))
        D = int(rng.choice([1, 5, 8, 33, 256, 1000]))
        xdt = dts[int(rng.integers(3))]
        gen = torch.Generator().manual_seed(900 + case)
        cuts = np.sort(rng.integers(0, N + 1, E - 1))
        sizes = np.diff(np.concatenate([[0], cuts, [N]])).tolist()
        # one pool for every expert, each at a random element offset after the previous one
        offs, cur = [], 0
        for n in sizes:
            cur += int(rng.integers(0, 9))
            offs.append(cur)
            cur += n * D
        pool = torch.randn(cur + 1, generator=gen).to(xdt).to(DEV)
        views = [pool[o: o + n * D].view(n, D) for o, n in zip(offs, sizes)]
        experts = [v.cpu() for v in views]
        idx = torch.from_numpy(rng.integers(0, T, N))
        w = torch.rand(N, generator=gen)
        idd, wd = idx.to(DEV), w.to(DEV).requires_grad_(True)
        leaf = pool.clone()
        xs = [leaf[o: o + n * D].view(n, D).requires_grad_(True) for o, n in zip(offs, sizes)]
        label = f"case {case}: T={T} E={E} N={N} D={D} {xdt} offsets {offs[:4]}"
        out = fastmoe_amd.grouped_weighted_scatter_add(xs, idd, wd, (T, D))
        want, acc, _ = oracle_fwd(experts, idx, w, T, xdt)
        np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32
                                      else want, err_msg=label)
        # grad_out at an odd element offset with an odd row padding
        go = torch.randn(T, D, generator=gen).to(xdt)
        pad, o = int(rng.integers(1, 6)), int(rng.integers(1, 8))
        gpool = torch.zeros(o + T * (D + pad), dtype=xdt, device=DEV)
        god = gpool[o:].as_strided((T, D), (D + pad, 1))
        god.copy_(go.to(DEV))
        grads = torch.autograd.grad(out, [wd, *xs], god)
        want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
        got_gx = np.concatenate([to_np(g).reshape(-1, D) for g in grads[1:]])
        np.testing.assert_array_equal(got_gx.view(want_gx.dtype), want_gx, err_msg=label)
        scale = abs_dot(experts, idx, go, T)
        err = np.abs(grads[0].double().cpu().numpy() - want_gw)
        assert np.all(err <= 1e-6 * scale + 1e-30), label
        # in place into an out view at an odd offset with padded rows: accumulates
        odt = dts[int(rng.integers(3))]
        prior = torch.randn(T, D, generator=gen).to(odt)
        opool = torch.zeros(o + T * (D + pad), dtype=odt, device=DEV)
        oview = opool[o:].as_strided((T, D), (D + pad, 1))
        oview.copy_(prior.to(DEV))
        fastmoe_amd.grouped_weighted_scatter_add(views, idd, wd.detach(), (T, D), out=oview,
                                                 mode="det")
        want_ip, _, _ = oracle_fwd(experts, idx, w, T, odt, acc_init=to_np(prior.float()).copy())
        np.testing.assert_array_equal(bits(oview), want_ip.view(np.uint32)
                                      if want_ip.dtype == np.float32 else want_ip, err_msg=label)


def test_random_inplace_against_oracle():
    """30 seeded random in-place calls (ops.py:389-390: accumulate into the given out): out in
    fp32, bf16 or f16 with random prior contents and sometimes a padded row stride; the
    deterministic mode bit-exact against the oracle started from out's values, the atomic mode
    (fp32 out) within the reordering bound."""
    rng = np.random.default_rng(77)
    dts = [torch.float32, torch.bfloat16, torch.float16]
    for case in range(30):
        T = int(rng.choice([1, 5, 64, 700, 2000]))
        E = int(rng.integers(1, 100))
        N = int(rng.integers(1, 4000))
        D = int(rng.choice([8, 24, 256, 1000, 2048]))
        pad = int(rng.choice([0, 0, 8, 40]))
        xdt, odt = dts[int(rng.integers(3))], dts[int(rng.integers(3))]
        mode = "atomic" if case % 4 == 1 else "det"
        gen = torch.Generator().manual_seed(100 + case)
        cuts = np.sort(rng.integers(0, N + 1, E - 1))
        sizes = np.diff(np.concatenate([[0], cuts, [N]])).tolist()
        idx = torch.from_numpy(rng.integers(0, T, N))
        w = torch.rand(N, generator=gen)
        experts = [torch.randn(n, D, generator=gen).to(xdt) for n in sizes]
        init = torch.randn(T, D, generator=gen).to(odt)
        big = torch.zeros(T, D + pad, dtype=odt, device=DEV)
        out = big[:, :D]
        out.copy_(init.to(DEV))
        xd, idd, wd = _to_dev(experts, idx, w)
        fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), out=out, mode=mode)
        torch.cuda.synchronize()
        label = f"case {case}: T={T} E={E} N={N} D={D} pad={pad} {xdt} out {odt} {mode}"
        want, acc, _ = oracle_fwd(experts, idx, w, T, odt, acc_init=init.float().numpy())
        if mode == "det":
            np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32
                                          else want, err_msg=label)
        else:
            kmax = int(np.bincount(idx.numpy(), minlength=T).max())
            scale = abs_sum(experts, idx, w, T) + np.abs(init.float().numpy())
            if odt == torch.float32:
                assert np.all(np.abs(out.cpu().numpy() - acc) <= reorder_tol(kmax + 1, scale)), label
            else:  # fp32 accumulation from the 16-bit initial contents, one rounding
                want16 = torch.from_numpy(want.view(np.int16)).view(odt).float().numpy()
                assert np.all(within_one_ulp16(out.float().cpu().numpy(), want16, odt, kmax + 1,
                                               scale)), label
        if pad:
            assert not bool(big[:, D:].any()), label  # the padding columns are never written


@pytest.mark.parametrize("path", list(_PLAN_PATHS))
@pytest.mark.parametrize("T,N", [(1, 1), (1, 5000), (2, 3), (2, 4500), (1, 100_000)])
def test_plan_few_tokens(T, N, path, kernel_options):
    """One or two tokens: a segment of thousands of rows (several partition slices feeding one
    bucket) and out-of-range indices mixed in; the plan (in exact stable order, with the longest
    segment recorded) and the forward against the oracle.  One token with 100,000 rows is the
    regression case of the plan's linear time (an ordering pass quadratic in the segment length
    takes minutes there); the one-launch plan's waves overflow their stashes there and
    re-stream their rows."""
    from oracle import cref

    kernel_options(plan=_PLAN_PATHS[path])
    gen = torch.Generator().manual_seed(43 + N)
    D = 12
    idx = torch.randint(0, T, (N,), generator=gen)
    idx[::7] = T          # out of range, both sides
    idx[3::11] = -2
    w = torch.rand(N, generator=gen)
    sizes = [N // 3, N - 2 * (N // 3), N // 3]
    experts = [torch.randn(n, D, generator=gen) for n in sizes]
    xd, idd, wd = _to_dev(experts, idx, w)
    meta, plan = ops.prepare_metadata_and_plan(xd, idd, wd, T)
    lib = fastmoe_amd._abi.lib()
    rp = plan[lib.fmoe_plan_row_ptr_offset(N, T):][: 4 * (T + 2)].view(torch.int32).cpu().numpy()
    rec = plan[lib.fmoe_plan_records_offset(N, T):][: 16 * N].view(torch.int64).view(N, 2).cpu()
    want_rp, want_g = cref.plan(idx.numpy(), T)
    np.testing.assert_array_equal(rp, want_rp)
    g = (rec[:, 1] >> 32).numpy().astype(np.int32)
    np.testing.assert_array_equal(g, want_g)  # every segment in ascending g
    st = ops.plan_status(plan).cpu().numpy()
    assert int(st[0]) == int((want_rp[T + 1] - want_rp[T]))
    assert int(st[2]) == (-1 if path in _NO_LONGEST else int(np.diff(want_rp)[:T].max()))
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D))
    want, _, bad = oracle_fwd(experts, idx, w, T, torch.float32)
    assert bad == want_rp[T + 1] - want_rp[T]
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))


def _sorted_plan(plan, N, T):
    """row_ptr, records ordered by g within every segment, and status words 0-1 of a plan."""
    lib = fastmoe_amd._abi.lib()
    h = plan.cpu()
    rp = h[lib.fmoe_plan_row_ptr_offset(N, T):][: 4 * (T + 2)].view(torch.int32).numpy()
    rec = h[lib.fmoe_plan_records_offset(N, T):][: 16 * N].view(torch.int64).view(N, 2).numpy()
    g = (rec[:, 1] >> 32).astype(np.int32)
    order = np.concatenate([np.arange(rp[b], rp[b + 1])[np.argsort(g[rp[b]:rp[b + 1]])]
                            for b in range(T + 1)]) if N else np.zeros(0, dtype=np.int64)
    return rp, rec[order], ops.plan_status(plan).cpu().numpy()[:2]


@pytest.mark.parametrize("case", ["e256", "e300", "e1", "empty_experts", "long", "i32_bf16w",
                                  "big_n", "big_n_long"])
def test_metadata_and_plan_in_one_call_equals_two_calls(case):
    """fmoe_build_metadata_and_plan writes exactly what fmoe_build_metadata + fmoe_build_plan
    write: the plan's own launches for up to 256 experts, the two calls otherwise (300 experts,
    or the radix plan: N > 2^20 rows over 4096 tokens averages 256 rows per token; over 65536
    tokens the ranged plan takes them in the one call)."""
    gen = torch.Generator().manual_seed(31)
    D, dtype, idt, wdt = 8, torch.float32, torch.int64, torch.float32
    if case in ("big_n", "big_n_long"):
        E, T, N, D = 16, 65536 if case == "big_n" else 4096, (1 << 20) + 5, 1
    else:
        E, T, N = {"e256": (256, 512, 4096), "e300": (300, 512, 4096), "e1": (1, 64, 500),
                   "empty_experts": (40, 100, 700), "long": (8, 40, 3000),
                   "i32_bf16w": (64, 256, 2048)}[case]
    if case == "i32_bf16w":
        idt, wdt, dtype = torch.int32, torch.bfloat16, torch.bfloat16
    cuts = torch.sort(torch.randint(0, N + 1, (E - 1,), generator=gen)).values.tolist()
    sizes = [b - a for a, b in zip([0] + cuts, cuts + [N])]
    if case == "empty_experts":
        sizes = [0] * 20 + sizes[20:-1] + [sizes[-1] + sum(sizes[:20])]
    hot = 3 if case == "long" else T
    idx = torch.randint(0, hot, (N,), generator=gen).to(idt)
    w = torch.rand(N, generator=gen).to(wdt)
    xs = [torch.randn(n, D, generator=gen).to(dtype).to(DEV) for n in sizes]
    idd, wd = idx.to(DEV), w.to(DEV)
    meta1, plan1 = ops.prepare_metadata_and_plan(xs, idd, wd, T)
    meta2 = fastmoe_amd.prepare_grouped_metadata(xs, DEV)
    plan2 = fastmoe_amd.build_plan(meta2, idd, wd, T)
    torch.cuda.synchronize()
    assert meta1.sizes == meta2.sizes and meta1.max_rows == meta2.max_rows
    for a, b in [(meta1.ptr_table, meta2.ptr_table), (meta1.chunk_sizes, meta2.chunk_sizes),
                 (meta1.offsets_full, meta2.offsets_full),
                 (meta1.max_rows_device, meta2.max_rows_device)]:
        assert torch.equal(a, b)
    rp1, rec1, st1 = _sorted_plan(plan1, N, T)
    rp2, rec2, st2 = _sorted_plan(plan2, N, T)
    np.testing.assert_array_equal(rp1, rp2)
    np.testing.assert_array_equal(rec1, rec2)
    np.testing.assert_array_equal(st1, st2)
    if case == "long":  # segments over 64 rows come out in ascending g
        g = (rec1[:, 1] >> 32).astype(np.int32)
        lib = fastmoe_amd._abi.lib()
        raw = plan1.cpu()[lib.fmoe_plan_records_offset(N, T):][: 16 * N].view(torch.int64)
        graw = (raw.view(N, 2)[:, 1].numpy() >> 32).astype(np.int32)
        for b in range(T):
            if rp1[b + 1] - rp1[b] > 64:
                assert np.array_equal(graw[rp1[b]:rp1[b + 1]], g[rp1[b]:rp1[b + 1]])


@pytest.mark.parametrize("path", ["auto", "bucketed"])
@pytest.mark.parametrize("case", ["topk", "long", "one_token", "invalid_i32", "empty", "bigT"])
def test_invert_scatter_index_matches_oracle(case, path, kernel_options):
    """fmoe_invert_scatter_index: row_ptr and the row list equal the oracle's stable inverse
    exactly -- top-k routing, segments longer than 64 rows (one of 3000 rows), out-of-range int32
    indices, no rows, and T above the LDS histogram (the global count path) -- through the
    automatic path (the radix plan) and the bucketed plan (option plan=2)."""
    from oracle import cref

    kernel_options(plan=0 if path == "auto" else _PLAN_PATHS["bucketed"])
    gen = torch.Generator().manual_seed(21)
    if case == "topk":
        _, T, idx, _, _ = _inputs("gigachat")
    elif case == "long":
        T = 40
        idx = torch.cat([torch.randint(0, 3, (300,), generator=gen),
                         torch.randint(0, T, (200,), generator=gen)])
        idx = idx[torch.randperm(idx.numel(), generator=gen)]
    elif case == "one_token":
        T, idx = 8, torch.randint(0, 2, (3000,), generator=gen)
    elif case == "invalid_i32":
        T = 64
        idx = torch.randint(0, T, (1000,), generator=gen)
        idx[::37] = -1
        idx[5::41] = T
        idx = idx.to(torch.int32)
    elif case == "empty":
        T, idx = 16, torch.zeros(0, dtype=torch.int64)
    else:
        T, idx = 40000, torch.randint(0, 40000, (80000,), generator=gen)
    row_ptr, rows = fastmoe_amd.invert_scatter_index(idx.to(DEV), T)
    want_rp, want_rows = cref.plan(idx.to(torch.int64).numpy(), T)
    np.testing.assert_array_equal(row_ptr.cpu().numpy(), want_rp)
    np.testing.assert_array_equal(rows.cpu().numpy(), want_rows)
    if case == "long":
        assert np.diff(want_rp)[:T].max() > 64
    if case == "invalid_i32":
        assert want_rp[T + 1] - want_rp[T] > 0


def test_metadata_matches_closed_forms():
    gen = torch.Generator().manual_seed(8)
    for E in (1, 7, 256, 300, 600):
        sizes = torch.randint(0, 5, (E,), generator=gen).tolist()
        sizes[E // 2] = 9
        experts = [torch.zeros(n, 8, device=DEV) for n in sizes]
        meta = fastmoe_amd.prepare_grouped_metadata(experts, DEV)
        ptr_table, chunk_sizes, expert_offsets, max_rows, num_experts = meta
        assert num_experts == E and max_rows == max(sizes)
        assert chunk_sizes.cpu().tolist() == sizes
        want_off = np.concatenate([[0], np.cumsum(sizes)])
        np.testing.assert_array_equal(meta.offsets_full.cpu().numpy(), want_off)
        np.testing.assert_array_equal(expert_offsets.cpu().numpy(), want_off[:E])
        got_ptr = ptr_table.cpu().tolist()
        assert got_ptr == [x.data_ptr() if n else 0 for x, n in zip(experts, sizes)]
        assert int(meta.max_rows_device.item()) == max(sizes)


@pytest.mark.parametrize("tile", [0, 44, 42, 28, 24, 18])
def test_fwd_det_every_tile_shape(tile, kernel_options):
    """The deterministic forward with each tile shape (option fwd_tile <U><R>: U vectors per lane
    per row, R rows per batch; 0 = the automatic choice by D and the rows per token) is the oracle's
    result bit for bit: segments of 1, 2 and 8 rows and ragged ones, D that the chunk divides and
    D that leaves a partial chunk, bf16 and fp32, overwrite and in-place accumulation."""
    kernel_options(fwd_tile=tile)
    gen = torch.Generator().manual_seed(400 + tile)
    for T, D, k, dt in [(300, 7168, 1, torch.bfloat16), (300, 7168, 2, torch.bfloat16),
                        (200, 3072, 8, torch.bfloat16), (257, 4104, 2, torch.bfloat16),
                        (150, 2048, 3, torch.float32), (64, 520, 1, torch.float32)]:
        N = T * k
        idx = torch.randperm(N, generator=gen) % T  # exactly k rows per token, scattered
        if k == 3:
            idx[::5] = torch.randint(0, 7, (len(idx[::5]),), generator=gen)  # ragged
        w = torch.rand(N, generator=gen)
        sizes = [N // 3, N - 2 * (N // 3), N // 3]
        experts = [torch.randn(n, D, generator=gen).to(dt) for n in sizes]
        xd, idd, wd = _to_dev(experts, idx, w)
        label = f"tile {tile}: T={T} D={D} k={k} {dt}"
        out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), mode="det")
        want, _, _ = oracle_fwd(experts, idx, w, T, dt)
        np.testing.assert_array_equal(bits(out), want.view(np.uint32) if want.dtype == np.float32
                                      else want, err_msg=label)
        init = torch.randn(T, D, generator=gen).to(dt)
        acc = init.to(DEV)
        fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), out=acc, mode="det")
        want, _, _ = oracle_fwd(experts, idx, w, T, dt, acc_init=init.float().numpy())
        np.testing.assert_array_equal(bits(acc), want.view(np.uint32) if want.dtype == np.float32
                                      else want, err_msg=label + " in place")


@pytest.mark.parametrize("D", [1, 256])
@pytest.mark.parametrize("kind", ["sum", "row_broadcast"])
def test_backward_of_an_expanded_grad_output(kind, D):
    """grad_output as autograd hands it over from a reduction or a broadcast: ``out.sum()`` gives
    an expanded all-ones tensor (strides (0, 0)), and a [1, D] row expanded to [T, D] has row
    stride 0.  grad_X bit-exact and grad_w within 1e-6 of sum|terms| against the oracle."""
    gen = torch.Generator().manual_seed(71 + D)
    T, sizes = 40, [30, 0, 50, 20]
    N = sum(sizes)
    idx = torch.randint(0, T, (N,), generator=gen)
    w = torch.rand(N, generator=gen)
    experts = [torch.randn(n, D, generator=gen).to(torch.bfloat16) for n in sizes]
    xs = [x.to(DEV).requires_grad_(True) for x in experts]
    wd = w.to(DEV).requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx.to(DEV), wd, (T, D))
    if kind == "sum":
        grads = torch.autograd.grad(out.sum(), [wd, *xs], allow_unused=True)
        go = torch.ones(T, D).to(torch.bfloat16)
    else:
        row = torch.randn(1, D, generator=gen).to(torch.bfloat16)
        god = row.to(DEV).expand(T, D)
        assert god.stride(0) == 0
        grads = torch.autograd.grad(out, [wd, *xs], god, allow_unused=True)
        go = row.expand(T, D).contiguous()
    torch.cuda.synchronize()
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
    got_gx = np.concatenate([to_np(g) for g, n in zip(grads[1:], sizes) if n])
    np.testing.assert_array_equal(got_gx, want_gx)
    scale = abs_dot(experts, idx, go, T)
    assert np.all(np.abs(grads[0].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


@pytest.mark.parametrize("path", ["auto", "bucketed"])
def test_many_experts_beyond_the_lds_tables(path, kernel_options):
    """5000 experts (0-2 rows each): more than the plan's LDS expert tables (4096) and the
    metadata's kernel-argument table (256), so the plan looks experts up in global memory and
    metadata and plan take separate calls -- the automatic plan (radix) and the bucketed plan;
    forward bits, grad_X bits and grad_w against the oracle."""
    kernel_options(plan=0 if path == "auto" else _PLAN_PATHS["bucketed"])
    gen = torch.Generator().manual_seed(41)
    E, T, D = 5000, 700, 24
    sizes = torch.randint(0, 3, (E,), generator=gen).tolist()
    N = sum(sizes)
    idx = torch.randint(0, T, (N,), generator=gen)
    w = torch.rand(N, generator=gen)
    experts = [torch.randn(n, D, generator=gen).to(torch.bfloat16) for n in sizes]
    xs = [x.to(DEV).requires_grad_(True) for x in experts]
    wd = w.to(DEV).requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx.to(DEV), wd, (T, D))
    go = torch.randn(T, D, generator=gen).to(torch.bfloat16)
    grads = torch.autograd.grad(out, [wd, *xs], go.to(DEV), allow_unused=True)
    torch.cuda.synchronize()
    want, _, _ = oracle_fwd(experts, idx, w, T, torch.bfloat16)
    np.testing.assert_array_equal(bits(out), want)
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
    got_gx = np.concatenate([to_np(g) for g, n in zip(grads[1:], sizes) if n])
    np.testing.assert_array_equal(got_gx, want_gx)
    scale = abs_dot(experts, idx, go, T)
    assert np.all(np.abs(grads[0].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


@pytest.mark.parametrize("path", list(_PLAN_PATHS))
def test_large_token_count_plan_paths(path, kernel_options):
    """T = 40000: the radix plan sorts in two 8-bit passes and scans row_ptr over three blocks of
    16384 bins; the bucketed plan groups the 40001 bins into buckets of 64; the one-launch plan
    spreads them over 255 workgroups."""
    kernel_options(plan=_PLAN_PATHS[path])
    D, T, k = 16, 40000, 2
    wl = Workload("bigT", T, D, 16, k, torch.float32, 13, False)
    idx, w, counts = make_routing(wl)
    experts = make_experts(counts, D, torch.float32, "cpu", 13)
    xd, idd, wd = _to_dev(experts, idx, w)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D))
    want, _, _ = oracle_fwd(experts, idx, w, T, torch.float32)
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))


@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
def test_plan_beyond_bucketed_token_limit(idx_dtype):
    """T = 5,000,000 token bins, above the bucketed plan's 2^22: the automatic choice takes the
    radix plan (three 8-bit passes).  Random rows over all of T, one token with about 89,000 rows
    (the regression case of linear time: an ordering pass quadratic in the segment length takes
    minutes there) and out-of-range indices on both sides; the plan (exact stable order, status
    words), the bare inverse and the forward against the oracle."""
    from oracle import cref

    gen = torch.Generator().manual_seed(97)
    T, N, D = 5_000_000, 300_000, 4
    idx = torch.randint(0, T, (N,), generator=gen)
    idx[torch.randperm(N, generator=gen)[:100_000]] = 4_321_987
    idx[::13] = T   # out of range, both sides (about 11% of the rows)
    idx[5::29] = -3
    idx = idx.to(idx_dtype)
    w = torch.rand(N, generator=gen)
    sizes = [N // 4, N // 2, N - N // 4 - N // 2]
    experts = [torch.randn(n, D, generator=gen) for n in sizes]
    xd, idd, wd = _to_dev(experts, idx, w)
    meta, plan = ops.prepare_metadata_and_plan(xd, idd, wd, T)
    lib = fastmoe_amd._abi.lib()
    rp = plan[lib.fmoe_plan_row_ptr_offset(N, T):][: 4 * (T + 2)].view(torch.int32).cpu().numpy()
    rec = plan[lib.fmoe_plan_records_offset(N, T):][: 16 * N].view(torch.int64).view(N, 2).cpu()
    want_rp, want_g = cref.plan(idx.to(torch.int64).numpy(), T)
    np.testing.assert_array_equal(rp, want_rp)
    np.testing.assert_array_equal((rec[:, 1] >> 32).numpy().astype(np.int32), want_g)
    np.testing.assert_array_equal((rec[:, 1] & 0xFFFFFFFF).numpy().astype(np.uint32),
                                  w.numpy()[want_g].view(np.uint32))
    seg = np.diff(want_rp)
    assert seg[:T].max() > 80_000  # the hot token, less the rows sent out of range below
    st = ops.plan_status(plan).cpu().numpy()
    assert int(st[0]) == int(seg[T]) and int(st[1]) == 0 and int(st[2]) == int(seg[:T].max())
    row_ptr, rows = fastmoe_amd.invert_scatter_index(idd, T)
    np.testing.assert_array_equal(row_ptr.cpu().numpy(), want_rp)
    np.testing.assert_array_equal(rows.cpu().numpy(), want_g)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D))
    want, _, bad = oracle_fwd(experts, idx.to(torch.int64), w, T, torch.float32)
    assert bad == seg[T]
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))


@pytest.mark.parametrize("mode", ["det", "atomic"])
def test_graph_capture_replays(mode):
    """In-place launch with precomputed metadata captured in a graph (run_on_cloud.py:66-92): every
    replay (with eager work in between) equals the oracle -- bit for bit in det mode, within the
    gap of two fp32 summation orders in atomic mode -- and the eager call."""
    wl, T, idx, w, experts = _inputs("gigachat", T=128)
    xd, idd, wd = _to_dev(experts, idx, w)
    want, acc, _ = oracle_fwd(experts, idx, w, T, torch.float32)
    k = int(np.bincount(idx.numpy(), minlength=T).max())
    scale = abs_sum(experts, idx, w, T)

    def check(out):
        if mode == "det":
            np.testing.assert_array_equal(bits(out), want.view(np.uint32))
        else:
            assert np.all(np.abs(out.cpu().numpy() - acc) <= reorder_tol(k, scale))

    meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
    out_static = torch.zeros(T, wl.D, dtype=torch.float32, device=DEV)
    fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), out=out_static, metadata=meta,
                                             mode=mode)
    torch.cuda.synchronize()
    check(out_static)
    eager = out_static.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        out_static.zero_()
        with torch.cuda.graph(g, stream=s):
            fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, wl.D), out=out_static,
                                                     metadata=meta, mode=mode)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(4):
        out_static.zero_()
        g.replay()
        torch.cuda.synchronize()
        check(out_static)
        if mode == "det":
            np.testing.assert_array_equal(bits(out_static), bits(eager))
        _ = (torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)).sum().item()


@pytest.mark.skip(reason="its one run (det mode, on the host path of commit b95310e) ended in a "
                         "host segmentation fault inside torch.cuda.CUDAGraph.capture_end, with no "
                         "GPU fault; no cause has been shown in this library's code, so the case "
                         "stays off the GPU and the library refuses such a capture with an error "
                         "(test_autograd_step_under_capture_raises)")
@pytest.mark.parametrize("mode", ["det", "atomic"])
def test_graph_capture_autograd_step_replays(mode):
    """The bench's timed step -- metadata, plan, forward and both backward passes through the
    autograd API -- captured once as a graph: every replay (with eager work in between) equals the
    oracle (forward and grad_X bits in det mode, the one-ulp bar in atomic mode with its fp32
    accumulator; grad_X bit for bit and grad_w within 1e-6 of sum|terms| in both) and, in det mode,
    the eager step bit for bit."""
    wl, T, idx, w, experts = _inputs("gigachat", T=128)
    xd, idd, wd = _to_dev(experts, idx, w)
    xs = [x.requires_grad_(True) for x in xd]
    wd.requires_grad_(True)
    go_cpu = torch.randn(T, wl.D, generator=torch.Generator().manual_seed(5)).to(wl.dtype)
    go = go_cpu.to(DEV)
    inputs = [wd, *xs]
    want, _, _ = oracle_fwd(experts, idx, w, T, wl.dtype)
    want16 = torch.from_numpy(want.view(np.int16)).view(wl.dtype).float().numpy()
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go_cpu)
    scale_fwd = abs_sum(experts, idx, w, T)
    scale_gw = abs_dot(experts, idx, go_cpu, T)
    k = int(np.bincount(idx.numpy(), minlength=T).max())

    def step():
        out = fastmoe_amd.grouped_weighted_scatter_add(xs, idd, wd, (T, wl.D), mode=mode)
        return (out, *torch.autograd.grad(out, inputs, go))

    def check(res):
        out, gw, gx = res[0], res[1], res[2:]
        if mode == "det":
            np.testing.assert_array_equal(bits(out), want)
        else:
            assert np.all(within_one_ulp16(out.float().cpu().numpy(), want16, wl.dtype, k,
                                           scale_fwd))
        np.testing.assert_array_equal(np.concatenate([to_np(t) for t in gx]), want_gx)
        assert np.all(np.abs(gw.double().cpu().numpy() - want_gw) <= 1e-6 * scale_gw + 1e-30)

    first = step()
    check(first)
    eager = [bits(t) for t in first]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static = step()
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        check(static)
        if mode == "det":
            for got, want_bits in zip(static, eager):
                np.testing.assert_array_equal(bits(got), want_bits)
        _ = (torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)).sum().item()


class _DirectCtx:
    """The autograd context's part that GroupedWeightedScatterAdd's forward/backward functions
    use (save_for_backward / saved_tensors), for calling them without the autograd engine."""

    def save_for_backward(self, *tensors):
        self.saved_tensors = tensors


def test_autograd_step_under_capture_raises():
    """The autograd forward that records a backward raises a clear RuntimeError under HIP graph
    capture, before any launch of this library; the graph captured so far (one torch kernel)
    still replays."""
    wl, T, idx, w, experts = _inputs("gigachat", T=16)
    xd, idd, wd = _to_dev(experts, idx, w)
    xs = [x.requires_grad_(True) for x in xd]
    bump = torch.zeros(4, device=DEV)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="graph capture is not supported"):
        with torch.cuda.graph(g):
            bump.add_(1)
            fastmoe_amd.grouped_weighted_scatter_add(xs, idd, wd, (T, wl.D))
    g.replay()
    torch.cuda.synchronize()
    assert bump.tolist() == [1.0] * 4


# (mode, kernel option "small"): the planned step (metadata + plan, forward, grad_X pass, grad_w
# pass -- what bench.py times at the headline shape) and the one-launch small path.
_DIRECT_STEPS = [("det", 1), ("det", 2), ("atomic", 1)]


@pytest.mark.parametrize("mode,small", _DIRECT_STEPS,
                         ids=[f"{m}-{'planned' if s == 1 else 'small'}" for m, s in _DIRECT_STEPS])
def test_graph_capture_direct_step_replays(mode, small, kernel_options):
    """bench.py's timed step: the launches of one autograd step, issued by the autograd path's own
    forward and backward functions on this thread, captured once as a graph -- the planned step
    (metadata + plan, forward, grad_X and grad_w passes) and, in det mode, the small path's two
    launches.  Every replay (with eager work in between) equals the oracle -- forward and grad_X
    bit for bit in det mode, the one-ulp bar in atomic mode, grad_w within 1e-6 of sum|terms| --
    and, in det mode, the eager step bit for bit."""
    wl, T, idx, w, experts = _inputs("gigachat", T=128)
    kernel_options(small=small)
    if mode == "det":  # the atomic modes never take the small path
        assert ops._use_small(idx.numel(), T, len(experts)) == (small == 2)
    xd, idd, wd = _to_dev(experts, idx, w)
    go_cpu = torch.randn(T, wl.D, generator=torch.Generator().manual_seed(5)).to(wl.dtype)
    go = go_cpu.to(DEV)
    want, _, _ = oracle_fwd(experts, idx, w, T, wl.dtype)
    want16 = torch.from_numpy(want.view(np.int16)).view(wl.dtype).float().numpy()
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go_cpu)
    scale_fwd = abs_sum(experts, idx, w, T)
    scale_gw = abs_dot(experts, idx, go_cpu, T)
    k = int(np.bincount(idx.numpy(), minlength=T).max())

    def step():
        with torch.no_grad():
            ctx = _DirectCtx()
            out = ops._combine_forward(ctx, mode, None, idd, wd, (T, wl.D), xd, True)
            gw, gx = ops._combine_backward(ctx, go, True, [True] * len(xd))
        return (out, gw, *gx)

    def check(res):
        out, gw, gx = res[0], res[1], res[2:]
        if mode == "det":
            np.testing.assert_array_equal(bits(out), want)
        else:
            assert np.all(within_one_ulp16(out.float().cpu().numpy(), want16, wl.dtype, k,
                                           scale_fwd))
        np.testing.assert_array_equal(np.concatenate([to_np(t) for t in gx]), want_gx)
        assert np.all(np.abs(gw.double().cpu().numpy() - want_gw) <= 1e-6 * scale_gw + 1e-30)

    first = step()
    torch.cuda.synchronize()
    check(first)
    eager = [bits(t) for t in first]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static = step()
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        check(static)
        if mode == "det":
            for got, want_bits in zip(static, eager):
                np.testing.assert_array_equal(bits(got), want_bits)
        _ = (torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)).sum().item()


@pytest.mark.parametrize("name", ["gigachat"])
def test_full_size_fwd_bwd_parity(name):
    """The BASELINE headline config at its full size: forward bit-exact, grad_X bit-exact,
    grad_w within 1e-6 of sum|terms|, against the C oracle."""
    wl = WORKLOADS[name]
    idx, w, counts = make_routing(wl)
    xd = make_experts(counts, wl.D, wl.dtype, DEV, wl.seed)
    idd, wd = idx.to(DEV), w.to(DEV).requires_grad_(True)
    xg = [x.requires_grad_(True) for x in xd]
    out = fastmoe_amd.grouped_weighted_scatter_add(xg, idd, wd, (wl.T, wl.D))
    go = torch.randn(wl.T, wl.D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(1)).to(wl.dtype)
    grads = torch.autograd.grad(out, [wd, *xg], go)
    experts = [x.detach().cpu() for x in xd]
    want, _, _ = oracle_fwd(experts, idx, w, wl.T, wl.dtype)
    np.testing.assert_array_equal(bits(out), want)
    del want
    want_gx, want_gw = oracle_bwd(experts, idx, w, wl.T, go.cpu())
    got_gx = np.concatenate([to_np(g) for g in grads[1:]])
    np.testing.assert_array_equal(got_gx, want_gx)
    scale = abs_dot(experts, idx, go.cpu(), wl.T)
    assert np.all(np.abs(grads[0].double().cpu().numpy() - want_gw) <= 1e-6 * scale + 1e-30)


@pytest.mark.parametrize("name", ["mid", "skewed"])
def test_full_size_forward_parity(name):
    """BASELINE configs 2 and 4 at their full sizes: the deterministic forward is bit-exact
    against the C oracle (skewed: Zipf-biased routing with empty and hot experts)."""
    wl = WORKLOADS[name]
    idx, w, counts = make_routing(wl)
    xd = make_experts(counts, wl.D, wl.dtype, DEV, wl.seed)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idx.to(DEV), w.to(DEV), (wl.T, wl.D))
    torch.cuda.synchronize()
    if name == "skewed":
        assert 0 in counts and max(counts) > 1.5 * wl.N / wl.E  # empty and hot experts
    experts = [x.cpu() for x in xd]
    want, _, bad = oracle_fwd(experts, idx, w, wl.T, wl.dtype)
    assert bad == 0
    np.testing.assert_array_equal(bits(out), want)


def test_full_size_properties_gigachat():
    """Size-independent properties at the headline size: doubling every gate doubles every output
    bit pattern exactly (a power-of-two scale is exact through the fp32 products and sum and the
    bf16 rounding), and the same rows given as one concatenated expert tensor give the same bits
    as the 256 separate buffers."""
    wl = WORKLOADS["gigachat"]
    idx, w, counts = make_routing(wl)
    xd = make_experts(counts, wl.D, wl.dtype, DEV, wl.seed)
    idd, wd = idx.to(DEV), w.to(DEV)
    shape = (wl.T, wl.D)
    out = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, shape)
    out2 = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, 2 * wd, shape)
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out2, out * 2)
    del out2
    one = fastmoe_amd.grouped_weighted_scatter_add([torch.cat(xd)], idd, wd, shape)
    assert torch.equal(one.view(torch.int16), out.view(torch.int16))


def test_full_size_det_repeatable_and_atomic_bounded():
    """BASELINE config 5 at its full size (T=32768, D=16384, E=256, top-2, bf16): ten
    deterministic runs are bit-identical and equal the oracle; each of ten atomic runs (fp32
    accumulation, one rounding) is within one ulp of the deterministic result plus the gap of two
    fp32 summation orders, and a packed-atomic run within the (k + 2) u sum|terms| model."""
    wl = WORKLOADS["detatomic"]
    idx, w, counts = make_routing(wl)
    xd = make_experts(counts, wl.D, wl.dtype, DEV, wl.seed)
    idd, wd = idx.to(DEV), w.to(DEV)
    shape = (wl.T, wl.D)
    det = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, shape, mode="det")
    det_bits = det.view(torch.int16).clone()
    for _ in range(9):
        again = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, shape, mode="det")
        assert torch.equal(again.view(torch.int16), det_bits)
    want, _, bad = oracle_fwd([x.cpu() for x in xd], idx, w, wl.T, wl.dtype)
    assert bad == 0
    np.testing.assert_array_equal(bits(det), want)  # and bit-exact against the oracle
    del want
    # sum|terms| per output element, torch fp32 ops on the GPU (a tolerance scale only)
    scale = torch.zeros(shape, device=DEV)
    scale.index_add_(0, idd, torch.cat(xd).float().abs() * wd.abs()[:, None])
    det32 = det.float()
    # one ulp of bf16 at the larger magnitude (frexp exponent - 8), plus two orders' fp32 gap
    for _ in range(10):
        atom = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, shape, mode="atomic").float()
        big = torch.maximum(atom.abs(), det32.abs())
        _, ex = torch.frexp(big)
        ulp = torch.where(big == 0, torch.full_like(big, 2.0 ** -133),
                          torch.ldexp(torch.ones_like(big), ex - 8).clamp_min(2.0 ** -133))
        tol = ulp + 2 * (wl.k - 1) * 2.0 ** -24 * (1 + 2.0 ** -20) * scale
        assert bool(((atom - det32).abs() <= tol).all())
    packed = fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, shape, mode="atomic_packed")
    tol = (wl.k + 2) * 2.0 ** -8 * (1 + 2.0 ** -6) * scale + 2.0 ** -133
    assert bool(((packed.float() - det32).abs() <= tol).all())


def test_packed_atomics_refuse_16bit_output_without_vector_layout():
    """Packed 16-bit atomics need element pairs (D % 8 == 0 here); the fp32-accumulating atomic
    mode takes any layout and meets the one-ulp bar there."""
    D, T = 100, 8
    gen = torch.Generator().manual_seed(8)
    xc = torch.randn(6, D, generator=gen).to(torch.bfloat16)
    idx = torch.randint(0, T, (6,), generator=gen)
    w = torch.rand(6, generator=gen)
    x, idd, wd = xc.to(DEV), idx.to(DEV), w.to(DEV)
    with pytest.raises(ValueError, match="FMOE_MODE_ATOMIC"):
        fastmoe_amd.weighted_scatter_add(x, idd, wd, (T, D), mode="atomic_packed")
    out = fastmoe_amd.weighted_scatter_add(x, idd, wd, (T, D), mode="atomic")
    want, _, _ = oracle_fwd([xc], idx, w, T, torch.bfloat16)
    want16 = torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy()
    k = int(np.bincount(idx.numpy(), minlength=T).max())
    scale = abs_sum([xc], idx, w, T)
    assert np.all(within_one_ulp16(out.float().cpu().numpy(), want16, torch.bfloat16, max(k, 2),
                                   scale))


def _as_f32(raw: np.ndarray, dtype) -> np.ndarray:
    """Values of raw storage bits (uint16 for bf16/f16, float32 otherwise) as float32."""
    if dtype == torch.bfloat16:
        return (raw.astype(np.uint32) << 16).view(np.float32)
    if dtype == torch.float16:
        return raw.view(np.float16).astype(np.float32)
    return raw.view(np.float32)


def _same_non_finite(got_raw, want_raw, dtype):
    """NaN where the oracle has NaN (any payload), and the same bits everywhere else (+-Inf too)."""
    g, w = _as_f32(got_raw, dtype), _as_f32(want_raw, dtype)
    np.testing.assert_array_equal(np.isnan(g), np.isnan(w))
    keep = ~np.isnan(w)
    np.testing.assert_array_equal(got_raw[keep], want_raw[keep])


@pytest.mark.parametrize("small", [1, 2], ids=["planned", "small"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_non_finite_values_propagate_like_the_oracle(dtype, small, kernel_options):
    """+-Inf and NaN in the expert rows and in grad_out: the deterministic forward and grad_X have
    NaN exactly where the oracle does and the oracle's bits elsewhere (infinities included); grad_w
    is NaN where the oracle's is and within the usual bar where it is finite."""
    kernel_options(small=small)
    wl, T, idx, w, experts = _inputs("gigachat", T=32 if small == 2 else 160)
    gen = torch.Generator().manual_seed(41)
    experts = [x.clone() for x in experts]
    for i, x in enumerate(experts):
        if x.shape[0] and i % 5 == 0:
            x[0, i % wl.D] = float("inf")
            x[-1, (3 * i) % wl.D] = float("nan")
            x[x.shape[0] // 2, (7 * i) % wl.D] = float("-inf")
    experts = [x.to(dtype) for x in experts]
    xd, idd, wd = _to_dev(experts, idx, w)
    xs = [x.requires_grad_(True) for x in xd]
    wd.requires_grad_(True)
    grad_out = torch.randn(T, wl.D, generator=gen)
    grad_out[1, 5], grad_out[2, 6], grad_out[3, 7] = float("inf"), float("nan"), float("-inf")
    grad_out = grad_out.to(dtype)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idd, wd, (T, wl.D), mode="det")
    grads = torch.autograd.grad(out, [wd, *xs], grad_out.to(DEV))
    torch.cuda.synchronize()
    want, _, _ = oracle_fwd(experts, idx, w, T, dtype)
    want = want.view(np.uint32) if want.dtype == np.float32 else want
    assert np.isnan(_as_f32(want, dtype)).any() and np.isinf(_as_f32(want, dtype)).any()
    _same_non_finite(bits(out), want, dtype)
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, grad_out)
    want_gx = want_gx.view(np.uint32) if want_gx.dtype == np.float32 else want_gx
    got_gx = np.concatenate([to_np(g) for g in grads[1:]], 0)
    got_gx = got_gx.view(np.uint32) if got_gx.dtype == np.float32 else got_gx
    _same_non_finite(got_gx, want_gx, dtype)
    gw = grads[0].double().cpu().numpy()
    np.testing.assert_array_equal(np.isnan(gw), np.isnan(want_gw))
    fin = np.isfinite(want_gw)
    np.testing.assert_array_equal(gw[~fin & ~np.isnan(want_gw)], want_gw[~fin & ~np.isnan(want_gw)])
    scale = abs_dot(experts, idx, grad_out, T)
    assert np.all(np.abs(gw[fin] - want_gw[fin]) <= 1e-6 * scale[fin] + 1e-30)


@pytest.mark.parametrize("small", [1, 2], ids=["planned", "small"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_subnormal_values_are_kept_like_the_oracle(dtype, small, kernel_options):
    """Expert rows, gates and grad_out scaled into the subnormal range: no stage flushes them to
    zero, so the deterministic forward and grad_X equal the oracle bit for bit."""
    kernel_options(small=small)
    wl, T, idx, w, experts = _inputs("gigachat", T=32 if small == 2 else 160)
    tiny = 2.0 ** -130  # below float32's (and bfloat16's) smallest normal, 2^-126
    experts = [(x.float() * tiny).to(dtype) for x in experts]
    assert any(bool((x.float().abs() < 2.0 ** -126).logical_and(x.float() != 0).any())
               for x in experts)
    xd, idd, wd = _to_dev(experts, idx, w)
    xs = [x.requires_grad_(True) for x in xd]
    grad_out = (torch.randn(T, wl.D, generator=torch.Generator().manual_seed(43)) * tiny).to(dtype)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idd, wd, (T, wl.D), mode="det")
    gxs = torch.autograd.grad(out, xs, grad_out.to(DEV))
    torch.cuda.synchronize()
    want, _, _ = oracle_fwd(experts, idx, w, T, dtype)
    got = bits(out)
    np.testing.assert_array_equal(got, want.view(np.uint32) if want.dtype == np.float32 else want)
    assert np.count_nonzero(got) > got.size // 2  # most sums are subnormal, not flushed
    want_gx, _ = oracle_bwd(experts, idx, w, T, grad_out)
    got_gx = np.concatenate([to_np(g) for g in gxs], 0)
    np.testing.assert_array_equal(got_gx.view(np.uint32) if got_gx.dtype == np.float32 else got_gx,
                                  want_gx.view(np.uint32) if want_gx.dtype == np.float32 else want_gx)
