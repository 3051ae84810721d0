"""The Python host path end to end on the CPU, against a recording stand-in for the C library.

No kernel runs here: the stand-in checks and records the arguments every C-ABI entry point
receives (sizes, dtype codes, strides, pointer/None choices) so that marshalling mistakes in
fastmoe_amd/ops.py show up without a GPU.  Numerics are covered by the GPU parity tests.
"""
from __future__ import annotations

import contextlib

import pytest
import torch

import fastmoe_amd
from fastmoe_amd import _abi, ops


class FakeLib:
    def __init__(self):
        self.calls = []
        self.real = _abi.lib()

    def fmoe_abi_version(self):
        return _abi.ABI_VERSION

    def fmoe_last_error(self):
        return b"fake"

    def fmoe_set_option(self, name, value, prev):
        return self.real.fmoe_set_option(name, value, prev)

    def fmoe_get_option(self, name, value):
        return self.real.fmoe_get_option(name, value)

    def fmoe_build_metadata(self, host_ptrs, host_rows, E, ptr_table, chunk, offsets, max_rows,
                            stream):
        assert isinstance(E, int) and E >= 1
        assert len(host_ptrs) == E and len(host_rows) == E
        assert all(isinstance(p, int) for p in (ptr_table, chunk, offsets, max_rows))
        self.calls.append(("metadata", E, list(host_rows)))
        return 0

    def fmoe_plan_workspace_bytes(self, N, T):
        return self.real.fmoe_plan_workspace_bytes(N, T)

    def fmoe_plan_status_offset(self):
        return 0

    def fmoe_plan_row_ptr_offset(self, N, T):
        return self.real.fmoe_plan_row_ptr_offset(N, T)

    def fmoe_plan_records_offset(self, N, T):
        return self.real.fmoe_plan_records_offset(N, T)

    def fmoe_build_plan(self, idx, idt, w, wdt, N, T, ptr_table, offsets, E, row_bytes, ws, stream):
        assert idt in (_abi.I64, _abi.I32) and wdt in (_abi.F32, _abi.BF16, _abi.F16)
        assert all(isinstance(p, int) for p in (idx, w, ptr_table, offsets, ws))
        self.calls.append(("plan", N, T, E, row_bytes, idt, wdt))
        return 0

    def fmoe_build_metadata_and_plan(self, host_ptrs, host_rows, E, ptr_table, chunk, offsets,
                                     max_rows, idx, idt, w, wdt, T, row_bytes, ws, stream):
        assert isinstance(E, int) and E >= 1 and len(host_ptrs) == E and len(host_rows) == E
        assert idt in (_abi.I64, _abi.I32) and wdt in (_abi.F32, _abi.BF16, _abi.F16)
        assert all(isinstance(p, int) for p in (ptr_table, chunk, offsets, max_rows, idx, w, ws))
        self.calls.append(("metadata_plan", E, list(host_rows), T, row_bytes, idt, wdt))
        return 0

    def fmoe_build_metadata_and_plan_from_slots(self, host_ptrs, host_rows, E, ptr_table, chunk,
                                                offsets, max_rows, slot_pos, T, k, w, wdt,
                                                row_bytes, ws, stream):
        assert isinstance(E, int) and E >= 1 and len(host_ptrs) == E and len(host_rows) == E
        assert wdt in (_abi.F32, _abi.BF16, _abi.F16) and 1 <= k <= 64
        assert all(isinstance(p, int) for p in (ptr_table, chunk, offsets, max_rows, slot_pos, w, ws))
        self.calls.append(("metadata_plan_slots", E, list(host_rows), T, k, row_bytes, wdt))
        return 0

    def fmoe_combine_fwd_workspace_bytes(self, mode, T, D, odt):
        return self.real.fmoe_combine_fwd_workspace_bytes(mode, T, D, odt)

    def fmoe_combine_fwd(self, mode, plan, idx, idt, w, wdt, ptr_table, offsets, E, N, T, D, xdt,
                         out, odt, ostride, acc, ws, ws_bytes, stream):
        if mode == _abi.MODE_DET:
            assert isinstance(plan, int)
        else:
            assert isinstance(idx, int) and isinstance(w, int)
        need = self.real.fmoe_combine_fwd_workspace_bytes(mode, T, D, odt)
        assert ws_bytes >= need and (need == 0 or isinstance(ws, int))
        self.calls.append(("fwd", mode, N, T, D, xdt, odt, ostride, acc))
        return 0

    def fmoe_combine_bwd(self, plan, N, T, D, xdt, gout, gdt, gstride, gx, gw, gwdt, stream):
        assert isinstance(plan, int) and isinstance(gout, int) and gdt == xdt
        self.calls.append(("bwd", N, T, D, xdt, gstride, gx is not None, gw is not None, gwdt))
        return 0

    def fmoe_combine_small_max_rows(self):
        return self.real.fmoe_combine_small_max_rows()

    def fmoe_combine_fwd_small(self, host_ptrs, host_rows, E, idx, idt, w, wdt, T, D, xdt, out,
                               odt, ostride, acc, status, stream):
        assert isinstance(E, int) and len(host_ptrs) == E and len(host_rows) == E
        assert idt in (_abi.I64, _abi.I32) and wdt in (_abi.F32, _abi.BF16, _abi.F16)
        assert all(isinstance(p, int) for p in (idx, w, out, status))
        self.calls.append(("fwd_small", E, list(host_rows), T, D, idt, wdt, xdt, odt, ostride,
                           acc))
        return 0

    def fmoe_combine_bwd_small(self, host_ptrs, host_rows, E, idx, idt, w, wdt, T, D, xdt, gout,
                               gdt, gstride, gx, gw, gwdt, stream):
        assert isinstance(E, int) and len(host_ptrs) == E and len(host_rows) == E
        assert all(isinstance(p, int) for p in (idx, w, gout)) and gdt == xdt
        self.calls.append(("bwd_small", E, list(host_rows), T, D, xdt, gstride, gx is not None,
                           gw is not None, gwdt))
        return 0


def _fake_lib(monkeypatch):
    f = FakeLib()
    monkeypatch.setattr(_abi, "lib", lambda: f)
    monkeypatch.setattr(ops, "_require_cuda", lambda t, what: None)
    monkeypatch.setattr(ops, "_stream_handle", lambda dev: 0)
    monkeypatch.setattr(ops, "_on_device", lambda dev: contextlib.nullcontext())
    return f


@pytest.fixture
def fake(monkeypatch):
    """The planned path (metadata + plan, forward, backward passes): the small path is off."""
    f = _fake_lib(monkeypatch)
    with _abi.options(small=1):
        yield f


@pytest.fixture
def fake_small(monkeypatch):
    """The default choice, which takes the one-launch small path for these sizes."""
    f = _fake_lib(monkeypatch)
    with _abi.options(small=0):
        yield f


def _experts(dtype=torch.bfloat16, sizes=(3, 0, 5), D=16):
    return [torch.randn(n, D).to(dtype) for n in sizes]


def test_autograd_forward_and_backward_calls(fake):
    xs = [x.requires_grad_(True) for x in _experts()]
    N = 8
    idx = torch.randint(0, 4, (N,))
    w = torch.rand(N, requires_grad=True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16))
    assert out.shape == (4, 16) and out.dtype == torch.bfloat16
    grads = torch.autograd.grad(out, [w, *xs], torch.ones(4, 16, dtype=torch.bfloat16))
    kinds = [c[0] for c in fake.calls]
    assert kinds == ["metadata_plan", "fwd", "bwd"]
    assert fake.calls[0] == ("metadata_plan", 3, [3, 0, 5], 4, 32, _abi.I64, _abi.F32)
    assert fake.calls[1] == ("fwd", _abi.MODE_DET, 8, 4, 16, _abi.BF16, _abi.BF16, 16, 0)
    # one call with both outputs (the library runs the grad_X pass, then the grad_w pass)
    assert fake.calls[2] == ("bwd", 8, 4, 16, _abi.BF16, 16, True, True, _abi.F32)
    assert grads[0].shape == (N,) and grads[0].dtype == torch.float32
    assert [g.shape[0] for g in grads[1:]] == [3, 0, 5]


class _Timer:
    def __init__(self):
        self.names = []

    def span(self, name):
        self.names.append(name)
        return contextlib.nullcontext()


def test_timed_backward_issues_each_pass_in_its_own_span(fake, monkeypatch):
    timer = _Timer()
    monkeypatch.setattr(ops, "_TIMER", timer)
    xs = [x.requires_grad_(True) for x in _experts()]
    w = torch.rand(8, requires_grad=True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.randint(0, 4, (8,)), w, (4, 16))
    torch.autograd.grad(out, [w, *xs], torch.ones(4, 16, dtype=torch.bfloat16))
    assert timer.names == ["metadata_plan", "fwd_det", "bwd_gx", "bwd_gw"]
    # grad_X pass, then grad_w pass
    assert fake.calls[2] == ("bwd", 8, 4, 16, _abi.BF16, 16, True, False, _abi.F32)
    assert fake.calls[3] == ("bwd", 8, 4, 16, _abi.BF16, 16, False, True, _abi.F32)


def test_fused_backward_is_one_call(fake):
    xs = [x.requires_grad_(True) for x in _experts()]
    w = torch.rand(8, requires_grad=True)
    with _abi.options(bwd_fused=1):
        out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.randint(0, 4, (8,)), w, (4, 16))
        torch.autograd.grad(out, [w, *xs], torch.ones(4, 16, dtype=torch.bfloat16))
    assert [c[0] for c in fake.calls] == ["metadata_plan", "fwd", "bwd"]
    assert fake.calls[2][6:8] == (True, True)


def test_backward_skips_unneeded_outputs(fake):
    xs = _experts(torch.float32)
    w = torch.rand(8, requires_grad=True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long), w, (2, 16))
    torch.autograd.grad(out, [w], torch.ones(2, 16))
    assert fake.calls[-1][6:8] == (False, True)
    fake.calls.clear()
    xs = [x.requires_grad_(True) for x in _experts(torch.float32)]
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long),
                                                   torch.rand(8), (2, 16))
    torch.autograd.grad(out, xs, torch.ones(2, 16))
    assert fake.calls[-1][6:8] == (True, False)


def test_atomic_mode_overwrites_and_defers_the_plan(fake):
    xs = _experts(torch.float32)
    out = torch.full((4, 16), 3.0)
    meta = fastmoe_amd.prepare_grouped_metadata(xs, "cuda")
    assert len(meta) == 5 and meta[3] == 5 and meta[4] == 3
    ptr_table, chunk_sizes, expert_offsets, max_rows, num_experts = meta
    assert expert_offsets.numel() == 3 and meta.offsets_full.numel() == 4
    fake.calls.clear()
    ret = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.int32),
                                                   torch.rand(8), (4, 16), out=out, metadata=meta,
                                                   mode="atomic")
    assert ret is out and torch.all(out == 3.0)  # in place: never re-zeroed by the API
    assert [c[0] for c in fake.calls] == ["fwd"]
    assert fake.calls[0][1] == _abi.MODE_ATOMIC and fake.calls[0][-1] == 1
    fake.calls.clear()
    # autograd path without gradients: no plan at all; the forward overwrites out (accumulate=0,
    # the library clears it), so the API allocates it without a zero-fill
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long),
                                                   torch.rand(8), (4, 16), mode="atomic")
    assert [c[0] for c in fake.calls] == ["metadata", "fwd"]
    assert fake.calls[1][1] == _abi.MODE_ATOMIC and fake.calls[1][-1] == 0
    # with gradients: the backward builds the plan it reads
    fake.calls.clear()
    xg = [x.requires_grad_(True) for x in _experts(torch.float32)]
    wg = torch.rand(8, requires_grad=True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xg, torch.zeros(8, dtype=torch.long), wg,
                                                   (4, 16), mode="atomic")
    assert [c[0] for c in fake.calls] == ["metadata", "fwd"]
    torch.autograd.grad(out, [wg, *xg], torch.ones(4, 16))
    assert [c[0] for c in fake.calls] == ["metadata", "fwd", "plan", "bwd"]


def test_gate_gradient_keeps_the_weights_shape_and_experts_kept_only_for_it(fake):
    xs = [x.requires_grad_(True) for x in _experts(torch.float32)]
    w = torch.rand(4, 2, requires_grad=True)  # [T, k]-shaped gates
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long), w, (2, 16))
    assert len(out.grad_fn.saved_tensors) == 2  # index and gates, as the reference saves
    assert all(a is b for a, b in zip(out.grad_fn.experts, xs))  # read by the grad_w pass
    (gw,) = torch.autograd.grad(out, [w], torch.ones(2, 16))
    assert gw.shape == w.shape
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long),
                                                   w.detach(), (2, 16))
    assert len(out.grad_fn.saved_tensors) == 2 and out.grad_fn.experts is None


@pytest.mark.parametrize("fixture", ["fake", "fake_small"])
def test_gate_gradient_refuses_experts_modified_in_place(fixture, request):
    """The grad_w pass reads the expert buffers: one modified in place after the forward makes
    the backward raise, as torch does for a modified saved tensor."""
    request.getfixturevalue(fixture)
    xs = [x.requires_grad_(True) for x in _experts(torch.float32)]
    w = torch.rand(8, requires_grad=True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long), w, (4, 16))
    with torch.no_grad():
        xs[2].mul_(2)
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        torch.autograd.grad(out, [w], torch.ones(4, 16))


def test_stale_metadata_is_rebuilt(fake):
    xs = _experts(torch.float32)
    meta = fastmoe_amd.prepare_grouped_metadata(xs, "cuda")
    other = _experts(torch.float32)
    fake.calls.clear()
    fastmoe_amd.grouped_weighted_scatter_add(other, torch.zeros(8, dtype=torch.long), torch.rand(8),
                                             (4, 16), out=torch.zeros(4, 16), metadata=meta)
    # the passed table does not describe `other`: metadata and plan are rebuilt in one call
    assert [c[0] for c in fake.calls] == ["metadata_plan", "fwd"]
    assert fake.calls[0][2] == [3, 0, 5]


def test_metadata_of_the_same_memory_under_another_view_does_not_match(fake):
    wide = torch.randn(3, 32)
    packed = wide.reshape(-1)[:48].view(3, 16)   # same address and rows as wide[:, :16]
    meta = fastmoe_amd.prepare_grouped_metadata([packed], "cuda")
    assert meta.matches([packed])
    strided = wide[:, :16]
    assert strided.data_ptr() == packed.data_ptr() and not meta.matches([strided])
    with pytest.raises(ValueError, match="row-contiguous"):
        fastmoe_amd.grouped_weighted_scatter_add([strided], torch.zeros(3, dtype=torch.long),
                                                 torch.rand(3), (2, 16), out=torch.zeros(2, 16),
                                                 metadata=meta)
    half = torch.randn(3, 16).to(torch.bfloat16)
    meta = fastmoe_amd.prepare_grouped_metadata([half], "cuda")
    as_f16 = half.view(torch.float16)
    assert not meta.matches([as_f16])
    fake.calls.clear()
    fastmoe_amd.grouped_weighted_scatter_add([as_f16], torch.zeros(3, dtype=torch.long),
                                             torch.rand(3), (2, 16),
                                             out=torch.zeros(2, 16, dtype=torch.float16),
                                             metadata=meta)
    assert fake.calls[0][0] == "metadata_plan" and fake.calls[1][5] == _abi.F16


def test_argument_validation(fake):
    xs = _experts(torch.float32)
    with pytest.raises(ValueError, match="total expert rows"):
        fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(7, dtype=torch.long),
                                                 torch.rand(7), (4, 16))
    with pytest.raises(TypeError):
        fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8), torch.rand(8), (4, 16))
    with pytest.raises(ValueError, match="out_shape"):
        fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long),
                                                 torch.rand(8), (4, 15))
    with pytest.raises(ValueError, match="row-contiguous"):
        fastmoe_amd.grouped_weighted_scatter_add([torch.randn(16, 4).t()], torch.zeros(4, dtype=torch.long),
                                                 torch.rand(4), (4, 16))
    with pytest.raises(ValueError, match="unit column stride"):
        fastmoe_amd.grouped_weighted_scatter_add(xs, torch.zeros(8, dtype=torch.long),
                                                 torch.rand(8), (4, 16), out=torch.zeros(16, 4).t())
    with pytest.raises(ValueError, match="empty"):
        fastmoe_amd.prepare_grouped_metadata([], "cuda")


def test_weighted_scatter_add_single_tensor(fake):
    src = torch.randn(10, 4)
    out = fastmoe_amd.weighted_scatter_add(src, torch.randint(0, 5, (10,)), torch.rand(10), (5, 4))
    assert out.shape == (5, 4)
    assert fake.calls[0] == ("metadata_plan", 1, [10], 5, 16, _abi.I64, _abi.F32)


def test_small_path_is_one_launch_per_direction(fake_small):
    xs = [x.requires_grad_(True) for x in _experts()]
    w = torch.rand(8, requires_grad=True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.randint(0, 4, (8,)), w, (4, 16))
    grads = torch.autograd.grad(out, [w, *xs], torch.ones(4, 16, dtype=torch.bfloat16))
    assert [c[0] for c in fake_small.calls] == ["fwd_small", "bwd_small"]
    assert fake_small.calls[0] == ("fwd_small", 3, [3, 0, 5], 4, 16, _abi.I64, _abi.F32,
                                   _abi.BF16, _abi.BF16, 16, 0)
    assert fake_small.calls[1] == ("bwd_small", 3, [3, 0, 5], 4, 16, _abi.BF16, 16, True, True,
                                   _abi.F32)
    assert grads[0].shape == (8,) and [g.shape[0] for g in grads[1:]] == [3, 0, 5]


def test_small_path_backward_of_one_gradient(fake_small):
    xs = _experts()
    w = torch.rand(8, requires_grad=True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, torch.randint(0, 4, (8,)), w, (4, 16))
    torch.autograd.grad(out, [w], torch.ones(4, 16, dtype=torch.bfloat16))
    assert fake_small.calls[1][7:9] == (False, True)


def test_small_path_in_place_accumulates(fake_small):
    fastmoe_amd.grouped_weighted_scatter_add(_experts(torch.float32),
                                             torch.randint(0, 4, (8,), dtype=torch.int32),
                                             torch.rand(8), (4, 16), out=torch.zeros(4, 16))
    assert fake_small.calls == [("fwd_small", 3, [3, 0, 5], 4, 16, _abi.I32, _abi.F32, _abi.F32,
                                 _abi.F32, 16, 1)]


def test_small_path_forward_only(fake_small):
    fastmoe_amd.grouped_weighted_scatter_add(_experts(), torch.randint(0, 4, (8,)), torch.rand(8),
                                             (4, 16))
    assert [c[0] for c in fake_small.calls] == ["fwd_small"]


@pytest.mark.parametrize("case", ["off", "plan_forced", "atomic", "experts", "rows", "scan"])
def test_small_path_not_taken(fake_small, case):
    """The small path stays out of forced plans, atomic modes, more than 256 experts or 4096 rows,
    and (by default) calls whose forward scan T * N exceeds 2^17."""
    sizes, T, opts, mode = (3, 0, 5), 4, {}, None
    if case == "off":
        opts = {"small": 1}
    elif case == "plan_forced":
        opts = {"plan": 3}
    elif case == "atomic":
        mode = "atomic"
    elif case == "experts":
        sizes = (1,) * 257
    elif case == "rows":
        sizes = (4097,)
    else:
        T = 1 << 15  # T * N = 2^18
    xs = [x.requires_grad_(True) for x in _experts(sizes=sizes, D=4)]
    N = sum(sizes)
    with _abi.options(**opts):
        fastmoe_amd.grouped_weighted_scatter_add(xs, torch.randint(0, T, (N,)),
                                                 torch.rand(N, requires_grad=True), (T, 4),
                                                 mode=mode)
    kinds = [c[0] for c in fake_small.calls]
    assert "fwd_small" not in kinds and ("fwd" in kinds)


def test_validating_in_place_call_checks_indices_before_accumulating(fake_small, monkeypatch):
    """With validate=True an in-place call of small-path size takes the planned path, whose index
    check runs before the forward launch (so ``out`` is untouched when it raises); without it,
    the one-launch small path."""
    order = []
    monkeypatch.setattr(ops, "_check_plan_status", lambda plan, T: order.append("check"))
    xs, idx, w = _experts(torch.float32), torch.randint(0, 4, (8,)), torch.rand(8)
    fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16), out=torch.zeros(4, 16),
                                             validate=True)
    kinds = [c[0] for c in fake_small.calls]
    assert kinds == ["metadata_plan", "fwd"] and order == ["check"]
    fake_small.calls.clear()
    fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16), out=torch.zeros(4, 16))
    assert [c[0] for c in fake_small.calls] == ["fwd_small"]


def _capture_on(monkeypatch):
    monkeypatch.setattr(ops, "_capturing", lambda t: True)


@pytest.mark.parametrize("path", ["planned", "small"])
def test_autograd_combine_refused_under_capture(path, monkeypatch):
    """Under HIP graph capture the autograd forward that records a backward, and the backward,
    raise a clear error before any launch; the forward without gradients and the in-place call
    stay capturable."""
    f = _fake_lib(monkeypatch)
    with _abi.options(small=1 if path == "planned" else 0):
        xs = [x.requires_grad_(True) for x in _experts()]
        idx = torch.randint(0, 4, (8,))
        w = torch.rand(8, requires_grad=True)
        _capture_on(monkeypatch)
        with pytest.raises(RuntimeError, match="graph capture is not supported"):
            fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16))
        with pytest.raises(RuntimeError, match="graph capture is not supported"):
            fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16), mode="det")
        assert f.calls == []
        with torch.no_grad():
            fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16))
        fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16), out=torch.zeros(4, 16))
        assert len(f.calls) >= 2
        # forward outside the capture, backward inside it
        monkeypatch.setattr(ops, "_capturing", lambda t: False)
        out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (4, 16))
        _capture_on(monkeypatch)
        n = len(f.calls)
        with pytest.raises(RuntimeError, match="backward under HIP graph capture"):
            torch.autograd.grad(out, [w, *xs], torch.ones(4, 16, dtype=torch.bfloat16))
        assert len(f.calls) == n


def test_autograd_permutation_refused_under_capture(monkeypatch):
    from fastmoe_amd import dispatch

    _capture_on(monkeypatch)
    monkeypatch.setattr(dispatch, "_require_cuda", lambda t, what: None)
    x = torch.randn(4, 8, requires_grad=True)
    with pytest.raises(RuntimeError, match="graph capture is not supported"):
        dispatch.permute_tokens(x, torch.randint(0, 3, (4, 2)), torch.rand(4, 2), 3)


def test_unit_gates_never_release_a_buffer_handed_out(monkeypatch):
    """A captured permutation backward keeps the raw address of its unit gates: every prefix handed
    out stays inside a buffer the module still holds, however many row counts follow."""
    from fastmoe_amd import dispatch

    monkeypatch.setattr(dispatch, "_ONES", {})
    monkeypatch.setattr(dispatch, "_RETIRED", [])
    dev = torch.device("cpu")
    handed = []
    for n in [5, 3000, 7, 100_000, 1, 2047, 250_000, 64, 9000, 1_000_003]:
        g = dispatch._unit_gates(n, dev)
        assert g.shape == (n,) and bool((g == 1).all())
        handed.append((g.data_ptr(), n))
        del g
    held = [dispatch._ONES[dev], *dispatch._RETIRED]
    spans = [(b.data_ptr(), b.data_ptr() + 4 * b.numel()) for b in held]
    for ptr, n in handed:
        assert any(lo <= ptr and ptr + 4 * n <= hi for lo, hi in spans)
    # growth at least doubles: the retired buffers hold fewer elements than the live one
    assert sum(b.numel() for b in dispatch._RETIRED) < dispatch._ONES[dev].numel()


def test_host_helper_validates_and_packs_expert_tables():
    """fastmoe_amd._host.experts: the (address, rows) table of a list of buffers, and the first
    offending buffer named for every kind of bad input."""
    from fastmoe_amd import _host

    base = torch.randn(40, 8)
    xs = [base[0:3], torch.empty(0, 8), base[10:15], torch.randn(1, 8)]
    hidden, rows, max_rows, table, vsum = _host.experts(xs)
    assert vsum == 0 and _host.experts(xs, True)[4] == _host.versions(xs)
    t = memoryview(table).cast("q").tolist()
    assert (hidden, rows, max_rows) == (8, 9, 5)
    assert t[:4] == [xs[0].data_ptr(), 0, xs[2].data_ptr(), xs[3].data_ptr()]
    assert t[4:] == [3, 0, 5, 1]
    cases = [
        ([base[:3], "x"], TypeError, r"expert_tensors\[1\] is not a tensor"),
        ([base[:3], base[:3].double()], ValueError, r"\[1\] differs in device/dtype"),
        ([base[:3], torch.randn(2, 9)], ValueError, r"\[1\] has shape \(2, 9\), expected \[\*, 8\]"),
        ([base[:3], torch.randn(8)], ValueError, r"\[1\] has shape \(8,\)"),
        ([torch.randn(8)], ValueError, r"\[0\] must be 2-D"),
        ([base[:3], base[:, :16].t()[:, :8]], ValueError, r"\[1\] must be row-contiguous"),
        ([base[:3], torch.randn(1, 8).expand(4, 8)], ValueError, r"row-contiguous \(strides \(0, 1\)\)"),
        ([base[:3], torch.randn(4, 8).to_sparse()], ValueError, r"\[1\] must be a dense"),
        ([], ValueError, "empty"),
    ]
    for bad, exc, msg in cases:
        with pytest.raises(exc, match=msg):
            _host.experts(bad)
    # one row with any row stride is row-contiguous (torch's is_contiguous)
    assert _host.experts([base[5:6], base[::5][:1]])[1] == 2


def test_host_helper_version_sum_grows_on_in_place_writes():
    from fastmoe_amd import _host

    xs = [torch.randn(3, 4) for _ in range(5)]
    v0 = _host.versions(xs)
    xs[3].add_(1)
    assert _host.versions(xs) > v0
    with pytest.raises(TypeError):
        _host.versions([xs[0], 3])


def test_host_helper_inference_tensors_raise_instead_of_crashing():
    """Inference tensors have no version counter, and their accessor throws a C++ exception: both
    helpers turn it into a ValueError rather than letting it cross the C API."""
    from fastmoe_amd import _host

    with torch.inference_mode():
        xs = [torch.randn(3, 4) for _ in range(2)]
    assert _host.experts(xs)[1] == 6  # no version counter asked for
    with pytest.raises(ValueError, match="version counter"):
        _host.experts(xs, True)
    with pytest.raises(ValueError, match="version counter"):
        _host.versions(xs)
