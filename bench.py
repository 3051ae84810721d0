"""Benchmark of the grouped MoE combine (forward + backward) on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload gigachat] [--mode det|atomic]

A step is one pass of the hot path over one batch: the public autograd entry point
``grouped_weighted_scatter_add`` (metadata build, plan build, forward kernel) followed by
``torch.autograd.grad`` through it (backward kernel: grad of every expert buffer and of the
gates).  Inputs are synthetic (seeded) and resident in HBM before the timed region.  The timed
region replays that step captured once as a HIP graph (all of its kernels run on every replay;
the host-side Python/autograd cost of E=256 tensors is excluded), as the reference's own kernel
benchmark does with CUDA graphs; the eager, host-inclusive step time is reported beside it
(``eager_ms_per_step``).  The default
workload is BASELINE.json's headline configuration: T=4096 tokens, D=16384, E=256 experts, top-8,
bf16 expert outputs, fp32 gates (the "gigachat" workload of fastmoe_amd.workloads).

Prints ONE JSON line.  ``value`` = algorithmic (compulsory) bytes of forward + backward per step
divided by the measured step time, in GB/s (1e9 B/s).  ``roofline`` reports the dominant kernel
(the one with the longest average launch: the forward or the backward's grad_X pass) from HIP
events recorded around its launches, on the stream it runs on.  ``cpu_baseline`` times the reference's CPU algorithm (oracle/torch_ref.py) on a
bounded sample of the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
# Memory-side float-atomic ceiling of one MI355X, measured with a synthetic kernel that issues the
# atomic forward's adds alone (64 consecutive elements per wave instruction): about 20.7 G 64-byte
# line requests per second, fp32 and packed bf16 alike.
ATOMIC_CEILING_LINES_PER_S = 20.7e9


def _atomic_rate(wl, mode, us, passes_us=None):
    """Request rate of an atomic-mode forward call (its fmoe_combine_fwd span of ``us``), against
    the measured atomic ceiling.  Each element add is one lane of a 64-lane instruction: fp32 adds
    (mode atomic, or any fp32 target) make N*D*4/64 line requests, packed 16-bit pairs N*D*2/64.
    ``passes_us``: the same call's span with every index out of range, i.e. what it spends besides
    the adds (mode atomic with a 16-bit output: the fp32 accumulator's init and store passes over
    T*D; otherwise the zero-fill of the overwritten output; plus a grid of waves that exit at
    once); the rate is then taken over the rest."""
    import torch

    out_bytes = 4 if (mode == "atomic" or wl.dtype == torch.float32) else 2
    lines = wl.N * wl.D * out_bytes / 64
    adds_us = us - passes_us if passes_us else us
    rate = lines / (adds_us * 1e-6)
    res = {"atomic_requests_per_launch": int(lines), "atomic_requests_per_s": round(rate / 1e9, 2),
           "atomic_ceiling_frac": round(rate / ATOMIC_CEILING_LINES_PER_S, 3),
           "note": "G 64-byte line requests/s; ceiling 20.7 G/s measured with a synthetic kernel"}
    if passes_us:
        acc = mode == "atomic" and wl.dtype != torch.float32
        res.update(call_us=round(us, 2), passes_us=round(passes_us, 2),
                   call_requests_per_s=round(lines / (us * 1e-6) / 1e9, 2),
                   passes=("fp32 accumulator init + store" if acc else "zero-fill of the output")
                   + ", timed as the call with every index out of range; the rate above is over "
                     "the call less this")
    return res


def _non_add_passes_us(wl, xs, mode, steps, dev):
    """HIP-event span of the atomic forward call (the autograd path's, which overwrites its
    output) with every scatter index out of range (see _atomic_rate)."""
    import torch

    import fastmoe_amd

    if mode not in ("atomic", "atomic_packed"):
        return None
    bad = torch.full((wl.N,), wl.T, dtype=torch.int64, device=dev)
    w = torch.ones(wl.N, device=dev)

    def step():
        with torch.no_grad():
            fastmoe_amd.grouped_weighted_scatter_add(xs, bad, w, (wl.T, wl.D), mode=mode,
                                                     validate=False)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    kernels, _ = _event_kernels(step, steps)
    return kernels["fwd_atomic"]["avg_us"] if "fwd_atomic" in kernels else None
METRIC = "combine fwd+bwd GB/s & % HBM peak at D=16384,E=256,top-8 bf16; latency ms"


class EventTimer:
    """Brackets each C-ABI launch with HIP events on the current (launch) stream."""

    def __init__(self):
        import torch

        self.torch = torch
        self.records = []
        self.enabled = False

    def span(self, name):
        timer = self

        class _Span:
            def __enter__(self_inner):
                if timer.enabled:
                    self_inner.a = timer.torch.cuda.Event(enable_timing=True)
                    self_inner.a.record()
                return self_inner

            def __exit__(self_inner, *exc):
                if timer.enabled:
                    b = timer.torch.cuda.Event(enable_timing=True)
                    b.record()
                    timer.records.append((name, self_inner.a, b))
                return False

        return _Span()

    def summary(self):
        out = {}
        for name, a, b in self.records:
            out.setdefault(name, []).append(a.elapsed_time(b) * 1e3)  # us
        return {k: {"launches": len(v), "avg_us": statistics.fmean(v),
                    "median_us": statistics.median(v)} for k, v in out.items()}


def _cpu_baseline(wl, sample_tokens: int, reps: int):
    """The reference's CPU combine (cat/mul/index_add_ + index_select/mul/split + gate dot) on a
    T=sample_tokens slice of the workload's routing recipe, all host threads."""
    import torch

    from fastmoe_amd.workloads import algorithmic_bytes, make_experts, make_routing
    from oracle import torch_ref

    torch.set_num_threads(os.cpu_count() or 1)
    idx, w, counts = make_routing(wl, sample_tokens)
    xs = make_experts(counts, wl.D, wl.dtype, "cpu", wl.seed)
    go = torch.randn(sample_tokens, wl.D, generator=torch.Generator().manual_seed(1)).to(wl.dtype)
    N = idx.numel()
    xb = torch.empty(0, dtype=wl.dtype).element_size()
    fwd_b, bwd_b = algorithmic_bytes(sample_tokens, wl.D, N, xb, xb)
    torch_ref.fwd_bwd_step(xs, idx, w, go, sample_tokens)  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        torch_ref.fwd_bwd_step(xs, idx, w, go, sample_tokens)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round((fwd_b + bwd_b) / med / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{wl.name} routing recipe at T={sample_tokens} tokens (N={N} rows), D={wl.D}, "
                   f"E={wl.E}, top-{wl.k}, {str(wl.dtype).replace('torch.', '')}; forward+backward "
                   f"of the reference CPU algorithm (oracle/torch_ref.fwd_bwd_step); median of "
                   f"{reps} after 1 warm-up; {med * 1e3:.1f} ms per step"),
        "ms_per_step": round(med * 1e3, 3),
        "cpu_model": _cpu_model(),
    }


def _time_standard(std_step, steps, warmup, fast_ms, what):
    """Eager event timing of a torch formulation of the same step (the reference's own comparison
    column, run_on_cloud.py:35-53) and its peak memory above the inputs."""
    import torch

    for _ in range(max(1, warmup)):
        std_step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        std_step()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    return {
        "ms_per_step": round(ms, 4),
        "peak_mem_gb": round((torch.cuda.max_memory_allocated() - base) / 2 ** 30, 3),
        "speedup_of_fast": round(ms / fast_ms, 2),
        "what": what,
    }


def _standard_combine_step(wl, xs, idx, w, grad_out, backward):
    """The reference's STANDARD combine in torch GPU ops on the same inputs: cat -> * w ->
    index_add_ into fp32 zeros (run_on_cloud.py:43-48) and, with backward, its autograd
    (index_select, mul, split, gate dot)."""
    import torch

    inputs = [w, *xs]

    def std_step():
        combined = torch.cat(xs, dim=0)
        weighted = combined * w.unsqueeze(-1)
        out = torch.zeros((wl.T, wl.D), device=idx.device)
        out.index_add_(0, idx, weighted)
        if backward:
            torch.autograd.grad(out, inputs, grad_out.float())
        return out

    what = ("torch GPU cat -> * w -> index_add_ into fp32 zeros"
            + (" + autograd backward" if backward else "") + ", eager")
    return std_step, what


def _standard_dispatch_step(wl, x, ids, gates, g_rows, g_sw, backward):
    """The reference's gate_and_sort permutation in torch GPU ops (tiny_model.py:108-138):
    argsort, reverse map, gate permutation, x_flat[rev] gather, bincount; with backward its
    autograd (index_put_ accumulate into x, gate scatter)."""
    import torch

    def std_step():
        flat = ids.view(-1)
        order = torch.argsort(flat)
        rev = torch.arange(wl.T, device=x.device).repeat_interleave(wl.k)[order]
        sw = gates.view(-1)[order]
        permuted = x[rev]
        torch.bincount(flat[order], minlength=wl.E)
        if backward:
            torch.autograd.grad([permuted, sw], [x, gates], [g_rows, g_sw])
        return permuted

    what = ("torch GPU argsort -> reverse map -> x[rev] gather -> bincount"
            + (" + autograd backward" if backward else "") + ", eager")
    return std_step, what


def _standard_moe_step(wl, x, ids, gates):
    """The reference's layer data movement in torch GPU ops, identity experts:
    gate_and_sort's sort + gather (tiny_model.py:108-138) and unpermute's STANDARD combine
    (:399-403, gates in the activation dtype as :100 casts them)."""
    import torch

    def std_step():
        with torch.no_grad():
            flat = ids.view(-1)
            order = torch.argsort(flat)
            rev = torch.arange(wl.T, device=x.device).repeat_interleave(wl.k)[order]
            sw = gates.view(-1)[order].type_as(x)
            permuted = x[rev]
            torch.bincount(flat[order], minlength=wl.E).tolist()
            x_out = permuted * sw.unsqueeze(-1)
            out = torch.zeros(wl.T, wl.D, device=x.device, dtype=x_out.dtype)
            return out.index_add_(0, rev, x_out)

    return std_step, "torch GPU argsort -> x[rev] -> bincount -> * w -> index_add_, eager"


def _verify_combine(wl, xs, idx, w, mode):
    """The reference harness's correctness check (run_on_cloud.py:13-32): the in-place fast path
    into fp32 zeros against cat -> * w -> index_add_ into fp32 zeros, both on the GPU, max |diff|
    against its 1e-4 tolerance."""
    import torch

    import fastmoe_amd

    with torch.no_grad():
        weighted = torch.cat(xs, dim=0) * w.unsqueeze(-1)
        out_std = torch.zeros((wl.T, wl.D), device=idx.device).index_add_(0, idx, weighted)
        del weighted
        out_fast = torch.zeros((wl.T, wl.D), device=idx.device)
        fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (wl.T, wl.D), out=out_fast, mode=mode)
        diff = (out_std - out_fast).abs().max().item()
    return {"max_abs_diff": diff, "tol": 1e-4, "passed": diff <= 1e-4,
            "against": "torch GPU cat -> * w -> index_add_ into fp32 zeros (run_on_cloud.py:13-32)"}


def _verify_dispatch(wl, x, ids, gates):
    """The permutation against the reference's torch sequence (tiny_model.py:108-138) with a
    stable argsort: reverse map, sorted gates and gathered rows must be equal exactly."""
    import torch

    import fastmoe_amd

    with torch.no_grad():
        p = fastmoe_amd.permute_tokens(x, ids, gates, wl.E)
        order = torch.argsort(ids.view(-1), stable=True)
        rev = torch.arange(wl.T, device=x.device).repeat_interleave(wl.k)[order]
        same = (torch.equal(p.reverse_map_indices, rev)
                and torch.equal(p.sorted_weights, gates.view(-1)[order]))
        diff = (p.permuted_data.float() - x[rev].float()).abs().max().item()
    return {"max_abs_diff": diff, "tol": 0.0, "passed": same and diff == 0.0,
            "against": "torch GPU stable argsort -> reverse map -> x[rev] (tiny_model.py:108-138)"}


def _verify_moe(wl, x, ids, gates, out):
    """The layer's combine against an fp32 torch sum of the same permuted products: the output
    is that sum rounded once, so within one ulp of the output dtype (2^-7 relative in bf16)."""
    import torch

    with torch.no_grad():
        order = torch.argsort(ids.view(-1), stable=True)
        rev = torch.arange(wl.T, device=x.device).repeat_interleave(wl.k)[order]
        sw = gates.view(-1)[order].type_as(x)
        ref = torch.zeros(wl.T, wl.D, device=x.device).index_add_(
            0, rev, x[rev].float() * sw.float().unsqueeze(-1))
        err = (out.float().view(wl.T, wl.D) - ref).abs()
        rel = 2.0 ** -7 if out.dtype == torch.bfloat16 else 2.0 ** -10 if out.dtype == torch.float16 else 1e-6
        ok = bool((err <= ref.abs() * rel + 1e-30).all())
        diff = err.max().item()
    return {"max_abs_diff": diff, "tol": f"{rel:g} * |ref| elementwise", "passed": ok,
            "against": "fp32 torch index_add_ of the stably permuted products (tiny_model.py:396-403)"}


class _StepCtx:
    """Stand-in for the autograd context of GroupedWeightedScatterAdd: with it the forward and
    backward functions of the autograd path (fastmoe_amd.ops._combine_forward / _combine_backward)
    issue exactly the launches an autograd step makes -- metadata + plan, forward, grad_X and
    grad_w passes -- without the autograd engine, all from the calling thread."""

    def save_for_backward(self, *tensors):
        self.saved_tensors = tensors


def _timed(fn, n):
    """(device ms per call between two events on the current stream, host wall ms per call)."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(n):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / n, (time.perf_counter() - t0) * 1e3 / n


def _event_kernels(step, steps):
    """Per-kernel durations: HIP events around every C-ABI launch, on the launch stream.  A sleep
    kernel first gives the GPU a backlog so that the host has enqueued each event-kernel-event
    triple before the GPU reaches it (the events then bracket the kernel, not host gaps)."""
    import torch

    from fastmoe_amd import ops

    timer = EventTimer()
    ops._TIMER = timer
    timer.enabled = True
    try:
        torch.cuda._sleep(int(steps * 3e-3 * 2.4e9))
        backlog = True
    except Exception:
        backlog = False
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    timer.enabled = False
    ops._TIMER = None
    return timer.summary(), backlog


def _graph_ms(capture_step, steps, warmup, after=None):
    """Replay time of one step captured as a HIP graph: (ms per replay, wall ms, error or None,
    ``after(captured outputs)`` or None).  ``after`` runs once the timed replays are done, while
    the graph (and so its outputs) is alive."""
    import torch

    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                capture_step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static = capture_step()
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
    except Exception as exc:  # capture unsupported: the caller reports eager numbers only
        return None, None, f"{type(exc).__name__}: {exc}", None
    ms, wall_ms = _timed(graph.replay, steps)
    checked = after(static) if after is not None else None
    del graph, static
    return ms, wall_ms, None, checked


def _replay_matches_eager(static, eager_step, exact_out):
    """Compares the captured step's outputs after its last replay with one eager step through the
    public autograd API: (all compared bits equal, what was compared).  ``exact_out`` False (the
    atomic modes, whose fp32 summation order varies run to run) leaves the output out."""
    import torch

    torch.cuda.synchronize()
    eager = eager_step()
    torch.cuda.synchronize()
    first = 0 if exact_out else 1
    pairs = list(zip(static, eager))[first:]
    same = len(static) == len(eager) and all(
        a.shape == b.shape and a.dtype == b.dtype
        and torch.equal(a.reshape(-1).view(torch.uint8), b.reshape(-1).view(torch.uint8))
        for a, b in pairs)
    what = ["out"] if exact_out else []
    if len(static) > 1:
        what += ["grad_w", "every expert's grad_X"]
    return same, "bits of " + ", ".join(what)


def _autograd_floor_ms(wl, xs, idx, w, grad_out, steps):
    """Host time per step of torch's autograd machinery alone for this call shape: a Function
    that takes the same arguments (indices, weights, out_shape, *expert_tensors), does no work and
    returns gradients of the same shapes, then torch.autograd.grad over [w, *xs] as the eager step
    does.  Everything the eager step costs above this is the library's own host work."""
    import torch

    N = sum(x.shape[0] for x in xs)
    sizes = [x.shape[0] for x in xs]
    gx_all = torch.empty(N, wl.D, dtype=wl.dtype, device=w.device)
    gw = torch.empty_like(w)

    class _NoOp(torch.autograd.Function):
        @staticmethod
        def forward(ctx, indices, weights, out_shape, *expert_tensors):
            ctx.save_for_backward(indices, weights, *expert_tensors)
            return torch.empty(out_shape, dtype=expert_tensors[0].dtype,
                               device=expert_tensors[0].device)

        @staticmethod
        def backward(ctx, g):
            return (None, gw, None, *torch.split(gx_all, sizes))

    inputs = [w, *xs]

    def step():
        out = _NoOp.apply(idx, w, (wl.T, wl.D), *xs)
        torch.autograd.grad(out, inputs, grad_out)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def _combine_inputs(wl, dev, backward, inplace=False):
    import torch

    from fastmoe_amd.workloads import make_experts, make_routing

    idx, w, counts = make_routing(wl)
    idx, w = idx.to(dev), w.to(dev)
    xs = make_experts(counts, wl.D, wl.dtype, dev, wl.seed)
    if backward:
        xs = [x.requires_grad_(True) for x in xs]
        w.requires_grad_(True)
    gen_dev = torch.Generator(device=dev)
    grad_out = torch.randn(wl.T, wl.D, device=dev, dtype=torch.float32,
                           generator=gen_dev.manual_seed(1)).to(wl.dtype)
    return idx, w, xs, grad_out


def _combine_steps(wl, xs, idx, w, grad_out, mode, backward, inplace, dev):
    """(public autograd / in-place step, graph-capturable step with the same launches)."""
    import torch

    import fastmoe_amd
    from fastmoe_amd import ops

    inputs = [w, *xs]
    if inplace:
        out_static = torch.zeros((wl.T, wl.D), device=dev)
        meta = fastmoe_amd.prepare_grouped_metadata(xs, dev)

        def step():
            out_static.zero_()
            return fastmoe_amd.grouped_weighted_scatter_add(
                xs, idx, w, (wl.T, wl.D), out=out_static, metadata=meta, mode=mode)
        return step, step

    def step():
        out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (wl.T, wl.D), mode=mode)
        if backward:
            return (out, *torch.autograd.grad(out, inputs, grad_out))
        return (out,)

    def direct_step():
        with torch.no_grad():
            ctx = _StepCtx()
            out = ops._combine_forward(ctx, mode, None, idx, w, (wl.T, wl.D), xs, backward)
            if backward:
                gw, gx = ops._combine_backward(ctx, grad_out, True, [True] * len(xs))
                return (out, gw, *gx)
        return (out,)
    return step, direct_step


def _summarize_kernels(kernels, kbytes):
    """Attach algorithmic bytes, GB/s and fraction of peak to the event-timed kernels; return the
    dominant (longest) one's name."""
    for name, k in kernels.items():
        if name in kbytes:
            k["algorithmic_bytes"] = kbytes[name]
            k["GBs"] = kbytes[name] / (k["avg_us"] * 1e-6) / 1e9
            k["frac"] = k["GBs"] / HBM_PEAK_GBS
    return max((n for n in kernels if n in kbytes), key=lambda n: kernels[n]["avg_us"])


def _config_line(name, mode, steps, warmup, dev):
    """One BASELINE configuration measured in this run: graph-replayed step, % of peak, the
    metadata + plan span and the dominant kernel (HIP events)."""
    import torch

    from fastmoe_amd.workloads import WORKLOADS, algorithmic_bytes, kernel_bytes

    wl = WORKLOADS[name]
    backward = wl.backward
    idx, w, xs, grad_out = _combine_inputs(wl, dev, backward)
    xb = torch.empty(0, dtype=wl.dtype).element_size()
    fwd_b, bwd_b = algorithmic_bytes(wl.T, wl.D, wl.N, xb, xb)
    step_bytes = fwd_b + (bwd_b if backward else 0)
    step, direct_step = _combine_steps(wl, xs, idx, w, grad_out, mode, backward, False, dev)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    kernels, _ = _event_kernels(step, steps)
    dom = _summarize_kernels(kernels, kernel_bytes(wl.T, wl.D, wl.N, xb, xb))
    ms, _, err, _ = _graph_ms(direct_step, steps, warmup)
    if ms is None:
        ms, _ = _timed(step, steps)
    plan_us = sum(v["avg_us"] for k, v in kernels.items() if k in ("metadata_plan", "plan", "metadata"))
    gbs = step_bytes / (ms * 1e-3) / 1e9
    repeat = None
    if name == "detatomic":
        # BASELINE's det-vs-atomic configuration: 10 runs on the same inputs; det must repeat bit
        # for bit, atomic is reported with its largest run-to-run difference
        with torch.no_grad():
            ref = step()[0].clone()
            same, worst = True, 0.0
            for _ in range(9):
                o = step()[0]
                same = same and torch.equal(o.view(torch.int16), ref.view(torch.int16))
                worst = max(worst, (o.float() - ref.float()).abs().max().item())
        repeat = {"runs": 10, "bit_identical": same, "max_abs_diff": worst}
    res = {
        "workload": name, "mode": mode, "backward": backward,
        "ms_per_step": round(ms, 4), "GBs": round(gbs, 1),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "timing": "hip-graph replay" if err is None else f"eager ({err})",
        "metadata_plan_us": round(plan_us, 2),
        "dominant_kernel": dom, "dominant_avg_us": round(kernels[dom]["avg_us"], 2),
        "dominant_frac": round(kernels[dom]["frac"], 4),
    }
    if repeat is not None:
        res["repeatability"] = repeat
    if mode != "det" and "fwd_atomic" in kernels:
        res["atomic"] = _atomic_rate(wl, mode, kernels["fwd_atomic"]["avg_us"],
                                     _non_add_passes_us(wl, xs, mode, steps, dev))
    del idx, w, xs, grad_out, step, direct_step
    torch.cuda.empty_cache()
    return res


# The other BASELINE configurations, measured in every default run beside the headline.
CONFIG_LINES = [("mid", "det"), ("mid", "atomic"), ("skewed", "det"), ("skewed", "atomic"),
                ("detatomic", "det"), ("detatomic", "atomic"), ("plumbing", "det")]


# --plan-sweep shapes: (tokens, rows, rows sent to one hot token).  Uniform random scatter
# indices over 256 experts of random sizes; the slot-map plan is timed where the rows are a top-k
# routing (rows = k * tokens, no hot token).
PLAN_SWEEP_CASES = [(4096, 32768, 0), (8192, 49152, 0), (32768, 65536, 0), (16384, 131072, 0),
                    (1, 131072, 0), (100, 131072, 65536), (32768, 262144, 0),
                    (32768, 262144, 65536), (65536, 1048576, 0), (1048576, 2097152, 0),
                    (131071, 4194304, 0)]
PLAN_PATHS = {"one_launch": 3, "ranged": 4, "bucketed": 2, "radix": 1, "automatic": 0}


def _plan_sweep(dev, reps=15):
    """Median HIP-event span (µs) of the metadata + plan call for every plan path forced in turn
    (a forced path whose limits do not hold falls back to the automatic choice, and is reported
    as null), plus the slot-map plan of a top-k routing.  The launches are queued behind a sleep
    kernel so that the events bracket the kernels."""
    import statistics

    import torch

    from fastmoe_amd import _abi, ops

    lib = _abi.lib()

    def span(fn):
        ts = []
        for r in range(reps + 3):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(2_000_000)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            if r >= 3:
                ts.append(a.elapsed_time(b) * 1e3)
        return round(statistics.median(ts), 1)

    rows = []
    for T, N, hot in PLAN_SWEEP_CASES:
        gen = torch.Generator().manual_seed(T + N)
        idx = torch.randint(0, T, (N,), generator=gen)
        if hot:
            idx[torch.randperm(N, generator=gen)[:hot]] = 7
        E = 256
        cuts = torch.sort(torch.randint(0, N + 1, (E - 1,), generator=gen)).values.tolist()
        sizes = [b - a for a, b in zip([0] + cuts, cuts + [N])]
        xd = [torch.empty(n, 8, device=dev) for n in sizes]
        idd, wd = idx.to(dev), torch.rand(N, generator=gen).to(dev)
        row = {"tokens": T, "rows": N, "hot_token_rows": hot, "us": {}}
        for name, code in PLAN_PATHS.items():
            with _abi.options(plan=code):
                if code and lib.fmoe_plan_path(N, T, E) != code:  # limits do not hold
                    row["us"][name] = None
                    continue
                row["us"][name] = span(lambda: ops.prepare_metadata_and_plan(xd, idd, wd, T))
        with _abi.options(plan=0):
            row["automatic_path"] = {v: k for k, v in PLAN_PATHS.items()}[lib.fmoe_plan_path(N, T, E)]
        k = N // T
        if not hot and k * T == N and k <= 64:
            # a top-k routing of the same size: token t's rows are the slots t*k .. t*k+k-1,
            # placed at random packed rows
            slot_pos = torch.randperm(N, generator=gen).to(torch.int32).to(dev)
            row["us"]["slot_map"] = span(
                lambda: ops.prepare_metadata_and_plan_from_slots(xd, slot_pos, wd, T, k))
        rows.append(row)
    return {"what": "metadata + plan span per plan path (median of %d, HIP events, µs)" % reps,
            "experts": 256, "cases": rows}


def _plan_floor(wl, dev, reps=50, rounds=3):
    """Graph-replayed forward of ``wl`` (µs per replay, min over rounds): the forward alone with
    its plan prebuilt, an empty kernel then the forward, each metadata + plan builder then the
    forward, and the plan launches alone.  The experts come from the dispatch permutation of the
    workload's top-k routing, so the slot-map plan applies; the forward's output is checked
    equal from both plans first."""
    import torch

    import fastmoe_amd
    from fastmoe_amd import _abi, ops
    from fastmoe_amd.workloads import make_topk

    T, D, E, k = wl.T, wl.D, wl.E, wl.k
    ids, gates = make_topk(wl)
    x = torch.randn(T, D, device=dev).to(wl.dtype)
    with torch.no_grad():
        p = fastmoe_amd.permute_tokens(x, ids.to(dev), gates.to(dev), E)
    counts = p.expert_counts.tolist()
    xs = [t.contiguous() for t in p.permuted_data.split(counts)]
    idd, wd, sp = p.reverse_map_indices, p.sorted_weights.float(), p.slot_pos
    meta, plan = ops.prepare_metadata_and_plan(xs, idd, wd, T)
    meta2, plan2 = ops.prepare_metadata_and_plan_from_slots(xs, sp, wd, T, k)
    out = torch.empty(T, D, dtype=wl.dtype, device=dev)
    out2 = torch.empty_like(out)
    ops._launch_fwd(meta, _abi.MODE_DET, plan, None, None, out, accumulate=False)
    ops._launch_fwd(meta2, _abi.MODE_DET, plan2, None, None, out2, accumulate=False)
    torch.cuda.synchronize()
    same = torch.equal(out.view(torch.int16), out2.view(torch.int16))
    tiny = torch.zeros(1, device=dev)

    def fwd():
        ops._launch_fwd(meta, _abi.MODE_DET, plan, None, None, out, accumulate=False)

    def idx_plan():
        return ops.prepare_metadata_and_plan(xs, idd, wd, T)

    def slot_plan():
        return ops.prepare_metadata_and_plan_from_slots(xs, sp, wd, T, k)

    def then_fwd(build):
        def step():
            m, pl = build()
            ops._launch_fwd(m, _abi.MODE_DET, pl, None, None, out, accumulate=False)
        return step

    steps = {
        "forward alone (plan prebuilt)": fwd,
        "empty kernel, then the forward": lambda: (tiny.add_(1.0), fwd()),
        "slot-map metadata + plan, then the forward": then_fwd(slot_plan),
        "scatter-index metadata + plan, then the forward": then_fwd(idx_plan),
        "slot-map metadata + plan alone": slot_plan,
        "scatter-index metadata + plan alone": idx_plan,
        "empty kernel alone": lambda: tiny.add_(1.0),
    }
    graphs = {}
    for name, fn in steps.items():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        graphs[name] = g
    res = {name: [] for name in graphs}
    for _ in range(rounds):  # the graphs alternate within each round
        for name, g in graphs.items():
            for _ in range(5):
                g.replay()
            torch.cuda._sleep(5_000_000)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                g.replay()
            b.record()
            torch.cuda.synchronize()
            res[name].append(a.elapsed_time(b) * 1e3 / reps)
    from fastmoe_amd.workloads import algorithmic_bytes

    fwd_b, _ = algorithmic_bytes(T, D, wl.N, x.element_size(), x.element_size())
    return {"workload": wl.name, "outputs_equal_from_both_plans": same,
            "bar_us_at_70pct": round(fwd_b / (0.7 * HBM_PEAK_GBS * 1e3), 1),
            "us_per_replay_min": {n: round(min(v), 1) for n, v in res.items()},
            "us_per_replay_all": {n: [round(x, 1) for x in v] for n, v in res.items()}}


def _cpu_model() -> str:
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="gigachat")
    ap.add_argument("--mode", default="det", choices=["det", "atomic", "atomic_packed"])
    ap.add_argument("--path", default="combine", choices=["combine", "dispatch", "moe"],
                    help="combine: the grouped combine (the headline); dispatch: the permutation "
                         "that feeds it (gate_and_sort's sort + gather) and its backward; moe: "
                         "the MoE layer's data movement, permutation then combine with identity "
                         "experts (forward; the combine's plan comes from the permutation)")
    ap.add_argument("--inplace", action="store_true",
                    help="the reference's kernel benchmark (run_on_cloud.py:56-96): fp32 out, "
                         "metadata prepared once, each step out.zero_() + the in-place call "
                         "(forward only)")
    ap.add_argument("--fwd-only", action="store_true",
                    help="time the forward alone (the default for forward-only workloads)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager steps instead of graph replays")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="K",
                    help="also run K plain 1 GiB device copies (a reference kernel of known bytes "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--cpu-sample-tokens", type=int, default=0,
                    help="tokens of the CPU baseline sample (0 = the whole workload)")
    ap.add_argument("--cpu-reps", type=int, default=8)
    ap.add_argument("--no-slot-plan", action="store_true",
                    help="moe path: build the combine's plan from the scatter index instead of "
                         "the permutation's slot map")
    ap.add_argument("--no-standard", action="store_true",
                    help="skip the torch STANDARD combine timed on the same GPU")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other BASELINE configurations (the 'configs' object)")
    ap.add_argument("--config-steps", type=int, default=10)
    ap.add_argument("--plan-sweep", action="store_true",
                    help="instead of a step: time every builder of the plan (the token-major "
                         "inverse of the scatter index) on a set of shapes, HIP events")
    ap.add_argument("--plan-floor", action="store_true",
                    help="instead of a step: graph-replayed forward of --workload alone, behind "
                         "an empty kernel, behind each plan builder, and each of those alone")
    args = ap.parse_args()

    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the combine is rank-local "
                                   "(each rank combines its own tokens after the expert-parallel "
                                   "all-to-all); run with --gpus 1",
                          "n_gpus": args.gpus}))
        return 2

    import torch

    import fastmoe_amd
    from fastmoe_amd.workloads import (WORKLOADS, algorithmic_bytes, dispatch_bytes,
                                       kernel_bytes, make_topk)

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.plan_sweep:
        print(json.dumps(_plan_sweep(dev)), flush=True)
        return 0
    if args.plan_floor:
        print(json.dumps(_plan_floor(WORKLOADS[args.workload], dev)), flush=True)
        return 0
    wl = WORKLOADS[args.workload]
    backward = wl.backward and not args.fwd_only and not args.inplace
    gen_dev = torch.Generator(device=dev)
    xb = torch.empty(0, dtype=wl.dtype).element_size()
    direct_step = None
    if args.path == "combine":
        metric = METRIC
        idx, w, xs, grad_out = _combine_inputs(wl, dev, backward)
        fwd_b, bwd_b = algorithmic_bytes(wl.T, wl.D, wl.N, xb, 4 if args.inplace else xb)
        step, direct_step = _combine_steps(wl, xs, idx, w, grad_out, args.mode, backward,
                                           args.inplace, dev)

        std = lambda: _standard_combine_step(wl, xs, idx, w, grad_out, backward)  # noqa: E731
        verify = lambda: _verify_combine(wl, xs, idx, w, args.mode)  # noqa: E731
    elif args.path == "moe":
        metric = ("MoE layer data movement GB/s & % HBM peak (permutation + grouped combine, "
                  "identity experts, forward)")
        backward = False
        ids, gates = make_topk(wl)
        ids, gates = ids.to(dev), gates.to(dev)
        x = torch.randn(wl.T, wl.D, device=dev, dtype=torch.float32,
                        generator=gen_dev.manual_seed(3)).to(wl.dtype)
        gates = gates.type_as(x)  # the layer's gates are in the activation dtype (tiny_model.py:100)
        pf, _ = dispatch_bytes(wl.T, wl.D, wl.N, xb)
        cf, _ = algorithmic_bytes(wl.T, wl.D, wl.N, xb, xb)
        fwd_b, bwd_b = pf + cf, 0
        use_slots = not args.no_slot_plan
        # rows per expert on the host once (the routing is the same every step), so the step has
        # no device->host synchronisation and can be captured in a graph
        with torch.no_grad():
            counts_host = fastmoe_amd.permute_tokens(x, ids, gates, wl.E).expert_counts.tolist()

        def step():
            with torch.no_grad():
                p = fastmoe_amd.permute_tokens(x, ids, gates, wl.E)
                parts = p.permuted_data.split(counts_host)
                return fastmoe_amd.unpermute(parts, p.reverse_map_indices, p.sorted_weights,
                                             (1, wl.T), permutation=p if use_slots else None)

        std = lambda: _standard_moe_step(wl, x, ids, gates)  # noqa: E731
        verify = lambda: _verify_moe(wl, x, ids, gates, step())  # noqa: E731
    else:
        metric = ("dispatch permutation fwd+bwd GB/s & % HBM peak (gate_and_sort sort + gather, "
                  "its backward)")
        ids, gates = make_topk(wl)
        ids, gates = ids.to(dev), gates.to(dev)
        x = torch.randn(wl.T, wl.D, device=dev, dtype=torch.float32,
                        generator=gen_dev.manual_seed(3)).to(wl.dtype)
        g_rows = torch.randn(wl.N, wl.D, device=dev, dtype=torch.float32,
                             generator=gen_dev.manual_seed(4)).to(wl.dtype)
        g_sw = torch.randn(wl.N, device=dev, generator=gen_dev.manual_seed(5))
        if backward:
            x.requires_grad_(True)
            gates.requires_grad_(True)
        fwd_b, bwd_b = dispatch_bytes(wl.T, wl.D, wl.N, xb)

        def step():
            p = fastmoe_amd.permute_tokens(x, ids, gates, wl.E)
            if backward:
                torch.autograd.grad([p.permuted_data, p.sorted_weights], [x, gates],
                                    [g_rows, g_sw])
            return p.permuted_data

        std = lambda: _standard_dispatch_step(wl, x, ids, gates, g_rows, g_sw,  # noqa: E731
                                              backward)
        verify = lambda: _verify_dispatch(wl, x, ids, gates)  # noqa: E731
    step_bytes = fwd_b + (bwd_b if backward else 0)

    if args.copy_probe:
        a = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(args.copy_probe):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    torch.cuda.reset_peak_memory_stats(dev)
    base_mem = torch.cuda.memory_allocated(dev)
    step()
    torch.cuda.synchronize()
    fast_peak = torch.cuda.max_memory_allocated(dev) - base_mem

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Eager steps through the public API (host-inclusive: Python + autograd over E expert tensors
    # is part of this number).
    # Eager steps and, for the combine's autograd step, torch's autograd floor for the same call,
    # alternated three times (the host's load varies): the best of each.
    eager = []
    floors = []
    for _ in range(3):
        eager.append(_timed(step, args.steps))
        if args.path == "combine" and backward:
            floors.append(_autograd_floor_ms(wl, xs, idx, w, grad_out, args.steps))
    eager_ms, eager_wall_ms = min(eager)
    floor_ms = min(floors) if floors else None
    kernels, backlog = _event_kernels(step, args.steps)

    graph_error = None
    replay_check = None
    ms = None
    if not args.eager:
        # The step captured once as a HIP graph and replayed: the timed region is pure device
        # work, the convention of the reference's own kernel benchmark (run_on_cloud.py:66-92).
        # The combine's step is captured from the launches the autograd path makes, issued by its
        # own forward and backward functions on this thread (_StepCtx), without the autograd
        # engine.
        after = None
        if direct_step is not None and not args.inplace:
            after = lambda static: _replay_matches_eager(static, step,  # noqa: E731
                                                         args.mode == "det")
        ms, wall_ms, graph_error, replay_check = _graph_ms(direct_step or step, args.steps,
                                                           args.warmup, after)
    if ms is not None:
        timing = "hip-graph replay of one captured step"
    else:
        ms, wall_ms = eager_ms, eager_wall_ms
        timing = "eager steps"
    wall = wall_ms * args.steps / 1e3

    # Dominant kernel: the single-kernel span with the longest average launch.
    kbytes = kernel_bytes(wl.T, wl.D, wl.N, xb, 4 if args.inplace else xb)
    dom_name = _summarize_kernels(kernels, kbytes)
    dom_bytes = kbytes[dom_name]
    dom_us = kernels[dom_name]["avg_us"]
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    traffic, traffic_info = None, None
    tfile = ROOT / "profiles" / f"traffic_{wl.name}_{dom_name}.json"
    if tfile.exists():
        from fastmoe_amd.build import source_hash

        tj = json.loads(tfile.read_text())
        traffic = tj.get("hbm_bytes_per_launch")
        traffic_info = {"file": str(tfile.relative_to(ROOT)), "commit": tj.get("commit"),
                        "sources_sha256": tj.get("sources_sha256"),
                        "matches_current_sources": tj.get("sources_sha256") == source_hash()}

    value = step_bytes / (ms * 1e-3) / 1e9
    res = {
        "metric": metric,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": str(wl.dtype).replace("torch.", "").replace("bfloat16", "bf16"),
        "data": "synthetic (seeded top-k routing of N(0,1) logits; N(0,1) expert outputs, one "
                "allocation per expert; fp32 softmax gates; N(0,1) grad_out)",
        "config": {
            "workload": wl.name, "path": args.path, "tokens": wl.T, "hidden": wl.D,
            "experts": wl.E, "top_k": wl.k, "rows": wl.N, "mode": args.mode, "backward": backward,
            "inplace": args.inplace,
            "fwd_bytes": fwd_b, "bwd_bytes": bwd_b if backward else 0,
        },
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "latency_ms": round(ms, 4),
        "tokens_per_s": round(wl.T / (ms * 1e-3), 1),
        "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
        "timing": timing,
        "eager_ms_per_step": round(eager_ms, 4),
        "eager_value": round(step_bytes / (eager_ms * 1e-3) / 1e9, 2),
        "eager_wall_ms_per_step": round(eager_wall_ms, 4),
        "eager_autograd_floor_ms": round(floor_ms, 4) if floor_ms is not None else None,
        "graph_error": graph_error,
        "graph_replay_matches_eager": replay_check[0] if replay_check else None,
        "graph_replay_compared": replay_check[1] if replay_check else None,
        "kernel_timing": "HIP events around each launch in eager steps queued behind a sleep kernel"
                         if backlog else "HIP events around each launch in eager steps",
        "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kernels.items()},
        "roofline": {
            "kernel": dom_name,
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_measured_on": traffic_info,
            "algorithmic_bytes": dom_bytes,
            "avg_launch_us": round(dom_us, 3),
        },
        "cpu_baseline": None,
    }
    if args.path == "combine" and args.mode != "det" and "fwd_atomic" in kernels:
        res["atomic"] = _atomic_rate(wl, args.mode, kernels["fwd_atomic"]["avg_us"],
                                     None if args.inplace else
                                     _non_add_passes_us(wl, xs, args.mode, args.steps, dev))
    if not args.no_standard:
        res["verify"] = verify()
        std_step, what = std()
        res["standard"] = _time_standard(std_step, args.steps, args.warmup, ms, what)
        res["peak_mem_gb"] = round(fast_peak / 2 ** 30, 3)
    if not args.no_cpu_baseline and args.path == "combine":
        res["cpu_baseline"] = _cpu_baseline(wl, args.cpu_sample_tokens or wl.T, args.cpu_reps)
    if (args.path == "combine" and not args.no_configs and not args.inplace
            and args.workload == "gigachat"):
        # the other BASELINE configurations, timed in this run (no CPU baseline)
        torch.cuda.empty_cache()
        res["configs"] = [_config_line(n, m, args.config_steps, 3, dev) for n, m in CONFIG_LINES]
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
