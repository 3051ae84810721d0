"""Seeded random campaigns on the GPU, broader than the per-feature random tests.

Each test draws a fixed number of cases from a seeded generator with log-uniform sizes (most
cases small, some up to tens of thousands of rows or tokens) and checks every case against the
C oracle with the bars of tests/test_parity_gpu.py:
  * autograd forward + backward over uniform, top-k and Zipf-skewed routing, up to 600 experts
    (beyond the 256 that one launch of metadata + plan takes), every plan path and both backward
    forms: forward bits, grad_X bits, grad_w within 1e-6 of sum|grad_out * X|;
  * the dispatch permutation (fwd + bwd) up to 4096 experts, and in-place calls into fp32 / bf16 /
    f16 outputs with prior contents and padded rows (det bit-exact, atomic within the two-order
    reordering bound);
  * the bare inverse of the scatter index, the combine planned from the permutation's slot map
    (fwd + bwd), and graph-captured in-place calls replayed three times.
Every assertion message names the case and its configuration.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import fastmoe_amd
from fastmoe_amd import ops
from oracle import cref
from tests.helpers import (abs_dot, abs_sum, bits, oracle_bwd, oracle_fwd, packed_tol,
                           reorder_tol, to_np, within_one_ulp16)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DTS = [torch.float32, torch.bfloat16, torch.float16]
# Wider runs of the same campaigns (off the suite, on a GPU box): FMOE_CAMPAIGN_SEED shifts every
# campaign's seed, FMOE_CAMPAIGN_SCALE multiplies its case count.
SEED_SHIFT = int(os.environ.get("FMOE_CAMPAIGN_SEED", "0"))
SCALE = max(1, int(os.environ.get("FMOE_CAMPAIGN_SCALE", "1")))


def _logu(rng, hi: int) -> int:
    """Log-uniform integer in [1, hi]."""
    return max(1, int(np.exp(rng.uniform(0, np.log(max(hi, 1))))))


def _split(rng, N: int, E: int):
    cuts = np.sort(rng.integers(0, N + 1, E - 1))
    return np.diff(np.concatenate([[0], cuts, [N]])).tolist()


def _expect_bits(got: torch.Tensor, want: np.ndarray, label: str) -> None:
    np.testing.assert_array_equal(bits(got), want.view(np.uint32) if want.dtype == np.float32
                                  else want, err_msg=label)


def test_campaign_autograd(kernel_options):
    rng = np.random.default_rng(1101 + SEED_SHIFT)
    for case in range(120 * SCALE):
        T = _logu(rng, 20000)
        D = int(rng.choice([1, 3, 8, 16, 64, 100, 512, 1024, 2048, 4104]))
        cap = max(1, min(65536, (1 << 21) // D, max(64 * T, 5000)))
        routing = ["uniform", "topk", "skew"][int(rng.integers(3))]
        if routing == "topk":
            k = int(rng.integers(1, 9))
            T = max(1, min(T, cap // k))
            E = int(rng.integers(k, 300))
            ids = np.argpartition(rng.random((T, E)), k - 1, axis=1)[:, :k].reshape(-1)
            idx = (np.arange(T * k) // k)[np.argsort(ids, kind="stable")]
            sizes = np.bincount(ids, minlength=E).tolist()
        else:
            N = _logu(rng, cap)
            E = int(rng.integers(1, 600))
            if routing == "uniform":
                idx = rng.integers(0, T, N)
            else:
                p = 1.0 / np.arange(1, T + 1) ** 1.1
                idx = rng.choice(T, N, p=p / p.sum())
            sizes = _split(rng, N, E)
        if rng.random() < 0.25:
            idx = idx.copy()
            idx[:: int(rng.integers(3, 40))] = T + int(rng.integers(0, 5))
        N = len(idx)
        xdt = DTS[int(rng.integers(3))]
        wdt = [torch.float32, torch.bfloat16][int(rng.integers(2))]
        idt = [torch.int64, torch.int32][int(rng.integers(2))]
        r, fused = rng.random(), bool(rng.random() < 0.25)
        # radix / bucketed / one launch / ranged / automatic (a forced path whose limits do not
        # hold falls back to the automatic choice)
        plan = 1 if r < 0.2 else (2 if r < 0.3 else (3 if r < 0.45 else (4 if r < 0.65 else 0)))
        # with the automatic plan, half the cases force the one-launch small path where its
        # limits (4096 rows, 256 experts) allow it; the others take the default choice
        small = 2 if plan == 0 and rng.random() < 0.5 else 0
        # forward mode: det mostly; the atomic modes in some cases (atomic_packed needs whole
        # 16-byte vectors of a 16-bit output)
        m = rng.random()
        mode = "atomic" if m < 0.15 else ("atomic_packed" if m < 0.25 else "det")
        if mode == "atomic_packed" and xdt != torch.float32 and D % 8:
            mode = "atomic"
        order = int(rng.integers(1, 3))  # the atomic grid's order
        kernel_options(plan=plan, bwd_fused=1 if fused else 0, small=small,
                       fwd_atomic_order=order)
        label = (f"autograd case {case}: T={T} N={N} E={E} D={D} {routing} {xdt} {wdt} {idt} "
                 f"plan={plan} fused={fused} small={small} mode={mode} order={order}")
        gen = torch.Generator().manual_seed((1101 + SEED_SHIFT) * 1000 + case)
        idx_t = torch.from_numpy(np.asarray(idx, dtype=np.int64)).to(idt)
        w = torch.rand(N, generator=gen).to(wdt)
        experts = [torch.randn(n, D, generator=gen).to(xdt) for n in sizes]
        xs = [x.to(DEV).requires_grad_(True) for x in experts]
        wd = w.to(DEV).requires_grad_(True)
        out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx_t.to(DEV), wd, (T, D), mode=mode)
        go = torch.randn(T, D, generator=gen).to(xdt)
        grads = torch.autograd.grad(out, [wd, *xs], go.to(DEV))
        want, acc, _ = oracle_fwd(experts, idx_t, w, T, xdt)
        if mode == "det":
            _expect_bits(out, want, label)
        else:
            i64 = idx_t.to(torch.int64).numpy()
            valid = (i64 >= 0) & (i64 < T)
            k = max(2, int(np.bincount(i64[valid], minlength=T).max()) if valid.any() else 2)
            fscale = abs_sum(experts, idx_t, w, T)
            got = out.detach().float().cpu().numpy()
            if xdt == torch.float32:
                assert np.all(np.abs(got - acc) <= reorder_tol(k, fscale)), label
            else:
                want16 = torch.from_numpy(want.view(np.int16)).view(xdt).float().numpy()
                if mode == "atomic":
                    assert np.all(within_one_ulp16(got, want16, xdt, k, fscale)), label
                else:
                    assert np.all(np.abs(got - want16) <= packed_tol(k, fscale, xdt)), label
        want_gx, want_gw = oracle_bwd(experts, idx_t, w, T, go)
        got_gx = np.concatenate([to_np(g).reshape(-1, D) for g in grads[1:]])
        np.testing.assert_array_equal(got_gx.view(want_gx.dtype), want_gx, err_msg=label)
        scale = abs_dot(experts, idx_t, go, T)
        err = np.abs(grads[0].double().cpu().numpy() - want_gw)
        rtol = 1e-6 if wdt == torch.float32 else 2.0 ** -8  # grad_w stored in the gates' dtype
        assert np.all(err <= 1e-6 * scale + rtol * np.abs(want_gw) + 1e-30), label


def test_campaign_permutation_and_inplace(kernel_options):
    rng = np.random.default_rng(2202 + SEED_SHIFT)
    for case in range(160 * SCALE):
        gen = torch.Generator().manual_seed((2202 + SEED_SHIFT) * 1000 + case)
        if case % 2:
            T, k = _logu(rng, 10000), int(rng.integers(1, 9))
            E = int(rng.choice([1, 2, 7, 64, 256, 1000, 1025, 3000, 4096]))
            D = int(rng.choice([1, 2, 7, 16, 100, 1024, 2048]))
            T = max(1, min(T, (1 << 21) // (k * D)))
            ids = torch.from_numpy(rng.integers(0, E, (T, k)))
            if rng.random() < 0.3:
                ids[torch.from_numpy(rng.random((T, k)) < 0.05)] = int(rng.choice([-1, E, E + 7]))
            if rng.random() < 0.5:
                ids = ids.to(torch.int32)
            xdt = DTS[int(rng.integers(3))]
            wdt = [torch.float32, torch.bfloat16][int(rng.integers(2))]
            label = f"permute case {case}: T={T} k={k} E={E} D={D} {xdt} {wdt} {ids.dtype}"
            w = torch.rand(T, k, generator=gen).to(wdt)
            x = torch.randn(T, D, generator=gen).to(xdt)
            xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
            p = fastmoe_amd.permute_tokens(xd, ids.to(DEV), wd, E)
            g_rows = torch.randn(T * k, D, generator=gen).to(xdt)
            g_sw = torch.randn(T * k, generator=gen).to(wdt)
            gx, gw = torch.autograd.grad([p.permuted_data, p.sorted_weights], [xd, wd],
                                         [g_rows.to(DEV), g_sw.to(DEV)])
            counts, offsets, rev, slot_pos, _ = cref.permute(ids.numpy(), E)
            np.testing.assert_array_equal(p.expert_counts.cpu().numpy(), counts, err_msg=label)
            np.testing.assert_array_equal(p.expert_offsets.cpu().numpy(), offsets, err_msg=label)
            np.testing.assert_array_equal(p.reverse_map_indices.cpu().numpy(), rev, err_msg=label)
            np.testing.assert_array_equal(p.slot_pos.cpu().numpy(), slot_pos, err_msg=label)
            want_w = np.empty(T * k, dtype=to_np(w).dtype)
            want_w[slot_pos] = to_np(w).reshape(-1)
            np.testing.assert_array_equal(to_np(p.sorted_weights), want_w, err_msg=label)
            np.testing.assert_array_equal(to_np(p.permuted_data), to_np(x)[rev], err_msg=label)
            want, _, _ = oracle_fwd([g_rows], torch.from_numpy(rev), torch.ones(T * k), T, xdt)
            _expect_bits(gx, want, label)
            np.testing.assert_array_equal(to_np(gw).reshape(-1), to_np(g_sw)[slot_pos],
                                          err_msg=label)
        else:
            T = _logu(rng, 20000)
            D = int(rng.choice([2, 8, 24, 256, 1000, 2048, 4104]))
            N = _logu(rng, max(1, min(50000, (1 << 21) // D, max(64 * T, 5000))))
            E = int(rng.integers(1, 400))
            pad = int(rng.choice([0, 0, 8, 40]))
            xdt, odt = DTS[int(rng.integers(3))], DTS[int(rng.integers(3))]
            mode = "atomic" if rng.random() < 0.4 else "det"
            r = rng.random()
            plan = 1 if r < 0.25 else (2 if r < 0.4 else 0)  # radix / bucketed / auto
            kernel_options(plan=plan)
            sizes = _split(rng, N, E)
            idx = torch.from_numpy(rng.integers(0, T, N))
            if rng.random() < 0.25:
                idx[:: int(rng.integers(3, 40))] = -1
            with_meta = bool(rng.random() < 0.5)
            label = (f"in-place case {case}: T={T} N={N} E={E} D={D} pad={pad} {xdt} out {odt} "
                     f"{mode} plan={plan} metadata={with_meta}")
            w = torch.rand(N, generator=gen)
            experts = [torch.randn(n, D, generator=gen).to(xdt) for n in sizes]
            init = torch.randn(T, D, generator=gen).to(odt)
            big = torch.zeros(T, D + pad, dtype=odt, device=DEV)
            out = big[:, :D]
            out.copy_(init.to(DEV))
            xd = [x.to(DEV) for x in experts]
            meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV) if with_meta else None
            fastmoe_amd.grouped_weighted_scatter_add(xd, idx.to(DEV), w.to(DEV), (T, D), out=out,
                                                     metadata=meta, mode=mode)
            want, acc, _ = oracle_fwd(experts, idx, w, T, odt, acc_init=init.float().numpy())
            if mode == "det":
                _expect_bits(out, want, label)
            else:
                valid = idx.numpy()[idx.numpy() >= 0]
                kmax = int(np.bincount(valid, minlength=T).max(initial=0))
                scale = abs_sum(experts, idx, w, T) + np.abs(init.float().numpy())
                if odt == torch.float32:
                    assert np.all(np.abs(out.cpu().numpy() - acc)
                                  <= reorder_tol(kmax + 1, scale)), label
                else:  # fp32 accumulation from the 16-bit initial contents, one rounding
                    want16 = torch.from_numpy(want.view(np.int16)).view(odt).float().numpy()
                    assert np.all(within_one_ulp16(out.float().cpu().numpy(), want16, odt,
                                                   kmax + 1, scale)), label
            if pad:
                assert not bool(big[:, D:].any()), label


def test_campaign_inverse_slot_plan_and_graphs(kernel_options):
    rng = np.random.default_rng(3303 + SEED_SHIFT)
    for case in range(150 * SCALE):
        gen = torch.Generator().manual_seed((3303 + SEED_SHIFT) * 1000 + case)
        kind = case % 3
        if kind == 0:
            T = _logu(rng, 60000)
            N = _logu(rng, min(200000, max(64 * T, 5000)))
            idt = [torch.int64, torch.int32][int(rng.integers(2))]
            idx = rng.integers(-2, T + 2, N) if rng.random() < 0.3 else rng.integers(0, T, N)
            label = f"inverse case {case}: T={T} N={N} {idt}"
            rp, rows = ops.invert_scatter_index(torch.from_numpy(idx).to(idt).to(DEV), T)
            want_rp, want_g = cref.plan(idx.astype(np.int64), T)
            np.testing.assert_array_equal(rp.cpu().numpy(), want_rp, err_msg=label)
            np.testing.assert_array_equal(rows.cpu().numpy(), want_g, err_msg=label)
        elif kind == 1:
            T, k = _logu(rng, 8000), int(rng.integers(1, 9))
            E = int(rng.choice([1, 3, 16, 64, 256, 257, 600]))
            D = int(rng.choice([8, 16, 64, 200, 1024, 2048]))
            T = max(1, min(T, (1 << 21) // (k * D)))
            xdt = DTS[int(rng.integers(3))]
            wdt = [torch.float32, torch.bfloat16][int(rng.integers(2))]
            ids = torch.from_numpy(rng.integers(0, E, (T, k)))
            label = f"slot-plan case {case}: T={T} k={k} E={E} D={D} {xdt} {wdt}"
            x = torch.randn(T, D, generator=gen).to(xdt)
            w = torch.rand(T, k, generator=gen).to(wdt)
            p = fastmoe_amd.permute_tokens(x.to(DEV), ids.to(DEV), w.to(DEV), E)
            counts = p.expert_counts.cpu().tolist()
            parts_cpu = [q.contiguous() for q in torch.split(p.permuted_data.cpu(), counts)]
            parts = [q.to(DEV).requires_grad_(True) for q in parts_cpu]
            sw = p.sorted_weights.detach().clone().requires_grad_(True)
            out = ops._GroupedCombinePermuted.apply((p.slot_pos, k), p.reverse_map_indices, sw,
                                                    (T, D), *parts)
            go = torch.randn(T, D, generator=gen).to(xdt)
            grads = torch.autograd.grad(out, [sw, *parts], go.to(DEV))
            rev, swc = p.reverse_map_indices.cpu(), p.sorted_weights.cpu()
            want, _, _ = oracle_fwd(parts_cpu, rev, swc, T, xdt)
            _expect_bits(out, want, label)
            want_gx, want_gw = oracle_bwd(parts_cpu, rev, swc, T, go)
            got_gx = np.concatenate([to_np(g).reshape(-1, D) for g in grads[1:]])
            np.testing.assert_array_equal(got_gx.view(want_gx.dtype), want_gx, err_msg=label)
            scale = abs_dot(parts_cpu, rev, go, T)
            rtol = 1e-6 if wdt == torch.float32 else 2.0 ** -8
            err = np.abs(grads[0].double().cpu().numpy() - want_gw)
            assert np.all(err <= 1e-6 * scale + rtol * np.abs(want_gw) + 1e-30), label
        else:
            T = _logu(rng, 4000)
            D = int(rng.choice([8, 64, 256, 1000, 2048]))
            N = _logu(rng, max(2, min(20000, (1 << 21) // D)))
            E = int(rng.integers(1, 300))
            xdt, odt = DTS[int(rng.integers(3))], DTS[int(rng.integers(3))]
            sizes = _split(rng, N, E)
            idx = torch.from_numpy(rng.integers(0, T, N))
            label = f"graph case {case}: T={T} N={N} E={E} D={D} {xdt} out {odt}"
            w = torch.rand(N, generator=gen)
            experts = [torch.randn(n, D, generator=gen).to(xdt) for n in sizes]
            xd = [e.to(DEV) for e in experts]
            idd, wd = idx.to(DEV), w.to(DEV)
            meta = fastmoe_amd.prepare_grouped_metadata(xd, DEV)
            out_static = torch.zeros(T, D, dtype=odt, device=DEV)
            fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), out=out_static,
                                                     metadata=meta)
            eager = bits(out_static).copy()
            want, _, _ = oracle_fwd(experts, idx, w, T, odt)
            _expect_bits(out_static, want, label)
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                out_static.zero_()
                with torch.cuda.graph(g, stream=s):
                    fastmoe_amd.grouped_weighted_scatter_add(xd, idd, wd, (T, D), out=out_static,
                                                             metadata=meta)
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            for r in range(3):
                out_static.zero_()
                g.replay()
                torch.cuda.synchronize()
                np.testing.assert_array_equal(bits(out_static), eager, err_msg=f"{label} replay {r}")
                _ = (torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)).sum().item()
            del g
