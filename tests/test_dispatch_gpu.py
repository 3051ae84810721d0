"""GPU parity of the dispatch permutation and the MoE layer stages (fastmoe_amd.dispatch, .moe).

Bars:
  * permute_tokens: counts, offsets, reverse map and slot -> row map equal the C oracle's stable
    counting sort exactly; sorted gates and permuted rows are bit copies.
  * its backward: grad of x_flat equals the oracle combine of the packed gradient rows with unit
    gates (ascending row order, fp32, rounded once) bit for bit; grad of the gates is the inverse
    permutation, bit for bit.
  * gate_and_sort / unpermute / MoEFeedForward: the reference's torch formulation of the same
    layer (tiny_model.py:79-164, :282-294, :396-409, with a stable argsort) on the same weights,
    fp32: permutation outputs bit-equal, layer output and every gradient within fp32 reordering
    bounds.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import fastmoe_amd
from fastmoe_amd.consts import MoEImplementation
from oracle import cref
from tests.helpers import bits, oracle_fwd, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _routing(T, E, k, seed, zipf=False):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    if zipf:
        bias = np.minimum(np.random.default_rng(seed).zipf(1.2, E), 10).astype(np.float32)
        logits = logits + torch.from_numpy(bias)[None, :]
    w, ids = torch.topk(logits, k, dim=-1)
    return ids, torch.softmax(w, -1, dtype=torch.float32)


def _check_permute(x, ids, w, E):
    T, k = ids.shape
    p = fastmoe_amd.permute_tokens(x.to(DEV), ids.to(DEV), w.to(DEV), E)
    torch.cuda.synchronize()
    counts, offsets, rev, slot_pos, bad = cref.permute(ids.numpy(), E)
    np.testing.assert_array_equal(p.expert_counts.cpu().numpy(), counts)
    np.testing.assert_array_equal(p.expert_offsets.cpu().numpy(), offsets)
    np.testing.assert_array_equal(p.reverse_map_indices.cpu().numpy(), rev)
    np.testing.assert_array_equal(p.slot_pos.cpu().numpy(), slot_pos)
    want_w = np.empty(T * k, dtype=to_np(w).dtype)
    want_w[slot_pos] = to_np(w).reshape(-1)
    np.testing.assert_array_equal(to_np(p.sorted_weights), want_w)
    want_x = to_np(x)[rev]
    np.testing.assert_array_equal(to_np(p.permuted_data), want_x)
    return p, bad


@pytest.mark.parametrize("T,D,E,k,dtype", [
    (256, 512, 8, 2, torch.float32),       # plumbing shape
    (512, 4096, 64, 6, torch.bfloat16),    # mid shape, scaled
    (256, 16384, 256, 8, torch.bfloat16),  # gigachat shape, scaled
    (300, 100, 16, 4, torch.float16),      # 200-byte rows: 4-byte copies
    (65, 7, 3, 3, torch.bfloat16),         # 14-byte rows: 2-byte copies
    (40, 64, 1, 1, torch.float32),         # one expert, k = 1
])
def test_permute_matches_oracle(T, D, E, k, dtype):
    ids, w = _routing(T, E, k, seed=T + D)
    x = torch.randn(T, D, generator=torch.Generator().manual_seed(1)).to(dtype)
    _check_permute(x, ids, w.to(dtype) if dtype != torch.float32 else w, E)


def test_permute_skewed_int32_ids_and_empty_experts():
    ids, w = _routing(2048, 256, 8, seed=3, zipf=True)
    x = torch.randn(2048, 256).to(torch.bfloat16)
    p, _ = _check_permute(x, ids.to(torch.int32), w, 256)
    assert (p.expert_counts == 0).any()


def test_permute_many_experts_uses_large_variant():
    ids, w = _routing(300, 3000, 4, seed=4)
    _check_permute(torch.randn(300, 32), ids, w, 3000)


def test_permute_random_shapes():
    """30 seeded random permutations against the oracle: tokens, top-k, experts (including more
    than 1024, the small-block ranking), row bytes (16-, 4- and 2-byte copies), id and gate
    dtypes, ids with repeats within a token, and out-of-range ids."""
    rng = np.random.default_rng(5150)
    dts = [torch.float32, torch.bfloat16, torch.float16]
    for case in range(30):
        T = int(rng.choice([1, 3, 64, 500, 2000]))
        E = int(rng.choice([1, 2, 17, 256, 1500, 4096]))
        k = int(rng.integers(1, 9))
        D = int(rng.choice([1, 7, 16, 100, 1024]))
        gen = torch.Generator().manual_seed(200 + case)
        ids = torch.from_numpy(rng.integers(0, E, (T, k)))
        if case % 4 == 0:
            ids[torch.from_numpy(rng.random((T, k)) < 0.05)] = E   # out of range
        if case % 4 == 2:
            ids = ids.to(torch.int32)
        w = torch.rand(T, k, generator=gen).to([torch.float32, torch.bfloat16][case % 2])
        x = torch.randn(T, D, generator=gen).to(dts[int(rng.integers(3))])
        p, bad = _check_permute(x, ids, w, E)
        assert bad == int(((ids < 0) | (ids >= E)).sum()), f"case {case}"


def test_permute_invalid_ids_go_last_and_validate_raises():
    ids, w = _routing(100, 8, 2, seed=5)
    ids[3, 0] = 8
    ids[50, 1] = -1
    x = torch.randn(100, 32)
    _, bad = _check_permute(x, ids, w, 8)
    assert bad == 2
    with pytest.raises(IndexError):
        fastmoe_amd.permute_tokens(x.to(DEV), ids.to(DEV), w.to(DEV), 8, validate=True)


def test_permute_strided_rows():
    ids, w = _routing(64, 8, 2, seed=6)
    base = torch.randn(64, 96)
    x = base[:, 16:80]  # row stride 96, unit column stride
    p = fastmoe_amd.permute_tokens(base.to(DEV)[:, 16:80], ids.to(DEV), w.to(DEV), 8)
    _, _, rev, _, _ = cref.permute(ids.numpy(), 8)
    np.testing.assert_array_equal(p.permuted_data.cpu().numpy(), x.numpy()[rev])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_permute_backward(dtype):
    T, D, E, k = 128, 320, 16, 4
    ids, w = _routing(T, E, k, seed=7)
    x = torch.randn(T, D).to(dtype)
    wd = w.to(dtype).to(DEV).requires_grad_(True)
    xd = x.to(DEV).requires_grad_(True)
    p = fastmoe_amd.permute_tokens(xd, ids.to(DEV), wd, E)
    g_rows = torch.randn(T * k, D, generator=torch.Generator().manual_seed(8)).to(dtype)
    g_sw = torch.randn(T * k, generator=torch.Generator().manual_seed(9)).to(dtype)
    gx, gw = torch.autograd.grad([p.permuted_data, p.sorted_weights], [xd, wd],
                                 [g_rows.to(DEV), g_sw.to(DEV)])
    _, _, rev, slot_pos, _ = cref.permute(ids.numpy(), E)
    want, _, _ = oracle_fwd([g_rows], torch.from_numpy(rev), torch.ones(T * k), T, dtype)
    np.testing.assert_array_equal(bits(gx), want.view(np.uint32) if dtype == torch.float32 else want)
    np.testing.assert_array_equal(to_np(gw).reshape(-1), to_np(g_sw)[slot_pos])


# ---- the layer: FAST (HIP permutation + grouped combine over the per-expert list) vs the
# reference's torch formulation on the same weights ------------------------------------------
def _reference_layer(layer, x):
    """tiny_model.py:79-164 (stable argsort), :282-294 and :396-409 (STANDARD), world size 1."""
    B, T, D = x.shape
    x_flat = x.view(-1, D)
    logits = layer.router(x_flat)
    tw, ti = torch.topk(logits, layer.top_k, dim=-1)
    tw = F.softmax(tw, dim=-1, dtype=torch.float32).type_as(x)
    flat = ti.view(-1)
    order = torch.argsort(flat, stable=True)
    rev = torch.arange(x_flat.shape[0], device=x.device).repeat_interleave(layer.top_k)[order]
    sw = tw.view(-1)[order]
    permuted = x_flat[rev]
    counts = torch.bincount(flat[order], minlength=layer.num_experts).tolist()
    outs = [e(c) if c.shape[0] else c for e, c in zip(layer.experts, permuted.split(counts))]
    x_out = torch.cat(outs, 0) * sw.unsqueeze(-1)
    out = torch.zeros(B * T, D, device=x.device, dtype=x_out.dtype).index_add_(0, rev, x_out)
    return out.view(B, T, D), permuted, rev, sw


def test_gate_and_sort_matches_reference_formulation():
    torch.manual_seed(0)
    layer = fastmoe_amd.MoEFeedForward(64, 128, 8, 2).to(DEV)
    x = torch.randn(2, 48, 64, device=DEV)
    permuted, rank_counts, counts_by_rank, rev, sw, shape = fastmoe_amd.gate_and_sort(
        x, layer.router, 2, 8)
    _, want_perm, want_rev, want_sw = _reference_layer(layer, x)
    assert shape == (2, 48) and rank_counts.tolist() == [192] and counts_by_rank.shape == (1, 8)
    assert torch.equal(rev, want_rev) and torch.equal(sw, want_sw)
    assert torch.equal(permuted, want_perm)


@pytest.mark.parametrize("shape", [(2, 40, 64, 96, 8, 2), (3, 50, 128, 64, 32, 4)])
@pytest.mark.parametrize("impl", [MoEImplementation.FAST, MoEImplementation.STANDARD])
def test_moe_layer_forward_backward(impl, shape):
    B, T, dim, ff, E, k = shape
    torch.manual_seed(1)
    layer = fastmoe_amd.MoEFeedForward(dim, ff, E, k, implementation=impl).to(DEV)
    x = torch.randn(B, T, dim, device=DEV, requires_grad=True)
    y = layer(x)
    go = torch.randn_like(y)
    params = [x, layer.router.weight, *[p for e in layer.experts for p in e.parameters()]]
    grads = torch.autograd.grad(y, params, go, allow_unused=True)
    x2 = x.detach().clone().requires_grad_(True)
    want, _, _, _ = _reference_layer(layer, x2)
    want_grads = torch.autograd.grad(want, [x2, *params[1:]], go, allow_unused=True)
    torch.testing.assert_close(y, want, rtol=1e-5, atol=1e-5)
    for g, wg in zip(grads, want_grads):
        if g is None or wg is None:  # an expert that received no rows
            assert g is None and wg is None
            continue
        torch.testing.assert_close(g, wg, rtol=1e-4, atol=1e-5)


def test_unpermute_list_equals_packed():
    """The per-expert list and its concatenation give the same combine bits (no cat needed)."""
    g = torch.Generator().manual_seed(2)
    sizes = [5, 0, 9, 2]
    xs = [torch.randn(n, 40, generator=g).to(DEV) for n in sizes]
    rev = torch.randint(0, 8, (16,), generator=g).to(DEV)
    sw = torch.rand(16, generator=g).to(DEV)
    a = fastmoe_amd.unpermute(xs, rev, sw, (2, 4))
    b = fastmoe_amd.unpermute(torch.cat(xs), rev, sw, (2, 4))
    assert torch.equal(a, b) and a.shape == (2, 4, 40)


# ---- the combine's plan built from the permutation's slot map ------------------------------------
def _plan_segments(plan, N, T):
    """{token: sorted [(g, w bits, src)]} of a plan workspace (device -> host)."""
    lib = fastmoe_amd._abi.lib()
    h = plan.cpu()
    rp = h[lib.fmoe_plan_row_ptr_offset(N, T):].view(torch.int32)[: T + 2].numpy()
    rec = h[lib.fmoe_plan_records_offset(N, T):][: 16 * N].view(torch.int64).view(-1, 2).numpy()
    st = h[lib.fmoe_plan_status_offset():][:12].view(torch.int32).numpy()
    segs = {}
    for t in range(T):
        rows = [(int(r[1] >> 32), int(r[1] & 0xFFFFFFFF), int(r[0])) for r in rec[rp[t]:rp[t + 1]]]
        segs[t] = sorted(rows)
    return rp, segs, st


def test_plan_from_slots_equals_plan_from_scatter_index():
    T, D, E, k = 300, 96, 16, 4
    ids, w = _routing(T, E, k, seed=21)
    x = torch.randn(T, D).to(DEV)
    p = fastmoe_amd.permute_tokens(x, ids.to(DEV), w.to(DEV), E)
    experts = [c.contiguous() for c in p.permuted_data.split(p.expert_counts.tolist())]
    meta = fastmoe_amd.prepare_grouped_metadata(experts, DEV)
    N = T * k
    general = fastmoe_amd.build_plan(meta, p.reverse_map_indices, p.sorted_weights, T)
    from_slots = fastmoe_amd.ops.build_plan_from_slots(meta, p.slot_pos, p.sorted_weights, T, k)
    torch.cuda.synchronize()
    rp_a, seg_a, st_a = _plan_segments(general, N, T)
    rp_b, seg_b, st_b = _plan_segments(from_slots, N, T)
    np.testing.assert_array_equal(rp_a, rp_b)
    assert seg_a == seg_b
    assert st_b[0] == 0 and st_b[2] == k and st_a[0] == 0


@pytest.mark.parametrize("E", [32, 300])
def test_metadata_and_slot_plan_in_one_call_equals_two_calls(E):
    """fmoe_build_metadata_and_plan_from_slots writes exactly what fmoe_build_metadata +
    fmoe_build_plan_from_slots write: one launch for up to 256 experts, the two calls above."""
    T, D, k = 300, 40, 4
    ids, w = _routing(T, E, k, seed=23)
    x = torch.randn(T, D).to(DEV)
    p = fastmoe_amd.permute_tokens(x, ids.to(DEV), w.to(DEV), E)
    experts = [c.contiguous() for c in p.permuted_data.split(p.expert_counts.tolist())]
    N = T * k
    meta1, plan1 = fastmoe_amd.ops.prepare_metadata_and_plan_from_slots(
        experts, p.slot_pos, p.sorted_weights, T, k)
    meta2 = fastmoe_amd.prepare_grouped_metadata(experts, DEV)
    plan2 = fastmoe_amd.ops.build_plan_from_slots(meta2, p.slot_pos, p.sorted_weights, T, k)
    torch.cuda.synchronize()
    for a, b in [(meta1.ptr_table, meta2.ptr_table), (meta1.chunk_sizes, meta2.chunk_sizes),
                 (meta1.offsets_full, meta2.offsets_full),
                 (meta1.max_rows_device, meta2.max_rows_device)]:
        assert torch.equal(a, b)
    rp1, seg1, st1 = _plan_segments(plan1, N, T)
    rp2, seg2, st2 = _plan_segments(plan2, N, T)
    np.testing.assert_array_equal(rp1, rp2)
    assert seg1 == seg2
    np.testing.assert_array_equal(st1[:3], st2[:3])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unpermute_with_permutation_is_bit_identical(dtype):
    T, D, E, k = 256, 192, 32, 6
    ids, w = _routing(T, E, k, seed=22)
    x = torch.randn(T, D).to(dtype).to(DEV)
    p = fastmoe_amd.permute_tokens(x, ids.to(DEV), w.to(dtype).to(DEV), E)
    parts = [c.clone().requires_grad_(True) for c in p.permuted_data.split(p.expert_counts.tolist())]
    sw = p.sorted_weights.detach().clone().requires_grad_(True)
    go = torch.randn(1, T, D, generator=torch.Generator().manual_seed(3)).to(dtype).to(DEV)
    a = fastmoe_amd.unpermute(parts, p.reverse_map_indices, sw, (1, T), permutation=p)
    ga = torch.autograd.grad(a, [sw, *parts], go)
    b = fastmoe_amd.unpermute(parts, p.reverse_map_indices, sw, (1, T))
    gb = torch.autograd.grad(b, [sw, *parts], go)
    assert torch.equal(a, b)
    for u, v in zip(ga, gb):
        assert torch.equal(u, v)


def test_plan_from_slots_with_inconsistent_slots_stays_in_bounds():
    """Out-of-range and repeated slot positions (an inconsistent caller) are clamped to zero-gate
    records on packed row 0: the combine runs, reads and writes only inside its buffers."""
    T, D, E, k = 64, 32, 4, 2
    N = T * k
    experts = [torch.randn(N // E, D, device=DEV) for _ in range(E)]
    meta = fastmoe_amd.prepare_grouped_metadata(experts, DEV)
    slots = torch.arange(N, dtype=torch.int32)
    slots[5] = N + 7
    slots[9] = -3
    slots[11] = slots[12]
    w = torch.rand(N, device=DEV)
    plan = fastmoe_amd.ops.build_plan_from_slots(meta, slots.to(DEV), w, T, k)
    out = torch.empty(T, D, device=DEV)
    fastmoe_amd.ops._launch_fwd(meta, fastmoe_amd._abi.MODE_DET, plan, None, None, out, False)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()


def test_graph_capture_of_the_layer_data_path_replays():
    """permute_tokens -> per-expert views -> unpermute with the slot-map plan, captured once as a
    graph: every replay equals the eager result bit for bit."""
    T, D, E, k = 256, 128, 16, 4
    ids, w = _routing(T, E, k, seed=31)
    x = torch.randn(T, D).to(torch.bfloat16).to(DEV)
    idd, wd = ids.to(DEV), w.to(DEV)
    counts = fastmoe_amd.permute_tokens(x, idd, wd, E).expert_counts.tolist()

    def step():
        p = fastmoe_amd.permute_tokens(x, idd, wd, E)
        parts = p.permuted_data.split(counts)
        return fastmoe_amd.unpermute(parts, p.reverse_map_indices, p.sorted_weights, (1, T),
                                     permutation=p)

    with torch.no_grad():
        eager = bits(step())
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            static = step()
        for _ in range(4):
            g.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(bits(static), eager)
            _ = (torch.randn(64, 64, device=DEV) @ torch.randn(64, 64, device=DEV)).sum().item()
