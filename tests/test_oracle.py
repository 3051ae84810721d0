"""Pin the C oracle (oracle/combine_ref.c) before trusting it (CPU only).

Each check is chosen so that a plausible mistake in the oracle -- a dropped term, a wrong index,
a swapped operand, FMA contraction, a wrong rounding -- fails at least one of them:
  * the reference's own known-answer form (tests/test_cpu_moe.py:94-114 in the reference):
    brute-force Python loop over rows, N=10, D=4, 5 output rows, duplicate indices;
  * bit-equality with torch's CPU path as the reference runs it (ops.py:373-384 per-expert
    index_add_ and run_on_cloud.py:17-20 cat/mul/index_add_) in fp32, with bf16 inputs too;
  * closed forms: doubling w doubles out exactly; a k=1 permutation is an exact scatter;
    all-ones inputs count multiplicities; empty experts add nothing; any split of the packed rows
    into experts gives the same bits; fp32 vs an fp64 sum is within the reordering bound;
  * backward: grad_X equals torch's index_select * w cast to the expert dtype bit for bit;
    grad_w equals torch autograd of the standard path in fp64;
  * plan: equals a stable argsort of idx; metadata equals numpy cumsum/max;
  * conversions: bf16/f16 rounding equals torch's .to() on ties, subnormals, overflow, NaN.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cref, torch_ref
from tests.helpers import to_np


def _routed(seed, T, D, E, k, dtype=torch.float32, empty=()):
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=gen)
    for e in empty:
        logits[:, e] = -1e9
    top_w, top_i = torch.topk(logits, k, dim=-1)
    top_w = torch.softmax(top_w, -1, dtype=torch.float32)
    flat = top_i.reshape(-1)
    order = torch.argsort(flat, stable=True)
    idx = torch.arange(T).repeat_interleave(k)[order]
    w = top_w.reshape(-1)[order].contiguous()
    counts = torch.bincount(flat, minlength=E).tolist()
    xs = [torch.randn(n, D, generator=gen).to(dtype) for n in counts]
    return xs, idx, w, counts


def _cref_fwd(xs, idx, w, T, D, acc=None):
    code = {torch.float32: cref.F32, torch.bfloat16: cref.BF16, torch.float16: cref.F16}[xs[0].dtype]
    out, bad = cref.combine_fwd([to_np(x) for x in xs], idx.numpy(), w.float().numpy(), T, D, code,
                                acc=acc)
    return out, bad


def test_known_answer_brute_force_loop():
    """The reference's only KAT of the path, seeded: loop `out[idx[i]] += src[i] * w[i]`."""
    gen = torch.Generator().manual_seed(0)
    N, D = 10, 4
    src = torch.randn(N, D, generator=gen)
    weights = torch.rand(N, generator=gen)
    indices = torch.randint(0, 5, (N,), generator=gen)
    out, bad = _cref_fwd([src], indices, weights, 5, D)
    gt = torch.zeros(5, D)
    for i in range(N):
        gt[indices[i].item()] += src[i] * weights[i].item()
    assert bad == 0
    np.testing.assert_array_equal(out, gt.numpy())  # same order, same fp32 rounding: exact


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_bitexact_vs_torch_reference_paths(dtype):
    xs, idx, w, counts = _routed(1, T=96, D=40, E=6, k=2, dtype=dtype, empty=(3,))
    assert counts[3] == 0
    T, D = 96, 40
    got, _ = _cref_fwd(xs, idx, w, T, D)
    fallback = torch_ref.fwd_fallback(xs, idx, w, (T, D))   # out dtype = weights.dtype = fp32
    cat = torch_ref.fwd_cat(xs, idx, w, (T, D))
    np.testing.assert_array_equal(got.view(np.uint32), fallback.numpy().view(np.uint32))
    np.testing.assert_array_equal(got.view(np.uint32), cat.numpy().view(np.uint32))


def test_accumulate_into_existing_out():
    xs, idx, w, _ = _routed(2, T=50, D=16, E=4, k=2)
    init = torch.randn(50, 16, generator=torch.Generator().manual_seed(3))
    got, _ = _cref_fwd(xs, idx, w, 50, 16, acc=init.numpy())
    want = torch_ref.fwd_fallback(xs, idx, w, (50, 16), out=init.clone())
    np.testing.assert_array_equal(got.view(np.uint32), want.numpy().view(np.uint32))


def test_linearity_doubling_w_is_exact():
    xs, idx, w, _ = _routed(4, T=64, D=24, E=5, k=3)
    a, _ = _cref_fwd(xs, idx, w, 64, 24)
    b, _ = _cref_fwd(xs, idx, w * 2, 64, 24)
    np.testing.assert_array_equal((a * 2).view(np.uint32), b.view(np.uint32))


def test_k1_permutation_is_exact_scatter():
    gen = torch.Generator().manual_seed(5)
    T, D = 37, 9
    x = torch.randn(T, D, generator=gen)
    perm = torch.randperm(T, generator=gen)
    w = torch.rand(T, generator=gen)
    got, _ = _cref_fwd([x[:10], x[10:]], perm, w, T, D)
    want = torch.zeros(T, D)
    want[perm] = x * w[:, None]
    np.testing.assert_array_equal(got, want.numpy())


def test_all_ones_counts_multiplicity():
    gen = torch.Generator().manual_seed(6)
    T, D, N = 11, 3, 60
    idx = torch.randint(0, T, (N,), generator=gen)
    got, _ = _cref_fwd([torch.ones(25, D), torch.ones(0, D), torch.ones(35, D)], idx,
                       torch.ones(N), T, D)
    counts = np.bincount(idx.numpy(), minlength=T).astype(np.float32)
    np.testing.assert_array_equal(got, np.repeat(counts[:, None], D, 1))


def test_split_invariance():
    xs, idx, w, _ = _routed(7, T=40, D=8, E=3, k=2)
    cat = torch.cat(xs)
    a, _ = _cref_fwd(xs, idx, w, 40, 8)
    b, _ = _cref_fwd([cat], idx, w, 40, 8)
    c, _ = _cref_fwd(list(torch.split(cat, [1, 0, 50, cat.shape[0] - 51])), idx, w, 40, 8)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(a, c)


def test_fp32_sum_within_reordering_bound_of_fp64():
    xs, idx, w, _ = _routed(8, T=30, D=12, E=4, k=4)
    got, _ = _cref_fwd(xs, idx, w, 30, 12)
    x64 = torch.cat(xs).double()
    exact = torch.zeros(30, 12, dtype=torch.float64).index_add_(0, idx, x64 * w.double()[:, None])
    scale = torch.zeros(30, 12, dtype=torch.float64).index_add_(0, idx, (x64 * w.double()[:, None]).abs())
    assert np.all(np.abs(got - exact.numpy()) <= 2 * 4 * 2.0 ** -24 * scale.numpy())


def test_invalid_indices_are_skipped_and_counted():
    x = torch.randn(5, 4)
    idx = torch.tensor([0, -1, 3, 7, 3])
    got, bad = _cref_fwd([x], idx, torch.ones(5), 4, 4)
    assert bad == 2
    want = torch.zeros(4, 4)
    want[0] += x[0]
    want[3] += x[2]
    want[3] += x[4]
    np.testing.assert_array_equal(got, want.numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_matches_torch(dtype):
    xs, idx, w, counts = _routed(9, T=48, D=32, E=5, k=2, dtype=dtype)
    T, D = 48, 32
    go = torch.randn(T, D, generator=torch.Generator().manual_seed(10)).to(dtype)
    code = cref.F32 if dtype == torch.float32 else cref.BF16
    gx, gw = cref.combine_bwd([to_np(x) for x in xs], idx.numpy(), w.numpy(), T, D, to_np(go), code)
    want_gx = torch.cat(torch_ref.bwd_grad_x(go, idx, w, counts, dtype))
    np.testing.assert_array_equal(gx, to_np(want_gx))
    want_gw = torch_ref.bwd_grad_w_fp64(xs, idx, w, go, T).numpy()
    scale = (go.double()[idx].abs() * torch.cat(xs).double().abs()).sum(-1).numpy()
    assert np.all(np.abs(gw - want_gw) <= 1e-12 * scale + 1e-300)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_backward_16bit_rounds_the_fp32_product_twice_like_torch(dtype):
    """grad_X of 16-bit experts is the fp32 product rounded to fp32, then cast (two roundings):
    torch's index_select * w then .to(dtype) (ops.py:344-353 + autograd's cast).  The inputs hold
    elements where rounding the exact product once would give another value, so an oracle that
    rounded once would fail here."""
    T, D, E, k = 300, 256, 8, 2
    xs, idx, w, counts = _routed(13, T=T, D=D, E=E, k=k, dtype=dtype)
    go = torch.randn(T, D, generator=torch.Generator().manual_seed(14)).to(dtype)
    code = cref.F16 if dtype == torch.float16 else cref.BF16
    gx, _ = cref.combine_bwd([to_np(x) for x in xs], idx.numpy(), w.numpy(), T, D, to_np(go), code,
                             want_w=False)
    want = torch.cat(torch_ref.bwd_grad_x(go, idx, w, counts, dtype))
    np.testing.assert_array_equal(gx, to_np(want))
    # one rounding of the exact (fp64) product, straight to the 16-bit format (torch's own
    # fp64 -> 16-bit cast goes through fp32, i.e. rounds twice itself)
    exact = (go.double()[idx] * w.double()[:, None]).numpy()
    if dtype == torch.float16:
        once = exact.astype(np.float16).view(np.uint16)
    else:  # 8 significant bits, half to even; the result is exact in bf16
        m, e = np.frexp(exact)
        once = to_np(torch.from_numpy(np.ldexp(np.round(m * 256) / 256, e)).to(dtype))
    assert np.count_nonzero(once != to_np(want)) > 0  # the double rounding is exercised


def test_backward_invalid_rows_get_zero():
    x = torch.randn(3, 4)
    idx = torch.tensor([1, 9, 0])
    go = torch.randn(2, 4)
    gx, gw = cref.combine_bwd([x.numpy()], idx.numpy(), np.ones(3, np.float32), 2, 4, go.numpy())
    assert np.all(gx[1] == 0) and gw[1] == 0
    np.testing.assert_array_equal(gx[0], go[1].numpy())
    # the zero is +0 whatever the gate's sign (the kernels store zeros; 0 * w would give -0)
    for code, dtype in ((cref.F32, torch.float32), (cref.BF16, torch.bfloat16)):
        xs = [to_np(x.to(dtype))]
        gx, _ = cref.combine_bwd(xs, idx.numpy(), np.array([1, -2, -1], np.float32), 2, 4,
                                 to_np(go.to(dtype)), code)
        raw = gx[1].view(np.uint32) if gx.dtype == np.float32 else gx[1]
        assert not raw.any()


def test_plan_is_stable_argsort():
    gen = torch.Generator().manual_seed(12)
    T, N = 23, 200
    idx = torch.randint(-2, T + 2, (N,), generator=gen).numpy()
    row_ptr, g_list = cref.plan(idx, T)
    key = np.where((idx >= 0) & (idx < T), idx, T)
    np.testing.assert_array_equal(g_list, np.argsort(key, kind="stable"))
    np.testing.assert_array_equal(row_ptr, np.concatenate([[0], np.cumsum(np.bincount(key, minlength=T + 1))]))


def test_metadata_closed_form():
    rows = [4, 0, 7, 1, 0]
    off, mx = cref.metadata(rows)
    np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(rows)]))
    assert mx == 7


def test_rounding_matches_torch_casts():
    vals = [0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,
            65504.0, 65519.0, 65520.0, 1e-5, 6.0e-8, 2.0 ** -24, 1.5 * 2.0 ** -24, 2.0 ** -25,
            3.0e38, -3.0e38, float("inf"), -float("inf"), 1e-40, 5.960464477539063e-08]
    gen = torch.Generator().manual_seed(13)
    rnd = (torch.randn(4000, generator=gen) * torch.exp2(torch.randint(-30, 30, (4000,), generator=gen).float()))
    a = torch.cat([torch.tensor(vals), rnd]).float()
    for code, dt in ((cref.BF16, torch.bfloat16), (cref.F16, torch.float16)):
        got = cref.round_to(a.numpy(), code)
        want = a.to(dt).view(torch.int16).numpy().view(np.uint16)
        np.testing.assert_array_equal(got, want)
        back = cref.widen(want, code)
        np.testing.assert_array_equal(back.view(np.uint32), a.to(dt).float().numpy().view(np.uint32))
    nan = cref.round_to(np.array([np.nan], np.float32), cref.BF16)
    assert nan[0] == 0x7FC0


class _Mutant:
    """Plausible oracle mistakes, planted in Python copies of the oracle's forward (CPU only);
    the pinning checks above must reject each of them."""

    @staticmethod
    def fwd(xs, idx, w, T, D, mistake):
        out = np.zeros((T, D), np.float32)
        g = 0
        for x in xs:
            for r in range(x.shape[0]):
                t = int(idx[g])
                if mistake == "drop_last_row" and g == len(idx) - 1:
                    g += 1
                    continue
                wg = np.float32(w[g])
                if mistake == "index_off_by_one":
                    t = (t + 1) % T
                if mistake == "fma":
                    out[t] = (out[t].astype(np.float64) + x[r].astype(np.float64) * wg).astype(np.float32)
                elif mistake == "reverse_order":
                    pass
                else:
                    out[t] = out[t] + x[r] * wg
                g += 1
        if mistake == "reverse_order":
            g = len(idx)
            for x in reversed(xs):
                for r in reversed(range(x.shape[0])):
                    g -= 1
                    out[int(idx[g])] = out[int(idx[g])] + x[r] * np.float32(w[g])
        return out


@pytest.mark.parametrize("mistake", ["drop_last_row", "index_off_by_one", "fma", "reverse_order"])
def test_pinning_checks_reject_planted_mistakes(mistake):
    xs, idx, w, _ = _routed(14, T=64, D=16, E=4, k=3)
    T, D = 64, 16
    good = torch_ref.fwd_fallback(xs, idx, w, (T, D)).numpy()
    np_xs = [x.numpy() for x in xs]
    ok = _Mutant.fwd(np_xs, idx.numpy(), w.numpy(), T, D, None)
    np.testing.assert_array_equal(ok.view(np.uint32), good.view(np.uint32))
    bad = _Mutant.fwd(np_xs, idx.numpy(), w.numpy(), T, D, mistake)
    assert not np.array_equal(bad.view(np.uint32), good.view(np.uint32))


@pytest.mark.parametrize("n", [3, 4, 8])
def test_reorder_tolerance_covers_two_summation_orders(n):
    """The tolerance the GPU tests allow between the atomic forward and the oracle: two fp32
    sums of the same n terms in different orders.  Each order lies within (n-1) u sum|terms| of
    the exact sum (u = 2^-24), so their gap can exceed that one-sided bound -- it does here for
    3 terms -- and never exceeds twice it (reorder_tol)."""
    from tests.helpers import reorder_tol

    rng = np.random.default_rng(n)
    M = 100_000
    x = rng.standard_normal((M, n)).astype(np.float32)
    perm = rng.permuted(np.tile(np.arange(n), (M, 1)), axis=1)
    xp = np.take_along_axis(x, perm, 1)
    s1 = np.zeros(M, np.float32)
    s2 = np.zeros(M, np.float32)
    for i in range(n):
        s1 = s1 + x[:, i]
        s2 = s2 + xp[:, i]
    scale = np.abs(x.astype(np.float64)).sum(1)
    gap = np.abs(s1.astype(np.float64) - s2.astype(np.float64))
    assert np.all(gap <= reorder_tol(n, scale))
    if n == 3:
        assert np.any(gap > (n - 1) * 2.0 ** -24 * scale)


def _round16(a: np.ndarray, dtype) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dtype).float().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [2, 3, 8])
def test_one_ulp_bar_covers_reordered_fp32_sums_and_rejects_two(dtype, n):
    """The bar of the atomic mode with a 16-bit output (fp32 accumulation, one rounding): two fp32
    sums of the same terms in different orders, each rounded once, pass within_one_ulp16; the same
    result moved by two spacings fails it."""
    from tests.helpers import ulp16, within_one_ulp16

    rng = np.random.default_rng(10 * n + (dtype == torch.float16))
    M = 100_000
    x = rng.standard_normal((M, n)).astype(np.float32)
    xp = np.take_along_axis(x, rng.permuted(np.tile(np.arange(n), (M, 1)), axis=1), 1)
    s1 = np.zeros(M, np.float32)
    s2 = np.zeros(M, np.float32)
    for i in range(n):
        s1 = s1 + x[:, i]
        s2 = s2 + xp[:, i]
    scale = np.abs(x.astype(np.float64)).sum(1)
    r1, r2 = _round16(s1, dtype), _round16(s2, dtype)
    assert np.all(within_one_ulp16(r2, r1, dtype, n, scale))
    if n > 2:  # (two terms add commutatively: one result)
        assert np.any(r1 != r2)  # the orders do round differently somewhere
    moved = r2 + 2 * ulp16(r2, dtype)
    assert np.mean(within_one_ulp16(moved, r1, dtype, n, scale)) < 0.01


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [2, 8])
def test_packed_bound_covers_rounding_at_every_add_and_catches_a_dropped_term(dtype, n):
    """packed_tol against a model of packed 16-bit atomics (every term rounded to 16 bits, every
    add rounded to 16 bits, round to nearest even, in any order): the model stays within the bound
    of the oracle's result (the sequential fp32 sum rounded once); dropping one term exceeds it
    on most outputs."""
    from tests.helpers import packed_tol

    rng = np.random.default_rng(20 * n + (dtype == torch.float16))
    M = 50_000
    x = rng.standard_normal((M, n)).astype(np.float32)
    xp = np.take_along_axis(x, rng.permuted(np.tile(np.arange(n), (M, 1)), axis=1), 1)
    oracle = np.zeros(M, np.float32)
    for i in range(n):
        oracle = oracle + x[:, i]
    oracle16 = _round16(oracle, dtype)
    scale = np.abs(x.astype(np.float64)).sum(1)

    def packed(cols):
        acc = np.zeros(M, np.float32)
        for i in cols:
            acc = _round16(acc + _round16(xp[:, i], dtype), dtype)
        return acc

    err = np.abs(packed(range(n)).astype(np.float64) - oracle16)
    assert np.all(err <= packed_tol(n, scale, dtype))
    dropped = np.abs(packed(range(1, n)).astype(np.float64) - oracle16)
    assert np.mean(dropped > packed_tol(n, scale, dtype)) > 0.5
