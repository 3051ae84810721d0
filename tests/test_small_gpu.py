"""GPU parity of the one-launch small path (fmoe_combine_fwd_small / fmoe_combine_bwd_small).

The small path must give what the planned path gives, bit for bit -- forward, grad_X and grad_w --
and the forward and grad_X must equal the C oracle bit for bit (grad_w within 1e-6 of
sum|terms|).  Each case runs the public autograd call twice, with the "small" option forcing the
small path (2) and turning it off (1).  The cases cover what the small kernels do differently
from the planned ones: tokens of more than 64 rows (the compaction window refills), indices out
of range (staged as -1), rows that are not 16-byte aligned (element loads), D that no 16-byte
vector divides (the scalar kernels), empty experts, the row and expert limits, int32 indices,
16-bit gates, a single token and rows of 32 KiB (where the planned grad_w pass stages grad_out
in LDS).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import fastmoe_amd
from fastmoe_amd import ops
from tests.helpers import abs_dot, bits, oracle_bwd, oracle_fwd, to_np, ulp16

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _long_segments(N, T, gen):
    """Most rows on token 0 (hundreds of rows: several 64-row windows), the rest spread."""
    idx = torch.randint(0, T, (N,), generator=gen)
    idx[torch.rand(N, generator=gen) < 0.7] = 0
    return idx


def _with_invalid(N, T, gen):
    idx = torch.randint(0, T, (N,), generator=gen)
    idx[::7] = T + 3
    idx[3::11] = -1
    return idx


# name -> (T, sizes per expert, D, expert dtype, index maker, options)
CASES = {
    "plumbing_f32": (256, [64] * 8, 512, torch.float32, None, {}),
    "decode_bf16": (64, [2] * 256, 7168, torch.bfloat16, None, {}),
    "f16_top4": (128, [16] * 32, 2048, torch.float16, None, {}),
    "odd_D": (50, [30, 0, 41, 9, 20], 100, torch.bfloat16, None, {}),
    "long_segments": (4, [400, 350, 250], 264, torch.bfloat16, _long_segments, {}),
    "invalid_indices": (40, [50, 0, 70, 30], 1024, torch.float32, _with_invalid, {}),
    "misaligned": (33, [20, 17, 0, 31], 264, torch.bfloat16, None, {"misalign": True}),
    "max_rows_experts": (512, [16] * 255 + [16], 256, torch.float32, None, {}),
    "int32_bf16_gates": (97, [60, 80, 0, 45], 1536, torch.bfloat16, None,
                         {"idx_dtype": torch.int32, "w_dtype": torch.bfloat16}),
    "one_token": (1, [13, 27], 4096, torch.bfloat16, None, {}),
    # rows of 32 KiB: the planned grad_w pass takes its LDS-staged form and the small backward
    # its 4-vector column step
    "wide_rows_bf16": (16, [16] * 8, 16384, torch.bfloat16, None, {}),
    "wide_rows_f32": (16, [8] * 16, 8192, torch.float32, None, {}),
}


def _make(case):
    T, sizes, D, dtype, idx_fn, opts = CASES[case]
    gen = torch.Generator().manual_seed(sum(map(ord, case)))
    N = sum(sizes)
    idx = torch.randint(0, T, (N,), generator=gen) if idx_fn is None else idx_fn(N, T, gen)
    w = torch.rand(N, generator=gen).to(opts.get("w_dtype", torch.float32))
    pad = 1 if opts.get("misalign") else 0
    xd = []
    for n in sizes:
        flat = torch.randn(n * D + pad, generator=gen).to(dtype).to(DEV)
        xd.append(flat[pad:].view(n, D))  # pad: the rows start 1 element past an allocation
    if pad:
        assert any(x.data_ptr() % 16 for x in xd if x.shape[0])
    go = torch.randn(T, D, generator=gen).to(dtype)
    return T, D, idx.to(opts.get("idx_dtype", torch.int64)), w, xd, go


def _fwd_bwd(xd, idx, w, go, T, D):
    xs = [x.detach().requires_grad_(True) for x in xd]
    wg = w.detach().clone().requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx, wg, (T, D))
    grads = torch.autograd.grad(out, [wg, *xs], go)
    torch.cuda.synchronize()
    return out, grads[0], torch.cat([g.detach() for g in grads[1:]], 0)


@pytest.mark.parametrize("case", list(CASES))
def test_small_path_equals_planned_path_and_oracle(case, kernel_options):
    T, D, idx, w, xd, go = _make(case)
    N, E = idx.numel(), len(xd)
    idd, wd, god = idx.to(DEV), w.to(DEV), go.to(DEV)
    print(f"small-path case {case}: T={T} D={D} N={N} E={E}", flush=True)
    kernel_options(small=2)
    assert ops._use_small(N, T, E)
    got = _fwd_bwd(xd, idd, wd, god, T, D)
    kernel_options(small=1)
    assert not ops._use_small(N, T, E)
    ref = _fwd_bwd(xd, idd, wd, god, T, D)
    for a, b in zip(got, ref):  # out, grad_w, grad_X
        np.testing.assert_array_equal(bits(a), bits(b))
    experts = [x.detach().cpu() for x in xd]
    want, _, _ = oracle_fwd(experts, idx, w, T, xd[0].dtype)
    np.testing.assert_array_equal(bits(got[0]), want.view(np.uint32) if want.dtype == np.float32
                                  else want)
    want_gx, want_gw = oracle_bwd(experts, idx, w, T, go)
    np.testing.assert_array_equal(to_np(got[2]), want_gx)
    tol = 1e-6 * abs_dot(experts, idx, go, T) + 1e-30
    if w.dtype != torch.float32:  # a 16-bit gate's gradient is rounded to its dtype once more
        tol = tol + ulp16(want_gw, w.dtype)
    assert np.all(np.abs(got[1].double().cpu().numpy() - want_gw) <= tol)


def test_small_path_in_place_accumulates_like_the_oracle(kernel_options):
    """The in-place call (the reference's out.zero_() + accumulate contract) through the small
    path: out keeps its contents where no row is routed and adds the rows in ascending order."""
    T, D, idx, w, xd, _ = _make("plumbing_f32")
    idx = idx.clone()
    idx[idx == 5] = 6  # token 5 gets no rows: keeps its contents
    gen = torch.Generator().manual_seed(3)
    out0 = torch.randn(T, D, generator=gen)
    kernel_options(small=2)
    out = out0.to(DEV)
    fastmoe_amd.grouped_weighted_scatter_add(xd, idx.to(DEV), w.to(DEV), (T, D), out=out)
    kernel_options(small=1)
    ref = out0.to(DEV)
    fastmoe_amd.grouped_weighted_scatter_add(xd, idx.to(DEV), w.to(DEV), (T, D), out=ref)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out), bits(ref))
    want, _, _ = oracle_fwd([x.cpu() for x in xd], idx, w, T, torch.float32,
                            acc_init=out0.numpy().copy())
    np.testing.assert_array_equal(bits(out), want.view(np.uint32))
    np.testing.assert_array_equal(bits(out[5]), bits(out0[5]))


def test_small_path_validate_raises_on_out_of_range_indices(kernel_options):
    T, D, idx, w, xd, _ = _make("invalid_indices")
    kernel_options(small=2)
    with pytest.raises(IndexError, match="outside"):
        fastmoe_amd.grouped_weighted_scatter_add(xd, idx.to(DEV), w.to(DEV), (T, D),
                                                 validate=True)
    torch.cuda.synchronize()



@pytest.mark.parametrize("force", [0, 2])
def test_validating_in_place_call_leaves_out_untouched(force, kernel_options):
    """A validating in-place call of small-path size raises IndexError before any forward launch,
    so ``out`` keeps its bits (a caller that catches the error and retries adds nothing twice)."""
    T, D, idx, w, xd, _ = _make("invalid_indices")
    kernel_options(small=force)
    out0 = torch.randn(T, D, generator=torch.Generator().manual_seed(11))
    out = out0.to(DEV)
    with pytest.raises(IndexError, match="outside"):
        fastmoe_amd.grouped_weighted_scatter_add(xd, idx.to(DEV), w.to(DEV), (T, D), out=out,
                                                 validate=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(out), bits(out0))
