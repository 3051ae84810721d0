"""The oracle against the golden fixtures (tests/golden/*.npz).

The fixtures hold the reference's CPU algorithm evaluated with torch's CPU ops at the reference's
call sites (cat / mul / index_add_, run_on_cloud.py:17-20 and ops.py:373-384; index_select / mul /
cast, ops.py:344-353), so each check below compares two independent implementations: the C
oracle's scalar loops and torch's kernels.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import cref, torch_ref
from tests.helpers import CODE, golden_names, load_golden, to_np

NAMES = golden_names()


def test_fixture_set_is_complete():
    assert set(NAMES) >= {"kat_n10_d4", "topk_f32_t32_d24", "zipf_bf16_t48_d36",
                          "topk_f16_t16_d24_bf16w", "long_segments_f32"}


def test_kat_matches_reference_loop():
    """tests/test_cpu_moe.py:94-114: the weighted scatter-add against its brute-force loop
    (the reference's tolerance 1e-5; here the two agree bit for bit, same order and rounding)."""
    c = load_golden("kat_n10_d4")
    assert np.abs(c["out"] - c["out_loop"]).max() < 1e-5
    np.testing.assert_array_equal(c["out"].view(np.uint32), c["out_loop"].view(np.uint32))


@pytest.mark.parametrize("name", NAMES)
def test_oracle_forward_matches_fixture(name):
    c = load_golden(name)
    acc, bad = cref.combine_fwd([to_np(x) for x in c["experts"]], c["idx"].numpy(),
                                to_np(c["w"].float()), c["T"], c["D"], CODE[c["x_dtype"]])
    assert bad == 0
    got = cref.round_to(acc, CODE[c["x_dtype"]])
    want = c["out"]
    np.testing.assert_array_equal(got.view(np.uint32) if got.dtype == np.float32 else got,
                                  want.view(np.uint32) if want.dtype == np.float32 else want)
    if "out_fb" in c:  # the CPU fallback's fp32 output is the unrounded accumulator
        np.testing.assert_array_equal(acc.view(np.uint32), c["out_fb"].view(np.uint32))


@pytest.mark.parametrize("name", NAMES)
def test_oracle_backward_matches_fixture(name):
    c = load_golden(name)
    gx, gw = cref.combine_bwd([to_np(x) for x in c["experts"]], c["idx"].numpy(),
                              to_np(c["w"].float()), c["T"], c["D"], to_np(c["grad_out"]),
                              CODE[c["x_dtype"]])
    want = c["grad_x"]
    np.testing.assert_array_equal(gx.view(np.uint32) if gx.dtype == np.float32 else gx,
                                  want.view(np.uint32) if want.dtype == np.float32 else want)
    # both sides are fp64 sums of exact products, in different orders
    x = torch.cat(c["experts"], 0).double()
    scale = (c["grad_out"].double()[c["idx"]] * x).abs().sum(1).numpy()
    assert np.all(np.abs(gw - c["grad_w"]) <= 1e-14 * scale + 1e-300)


@pytest.mark.parametrize("name", NAMES)
def test_torch_restatement_reproduces_fixture(name):
    """Guards the fixtures against drift of torch's CPU kernels (and of oracle/torch_ref)."""
    c = load_golden(name)
    out = torch_ref.fwd_cat(c["experts"], c["idx"], c["w"], (c["T"], c["D"])).to(c["x_dtype"])
    np.testing.assert_array_equal(to_np(out), c["out"])
    sizes = [x.shape[0] for x in c["experts"]]
    gx = torch.cat(torch_ref.bwd_grad_x(c["grad_out"], c["idx"], c["w"], sizes, c["x_dtype"]), 0)
    np.testing.assert_array_equal(to_np(gx), c["grad_x"])


PERMUTE_NAMES = __import__("tests.helpers", fromlist=["x"]).permute_golden_names()


def test_permutation_fixture_set_is_complete():
    assert set(PERMUTE_NAMES) >= {"permute_topk_bf16_t40_d24", "permute_zipf_f32_t64_d16"}


@pytest.mark.parametrize("name", PERMUTE_NAMES)
def test_oracle_permutation_matches_fixture(name):
    """The C oracle's stable counting sort against the reference's torch calls
    (tiny_model.py:108-138 with a stable argsort) stored in the fixture."""
    from tests.helpers import load_permute_golden

    c = load_permute_golden(name)
    counts, offsets, rev, slot_pos, bad = cref.permute(c["ids"].numpy(), c["E"])
    assert bad == 0
    np.testing.assert_array_equal(counts, c["counts"])
    np.testing.assert_array_equal(offsets, c["offsets"])
    np.testing.assert_array_equal(rev, c["rev"])
    np.testing.assert_array_equal(slot_pos, c["slot_pos"])
    np.testing.assert_array_equal(to_np(c["x"])[rev], c["permuted"])
    sorted_gates = np.empty_like(c["sorted_gates"])
    sorted_gates[slot_pos] = to_np(c["gates"]).reshape(-1)
    np.testing.assert_array_equal(sorted_gates, c["sorted_gates"])
