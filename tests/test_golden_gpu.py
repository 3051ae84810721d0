"""The HIP combine against the golden fixtures (tests/golden/*.npz): forward bit for bit in the
deterministic mode, grad_X bit for bit, grad_w within 1e-6 * sum_d |grad_out * X| of the fp64
value; int64 and int32 scatter indices."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import fastmoe_amd
from tests.helpers import golden_names, load_golden, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
@pytest.mark.parametrize("name", golden_names())
def test_hip_path_matches_fixture(name, index_dtype):
    c = load_golden(name)
    xs = [x.to(DEV).requires_grad_(True) for x in c["experts"]]
    idx = c["idx"].to(index_dtype).to(DEV)
    w = c["w"].to(DEV).requires_grad_(True)
    out = fastmoe_amd.grouped_weighted_scatter_add(xs, idx, w, (c["T"], c["D"]), mode="det")
    np.testing.assert_array_equal(to_np(out), c["out"])
    grads = torch.autograd.grad(out, [w, *xs], c["grad_out"].to(DEV))
    gx = torch.cat([g.detach() for g in grads[1:]], 0)
    np.testing.assert_array_equal(to_np(gx), c["grad_x"])
    x = torch.cat(c["experts"], 0).double()
    scale = (c["grad_out"].double()[c["idx"]] * x).abs().sum(1).numpy()
    assert grads[0].dtype == c["w_dtype"]
    tol = 1e-6 if c["w_dtype"] == torch.float32 else 2.0 ** -8  # grad_w stored in the gates' dtype
    err = np.abs(grads[0].double().cpu().numpy() - c["grad_w"])
    assert np.all(err <= tol * scale + 1e-30)


@pytest.mark.parametrize("name", ["kat_n10_d4", "long_segments_f32"])
def test_weighted_scatter_add_matches_fixture(name):
    """The single-tensor entry point (ops.py:397-398), into a caller-provided zero output."""
    c = load_golden(name)
    src = torch.cat(c["experts"], 0).to(DEV)
    out = torch.zeros(c["T"], c["D"], device=DEV)
    fastmoe_amd.weighted_scatter_add(src, c["idx"].to(DEV), c["w"].to(DEV), (c["T"], c["D"]),
                                     out=out)
    np.testing.assert_array_equal(to_np(out).view(np.uint32), c["out_fb"].view(np.uint32))


@pytest.mark.parametrize("name", __import__("tests.helpers", fromlist=["x"]).permute_golden_names())
@pytest.mark.parametrize("id_dtype", [torch.int64, torch.int32])
def test_permute_tokens_matches_fixture(name, id_dtype):
    from tests.helpers import load_permute_golden

    c = load_permute_golden(name)
    p = fastmoe_amd.permute_tokens(c["x"].to(DEV), c["ids"].to(id_dtype).to(DEV),
                                   c["gates"].to(DEV), c["E"])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(p.expert_counts.cpu().numpy(), c["counts"])
    np.testing.assert_array_equal(p.expert_offsets.cpu().numpy(), c["offsets"])
    np.testing.assert_array_equal(p.reverse_map_indices.cpu().numpy(), c["rev"])
    np.testing.assert_array_equal(p.slot_pos.cpu().numpy(), c["slot_pos"])
    np.testing.assert_array_equal(to_np(p.sorted_weights), c["sorted_gates"])
    np.testing.assert_array_equal(to_np(p.permuted_data), c["permuted"])
