"""Host-side logic of the operator API that needs no GPU: the drop-in surface, refusals of CPU
tensors, mode parsing, workload generation and the byte accounting of the roofline."""
from __future__ import annotations

import inspect

import numpy as np
import pytest
import torch

import fastmoe_amd
from fastmoe_amd import ops
from fastmoe_amd.consts import MoEImplementation
from fastmoe_amd.kernels import ops as kops
from fastmoe_amd.workloads import WORKLOADS, algorithmic_bytes, make_experts, make_routing


def test_reference_names_and_signatures():
    """Same public names and positional parameters as src/fastmoe/kernels/ops.py:200,365,397."""
    sig = inspect.signature(kops.grouped_weighted_scatter_add)
    assert list(sig.parameters)[:6] == ["expert_tensors", "indices", "weights", "out_shape", "out",
                                        "metadata"]
    assert sig.parameters["out"].default is None and sig.parameters["metadata"].default is None
    sig = inspect.signature(kops.weighted_scatter_add)
    assert list(sig.parameters)[:5] == ["src", "indices", "weights", "out_shape", "out"]
    assert list(inspect.signature(kops.prepare_grouped_metadata).parameters)[:2] == [
        "expert_tensors", "device"]
    assert issubclass(kops.GroupedWeightedScatterAdd, torch.autograd.Function)
    assert MoEImplementation.FAST == "fast" and MoEImplementation.STANDARD == "standard"


def test_cpu_tensors_raise_instead_of_falling_back():
    src = torch.randn(10, 4)
    idx = torch.randint(0, 5, (10,))
    w = torch.rand(10)
    with pytest.raises(RuntimeError, match="only on the GPU"):
        fastmoe_amd.weighted_scatter_add(src, idx, w, (5, 4))
    with pytest.raises(RuntimeError, match="only on the GPU"):
        fastmoe_amd.grouped_weighted_scatter_add([src], idx, w, (5, 4), out=torch.zeros(5, 4))
    with pytest.raises(RuntimeError, match="only on the GPU"):
        fastmoe_amd.prepare_grouped_metadata([src], "cpu")


def test_mode_parsing(monkeypatch):
    assert ops._mode_code(None) == ops._abi.MODE_DET
    assert ops._mode_code("atomic") == ops._abi.MODE_ATOMIC
    assert ops._mode_code("atomic_packed") == ops._abi.MODE_ATOMIC_PACKED
    monkeypatch.setattr(ops, "_DEFAULT_MODE", "atomic")  # FASTMOE_COMBINE_MODE, read at import
    assert ops._mode_code(None) == ops._abi.MODE_ATOMIC
    with pytest.raises(ValueError):
        ops._mode_code("fast")


def test_workloads_match_baseline_configs():
    wl = WORKLOADS["gigachat"]
    assert (wl.T, wl.D, wl.E, wl.k, wl.dtype) == (4096, 16384, 256, 8, torch.bfloat16)
    fwd, bwd = algorithmic_bytes(wl.T, wl.D, wl.N, 2, 2)
    # compulsory bytes: fwd = N*D*2 + T*D*2 + 12N, bwd = T*D*2 + 2*N*D*2 + 16N
    assert (fwd, bwd, fwd + bwd) == (1208352768, 2282225664, 3490578432)
    assert algorithmic_bytes(256, 512, 512, 4, 4) == (1579008, 2629632)
    assert algorithmic_bytes(8192, 4096, 49152, 2, 2)[0] == 470351872
    assert algorithmic_bytes(16384, 7168, 131072, 2, 2)[0] == 2115502080
    assert algorithmic_bytes(32768, 16384, 65536, 2, 2)[0] == 3222011904


def test_routing_generator_is_topk_structured_and_seeded():
    wl = WORKLOADS["plumbing"]
    idx, w, counts = make_routing(wl)
    idx2, w2, counts2 = make_routing(wl)
    assert torch.equal(idx, idx2) and torch.equal(w, w2) and counts == counts2
    assert idx.numel() == wl.N == sum(counts) and len(counts) == wl.E
    per_token = np.bincount(idx.numpy(), minlength=wl.T)
    assert np.all(per_token == wl.k)
    sums = torch.zeros(wl.T).index_add_(0, idx, w)
    assert torch.allclose(sums, torch.ones(wl.T), atol=1e-6)  # softmax over each token's top-k
    xs = make_experts(counts, wl.D, wl.dtype, "cpu", wl.seed)
    assert [x.shape[0] for x in xs] == counts


def test_skewed_routing_has_empty_and_hot_experts():
    wl = WORKLOADS["skewed"]
    _, _, counts = make_routing(wl, 2048)
    c = np.array(counts)
    # bias = min(zipf(1.2), 10): experts whose draw reaches the clip take nearly all rows
    assert (c == 0).sum() > 50 and c.max() > 1.5 * c.mean()
