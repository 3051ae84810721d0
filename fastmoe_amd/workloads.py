"""Synthetic combine workloads (the five BASELINE configurations plus the reference's own bench).

Routing follows the reference's producer, MoEFeedForward.gate_and_sort
(src/fastmoe/models/tiny_model.py:94-138): router logits -> top-k -> fp32 softmax over the top-k
-> sort the flattened expert ids (stable here, so inputs are reproducible) -> scatter index
(``reverse_map_indices``), sorted gates and per-expert row counts.  Expert outputs are ~N(0, 1)
in separate allocations, one per expert, sized by the routing counts.

The "published" workload restates the reference's kernel benchmark shape instead
(src/fastmoe/benchmarks/run_on_cloud.py:207-214, config.py:81-89): 256 experts x 64 rows,
``randint`` scatter indices over 4096 tokens, ``rand`` weights, fp32.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import numpy as np
import torch


@dataclass(frozen=True)
class Workload:
    name: str
    T: int          # tokens (rows of out)
    D: int          # hidden size
    E: int          # experts
    k: int          # top-k
    dtype: torch.dtype
    seed: int
    backward: bool  # the configuration is quoted for fwd + bwd
    routing: str = "topk"   # "topk" | "zipf" | "randint"

    @property
    def N(self) -> int:
        return self.T * self.k


WORKLOADS = {
    "plumbing": Workload("plumbing", 256, 512, 8, 2, torch.float32, 0, True),
    "mid": Workload("mid", 8192, 4096, 64, 6, torch.bfloat16, 1, False),
    "gigachat": Workload("gigachat", 4096, 16384, 256, 8, torch.bfloat16, 2, True),
    "skewed": Workload("skewed", 16384, 7168, 256, 8, torch.bfloat16, 3, False, "zipf"),
    "detatomic": Workload("detatomic", 32768, 16384, 256, 2, torch.bfloat16, 4, False),
    "published": Workload("published", 4096, 16384, 256, 4, torch.float32, 5, False, "randint"),
}


def zipf_bias(E: int, seed: int) -> np.ndarray:
    """Per-expert logit bias: Zipf(s=1.2) draws clipped at 10, so a few experts take most rows."""
    return np.minimum(np.random.default_rng(seed).zipf(1.2, E), 10).astype(np.float32)


def make_routing(wl: Workload, T: int | None = None) -> Tuple[torch.Tensor, torch.Tensor, List[int]]:
    """(scatter index int64[N], gate weights fp32[N], rows per expert) on the CPU, seeded."""
    T = wl.T if T is None else T
    gen = torch.Generator().manual_seed(wl.seed)
    if wl.routing == "randint":
        rows = wl.N // wl.E if T == wl.T else max(1, T * wl.k // wl.E)
        N = rows * wl.E
        idx = torch.randint(0, T, (N,), generator=gen)
        w = torch.rand(N, generator=gen)
        return idx, w, [rows] * wl.E
    logits = torch.randn(T, wl.E, generator=gen)
    if wl.routing == "zipf":
        logits = logits + torch.from_numpy(zipf_bias(wl.E, wl.seed))[None, :]
    top_w, top_i = torch.topk(logits, wl.k, dim=-1)
    top_w = torch.softmax(top_w, dim=-1, dtype=torch.float32)
    flat_e = top_i.reshape(-1)
    order = torch.argsort(flat_e, stable=True)
    idx = torch.arange(T).repeat_interleave(wl.k)[order]
    w = top_w.reshape(-1)[order].contiguous()
    counts = torch.bincount(flat_e, minlength=wl.E).tolist()
    return idx.contiguous(), w, counts


def make_topk(wl: Workload, T: int | None = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """The routing decision before the sort: (expert ids int64[T, k], fp32 gates [T, k]), seeded
    like make_routing (same logits, so the same rows result)."""
    if wl.routing == "randint":
        raise ValueError("the randint workload has no top-k routing decision")
    T = wl.T if T is None else T
    gen = torch.Generator().manual_seed(wl.seed)
    logits = torch.randn(T, wl.E, generator=gen)
    if wl.routing == "zipf":
        logits = logits + torch.from_numpy(zipf_bias(wl.E, wl.seed))[None, :]
    top_w, top_i = torch.topk(logits, wl.k, dim=-1)
    return top_i.contiguous(), torch.softmax(top_w, dim=-1, dtype=torch.float32).contiguous()


def make_experts(counts: List[int], D: int, dtype: torch.dtype, device, seed: int) -> List[torch.Tensor]:
    """One ~N(0, 1) buffer per expert, each its own allocation (empty experts get [0, D])."""
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed + 1000)
    out = []
    for n in counts:
        if dev.type == "cuda":
            x = torch.randn(n, D, generator=gen, device=dev, dtype=torch.float32).to(dtype)
        else:
            x = torch.randn(n, D, generator=gen, dtype=torch.float32).to(dtype)
        out.append(x)
    return out


def algorithmic_bytes(T: int, D: int, N: int, x_bytes: int, out_bytes: int, gate_bytes: int = 4,
                      grad_w: bool = True) -> Tuple[int, int]:
    """Compulsory HBM bytes (forward, backward) of one combine.

    forward : read X (N*D) + write out (T*D) + read idx (8 B) and w (gate_bytes) per row
    backward: read grad_out (T*D) + read X (N*D, for grad_w) + write grad_X (N*D)
              + read idx and w + write grad_w (gate_bytes) per row
    """
    fwd = N * D * x_bytes + T * D * out_bytes + N * (8 + gate_bytes)
    bwd = T * D * x_bytes + N * D * x_bytes * (2 if grad_w else 1) + N * (8 + gate_bytes)
    if grad_w:
        bwd += N * gate_bytes
    return fwd, bwd


def dispatch_bytes(T: int, D: int, N: int, x_bytes: int, gate_bytes: int = 4) -> Tuple[int, int]:
    """Compulsory HBM bytes (forward, backward) of one dispatch permutation.

    forward : read x (T*D) + write the packed rows (N*D) + per slot: read id (8) and gate, write
              sorted gate, reverse map (8) and slot -> row map (4)
    backward: read the packed-row gradient (N*D) + write grad x (T*D) + per slot: read reverse map
              (8) and unit gate (4), read gate grad, slot -> row map (4), write gate grad
    """
    fwd = T * D * x_bytes + N * D * x_bytes + N * (8 + 2 * gate_bytes + 8 + 4)
    bwd = N * D * x_bytes + T * D * x_bytes + N * (8 + 4 + 2 * gate_bytes + 4)
    return fwd, bwd


def kernel_bytes(T: int, D: int, N: int, x_bytes: int, out_bytes: int,
                 gate_bytes: int = 4) -> dict:
    """Compulsory HBM bytes of one launch of each kernel of the step, by timing-span name.

    fwd_det / fwd_atomic : the forward (as ``algorithmic_bytes``)
    bwd_gx               : read grad_out (T*D) + write grad_X (N*D) + read idx and w per row
    bwd_gw               : read grad_out (T*D) + read X (N*D) + read idx, write grad_w per row
    bwd                  : both gradients in one pass (as ``algorithmic_bytes``)
    fwd_small, bwd_small : the one-launch small path's forward and backward (as fwd_det, bwd)
    permute_gather       : read x (T*D) + write the packed rows (N*D) + read slot_pos per slot
    """
    fwd, bwd = algorithmic_bytes(T, D, N, x_bytes, out_bytes, gate_bytes)
    return {
        "permute_gather": T * D * x_bytes + N * D * x_bytes + N * 4,
        "fwd_det": fwd,
        "fwd_atomic": fwd,
        "bwd_gx": T * D * x_bytes + N * D * x_bytes + N * (8 + gate_bytes),
        "bwd_gw": T * D * x_bytes + N * D * x_bytes + N * (8 + gate_bytes),
        "bwd": bwd,
        "fwd_small": fwd,
        "bwd_small": bwd,
    }
