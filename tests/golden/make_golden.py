"""Writes the golden fixtures of this directory (run from the repository root):

    python tests/golden/make_golden.py

Each ``<name>.npz`` holds seeded inputs of the combine and the outputs of the reference's CPU
algorithm on them, computed with torch CPU ops exactly as the reference calls them:

  out     torch.cat -> * w[:, None] -> index_add_ into fp32 zeros, then cast to the expert dtype
          (src/fastmoe/benchmarks/run_on_cloud.py:17-20; the GPU autograd path returns the expert
          dtype, src/fastmoe/kernels/ops.py:327)
  out_fb  the per-expert index_add_ of the CPU fallback into a weights-dtype output
          (src/fastmoe/kernels/ops.py:373-384), fp32 gates only
  grad_x  grad_out.index_select(0, idx) * w[:, None], cast back to the expert dtype by autograd
          (src/fastmoe/kernels/ops.py:344-353)
  grad_w  sum_d grad_out[idx[g], d] * X[g, d] in fp64 (autograd of the STANDARD combine,
          src/fastmoe/models/tiny_model.py:400-403; the reference's fast path returns none)

The ``permute_*`` cases hold the dispatch permutation of src/fastmoe/models/tiny_model.py:94-138
(stable argsort) on seeded top-k routing.

The ``kat_n10_d4`` case is the shape of the reference's only known-answer test
(tests/test_cpu_moe.py:94-114, N=10, D=4, 5 tokens), seeded here; ``out_loop`` is that test's
brute-force loop.  16-bit tensors are stored as their uint16 bit patterns; dtypes as strings.
Nothing here imports the reference: torch is the library the reference itself calls.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from fastmoe_amd.workloads import Workload, make_experts, make_routing  # noqa: E402
from oracle import torch_ref  # noqa: E402

NAMES = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _store(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _case(xs, idx, w, T, grad_out, with_fallback: bool) -> dict:
    D = xs[0].shape[1]
    xdt = xs[0].dtype
    acc = torch_ref.fwd_cat(xs, idx, w, (T, D))          # fp32 (fp32 or promoted product)
    out = acc.to(xdt)
    sizes = [x.shape[0] for x in xs]
    gx = torch.cat(torch_ref.bwd_grad_x(grad_out, idx, w, sizes, xdt), 0)
    gw = torch_ref.bwd_grad_w_fp64(xs, idx, w, grad_out, T)
    case = {
        "x": _store(torch.cat(xs, 0)),
        "sizes": np.array(sizes, dtype=np.int64),
        "idx": idx.numpy().astype(np.int64),
        "w": _store(w),
        "grad_out": _store(grad_out),
        "T": np.array(T, dtype=np.int64),
        "D": np.array(D, dtype=np.int64),
        "x_dtype": np.array(NAMES[xdt]),
        "w_dtype": np.array(NAMES[w.dtype]),
        "out": _store(out),
        "grad_x": _store(gx),
        "grad_w": gw.numpy().astype(np.float64),
    }
    if with_fallback:
        case["out_fb"] = _store(torch_ref.fwd_fallback(xs, idx, w, (T, D)))
    return case


def kat_n10_d4() -> dict:
    gen = torch.Generator().manual_seed(94)
    N, D, T = 10, 4, 5
    src = torch.randn(N, D, generator=gen)
    weights = torch.rand(N, generator=gen)
    indices = torch.randint(0, T, (N,), generator=gen)
    grad_out = torch.randn(T, D, generator=gen)
    case = _case([src], indices, weights, T, grad_out, True)
    loop = torch.zeros(T, D)
    for i in range(N):  # tests/test_cpu_moe.py:105-110
        loop[indices[i].item()] += src[i] * weights[i].item()
    case["out_loop"] = loop.numpy()
    return case


def routed(name: str, T: int, D: int, E: int, k: int, dtype, seed: int, routing: str = "topk",
           w_dtype=torch.float32) -> dict:
    wl = Workload(name, T, D, E, k, dtype, seed, True, routing)
    idx, w, counts = make_routing(wl)
    xs = make_experts(counts, D, dtype, "cpu", seed)
    w = w.to(w_dtype)
    grad_out = torch.randn(T, D, generator=torch.Generator().manual_seed(seed + 7)).to(dtype)
    return _case(xs, idx, w, T, grad_out, w_dtype == torch.float32)


def long_segments() -> dict:
    """Three tokens receive 200 rows (randint scatter indices, the shape of the reference's kernel
    benchmark, run_on_cloud.py:207-214): segments far longer than 64 rows."""
    gen = torch.Generator().manual_seed(207)
    E, rows, D, T = 5, 40, 8, 3
    idx = torch.randint(0, T, (E * rows,), generator=gen)
    w = torch.rand(E * rows, generator=gen)
    xs = [torch.randn(rows, D, generator=gen) for _ in range(E)]
    grad_out = torch.randn(T, D, generator=gen)
    return _case(xs, idx, w, T, grad_out, True)


def permute_case(T: int, D: int, E: int, k: int, dtype, seed: int, zipf: bool = False) -> dict:
    """The dispatch permutation (src/fastmoe/models/tiny_model.py:94-138) evaluated with the
    reference's own torch calls, argsort made stable: expert ids, gates, token rows, and the
    expected counts, offsets, reverse map, slot -> row map, sorted gates and gathered rows."""
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=gen)
    if zipf:
        logits = logits + torch.from_numpy(np.minimum(np.random.default_rng(seed).zipf(1.2, E), 10)
                                           .astype(np.float32))[None, :]
    x = torch.randn(T, D, generator=gen).to(dtype)
    topk_weights, topk_indices = torch.topk(logits, k, dim=-1)                      # :95
    topk_weights = torch.softmax(topk_weights, dim=-1, dtype=torch.float32).to(dtype)  # :100
    flat = topk_indices.view(-1)
    sort_indices = torch.argsort(flat, stable=True)                                 # :112
    rev = torch.arange(T).repeat_interleave(k)[sort_indices]                        # :121-125
    sorted_weights = topk_weights.view(-1)[sort_indices]                            # :128
    permuted = x[rev]                                                               # :133
    counts = torch.bincount(flat[sort_indices], minlength=E)                        # :138
    slot_pos = torch.empty_like(sort_indices)
    slot_pos[sort_indices] = torch.arange(T * k)
    return {
        "ids": topk_indices.numpy().astype(np.int64),
        "gates": _store(topk_weights),
        "x": _store(x),
        "E": np.array(E, dtype=np.int64),
        "x_dtype": np.array(NAMES[dtype]),
        "counts": counts.numpy().astype(np.int64),
        "offsets": np.concatenate([[0], np.cumsum(counts.numpy())]).astype(np.int64),
        "rev": rev.numpy().astype(np.int64),
        "slot_pos": slot_pos.numpy().astype(np.int32),
        "sorted_gates": _store(sorted_weights),
        "permuted": _store(permuted),
    }


CASES = {
    "kat_n10_d4": kat_n10_d4,
    # plumbing recipe (top-2 of 8 experts, fp32) at a fixture-sized T and D
    "topk_f32_t32_d24": lambda: routed("topk_f32", 32, 24, 8, 2, torch.float32, 0),
    # skewed recipe (Zipf expert bias: empty experts), bf16, D not a multiple of 8
    "zipf_bf16_t48_d36": lambda: routed("zipf_bf16", 48, 36, 6, 3, torch.bfloat16, 3, "zipf"),
    # fp16 expert outputs with bf16 gates (the product promotes to fp32)
    "topk_f16_t16_d24_bf16w": lambda: routed("topk_f16", 16, 24, 4, 2, torch.float16, 5,
                                             w_dtype=torch.bfloat16),
    "long_segments_f32": long_segments,
    # the dispatch permutation that produces such scatter indices
    "permute_topk_bf16_t40_d24": lambda: permute_case(40, 24, 8, 3, torch.bfloat16, 11),
    "permute_zipf_f32_t64_d16": lambda: permute_case(64, 16, 12, 4, torch.float32, 12, zipf=True),
}


def main() -> None:
    for name, fn in CASES.items():
        case = fn()
        np.savez_compressed(HERE / f"{name}.npz", **case)
        print(f"wrote {name}.npz: " + ", ".join(f"{k}{list(v.shape)}" for k, v in case.items()))


if __name__ == "__main__":
    main()
