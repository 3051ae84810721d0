"""Shared helpers of the test-suite: tensor <-> numpy bit patterns and oracle drivers."""
from __future__ import annotations

import numpy as np
import torch

from oracle import cref

CODE = {torch.float32: cref.F32, torch.bfloat16: cref.BF16, torch.float16: cref.F16}


def to_np(t: torch.Tensor) -> np.ndarray:
    """Host numpy array of a tensor's storage: fp32 as float32, bf16/f16 as uint16 bits."""
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bit patterns (uint16 / uint32) for exact comparisons."""
    a = to_np(t)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def oracle_fwd(experts, idx, w, T, out_dtype, acc_init=None):
    """Expected output bits (storage of out_dtype) and the fp32 accumulator."""
    D = experts[0].shape[1]
    xs = [to_np(x) for x in experts]
    acc, bad = cref.combine_fwd(xs, to_np(idx.long()), to_np(w.float()), T, D,
                                CODE[experts[0].dtype], acc=acc_init)
    return cref.round_to(acc, CODE[out_dtype]), acc, bad


def oracle_bwd(experts, idx, w, T, grad_out):
    D = experts[0].shape[1]
    xs = [to_np(x) for x in experts]
    return cref.combine_bwd(xs, to_np(idx.long()), to_np(w.float()), T, D, to_np(grad_out),
                            CODE[experts[0].dtype])


def abs_dot(experts, idx, grad_out, T):
    """sum_d |grad_out[idx[g], d] * X[g, d]| per row (the scale of grad_w's rounding error)."""
    x = torch.cat([e.detach().float().cpu() for e in experts], 0).abs()
    go = grad_out.detach().float().cpu().abs()
    i = idx.cpu().long()
    valid = (i >= 0) & (i < T)
    out = torch.empty(x.shape[0], dtype=torch.float64)
    step = 2048  # bounded temporaries at full workload sizes
    for a in range(0, x.shape[0], step):
        rows = go[i[a: a + step].clamp(0, T - 1)].double()
        out[a: a + step] = (rows * x[a: a + step].double()).sum(-1) * valid[a: a + step].double()
    return out.numpy()


def reorder_tol(n_terms: int, scale):
    """Largest gap between two fp32 sums of the same n_terms values added in different orders.

    Recursive summation of n terms in fp32 lies within (n-1) * u * sum|terms| of the exact sum,
    u = 2^-24, to first order (Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed.,
    section 4.2); two different orders can therefore differ by twice that.  ``scale`` is
    sum|terms| per element; the factor (1 + 2^-20) covers the second-order term.
    """
    return 2.0 * max(n_terms - 1, 1) * 2.0 ** -24 * (1.0 + 2.0 ** -20) * scale + 1e-30


# bf16 / f16: unit roundoff, significand bits (with the implicit one), smallest spacing
_U16 = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
_P16 = {torch.bfloat16: 8, torch.float16: 11}
_MIN_ULP16 = {torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24}


def ulp16(x, dtype):
    """Spacing of the bf16 / f16 grid at |x| (at a power of two: the spacing above it)."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    _, e = np.frexp(a)  # a = m * 2^e, 0.5 <= m < 1
    ulp = np.ldexp(1.0, e - _P16[dtype])
    return np.where(a == 0, _MIN_ULP16[dtype], np.maximum(ulp, _MIN_ULP16[dtype]))


def within_one_ulp16(got, want, dtype, n_terms: int, scale):
    """The "<= 1 ulp after fp32 accumulation" bar for a 16-bit output: ``got`` is some fp32 sum
    of the terms rounded once to ``dtype``, ``want`` the oracle's (the sequential fp32 sum rounded
    once).  The two fp32 sums differ by at most reorder_tol(n_terms, scale); each rounding moves a
    value by at most half a spacing, so the results differ by at most one spacing (taken at the
    larger magnitude) plus that gap.  Elementwise boolean."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    tol = ulp16(np.maximum(np.abs(got), np.abs(want)), dtype) + reorder_tol(n_terms, scale)
    return np.abs(got - want) <= tol


def packed_tol(n_terms: int, scale, dtype):
    """Error bound of packed 16-bit atomics against the oracle's 16-bit result: each of the n
    terms is rounded to 16 bits and each of the n adds rounds the running sum (at most u times
    sum|terms| each, u the unit roundoff), and the oracle's own result is one rounding of its fp32
    sum: (n + 2) u sum|terms|, first order; the factor (1 + 2^-6) covers the higher-order terms."""
    return (n_terms + 2) * _U16[dtype] * (1.0 + 2.0 ** -6) * scale + _MIN_ULP16[dtype]


def abs_sum(experts, idx, w, T):
    """sum_g |w[g] * X[g, d]| per output element (scale of reordering error of a fp32 sum)."""
    D = experts[0].shape[1]
    xs = [to_np(x) for x in experts]
    code = CODE[experts[0].dtype]
    xs_abs = [np.abs(cref.widen(x, code)) for x in xs]
    acc, _ = cref.combine_fwd(xs_abs, to_np(idx.long()), np.abs(to_np(w.float())), T, D, cref.F32)
    return acc


# ---- golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py) -------------
GOLDEN_DIR = __import__("pathlib").Path(__file__).resolve().parent / "golden"
_TORCH_DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def golden_names():
    """The combine fixtures."""
    return sorted(p.stem for p in GOLDEN_DIR.glob("*.npz") if not p.stem.startswith("permute_"))


def permute_golden_names():
    """The dispatch-permutation fixtures."""
    return sorted(p.stem for p in GOLDEN_DIR.glob("permute_*.npz"))


def load_permute_golden(name: str) -> dict:
    """A permutation fixture as CPU tensors (ids, gates, x) plus the stored expected arrays."""
    z = np.load(GOLDEN_DIR / f"{name}.npz", allow_pickle=False)
    dt = _TORCH_DTYPES[str(z["x_dtype"])]
    case = {k: z[k] for k in z.files}
    case.update(ids=torch.from_numpy(z["ids"].copy()), gates=_from_store(z["gates"], dt),
                x=_from_store(z["x"], dt), E=int(z["E"]), dtype=dt)
    return case


def _from_store(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype in (torch.bfloat16, torch.float16):
        return torch.from_numpy(a.view(np.int16).copy()).view(dtype)
    return torch.from_numpy(a.copy())


def load_golden(name: str) -> dict:
    """A fixture as CPU tensors: experts (list), idx, w, grad_out, T, D, and the stored expected
    arrays (bit patterns) under their own keys."""
    z = np.load(GOLDEN_DIR / f"{name}.npz", allow_pickle=False)
    xdt = _TORCH_DTYPES[str(z["x_dtype"])]
    wdt = _TORCH_DTYPES[str(z["w_dtype"])]
    x = _from_store(z["x"], xdt)
    sizes = [int(s) for s in z["sizes"]]
    case = {k: z[k] for k in z.files}
    case.update(
        experts=[t.contiguous() for t in torch.split(x, sizes)],
        idx=torch.from_numpy(z["idx"].copy()),
        w=_from_store(z["w"], wdt),
        grad_out=_from_store(z["grad_out"], xdt),
        T=int(z["T"]),
        D=int(z["D"]),
        x_dtype=xdt,
        w_dtype=wdt,
    )
    return case
