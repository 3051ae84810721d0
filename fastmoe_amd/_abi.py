"""ctypes binding of ``libfastmoe_amd.so`` (the C ABI declared in ``include/fastmoe_amd.h``).

The library is built in-tree by ``python -m fastmoe_amd.build``.  There is no fallback: if the
library is missing or does not load, :func:`lib` raises, so no caller can silently run anything
but the gfx950 kernels.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfastmoe_amd.so"

ABI_VERSION = 2

# enum fmoe_dtype / fmoe_mode / fmoe_status (include/fastmoe_amd.h)
F32, BF16, F16, I64, I32 = 0, 1, 2, 3, 4
MODE_DET, MODE_ATOMIC, MODE_ATOMIC_PACKED = 0, 1, 2
OK, EINVAL, EHIP, ERANGE = 0, -1, -2, -3

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p

# name -> (restype, argtypes); exactly the symbols of include/fastmoe_amd.h
SIGNATURES: dict[str, tuple] = {
    "fmoe_abi_version": (_c_int, []),
    "fmoe_last_error": (ctypes.c_char_p, []),
    "fmoe_set_option": (_c_int, [ctypes.c_char_p, _c_i64, ctypes.POINTER(_c_i64)]),
    "fmoe_get_option": (_c_int, [ctypes.c_char_p, ctypes.POINTER(_c_i64)]),
    "fmoe_build_metadata": (
        _c_int,
        [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp],
    ),
    "fmoe_plan_path": (_c_int, [_c_i64, _c_i64, _c_i64]),
    "fmoe_plan_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "fmoe_plan_status_offset": (_c_i64, []),
    "fmoe_plan_row_ptr_offset": (_c_i64, [_c_i64, _c_i64]),
    "fmoe_plan_records_offset": (_c_i64, [_c_i64, _c_i64]),
    "fmoe_build_plan": (
        _c_int,
        [_c_vp, _c_int, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp, _c_vp],
    ),
    "fmoe_build_metadata_and_plan": (
        _c_int,
        [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
         _c_int, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_vp],
    ),
    "fmoe_build_plan_from_slots": (
        _c_int,
        [_c_vp, _c_i64, _c_i64, _c_vp, _c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp],
    ),
    "fmoe_build_metadata_and_plan_from_slots": (
        _c_int,
        [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
         _c_i64, _c_i64, _c_vp, _c_int, _c_i64, _c_vp, _c_vp],
    ),
    "fmoe_invert_scatter_index": (
        _c_int, [_c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp],
    ),
    "fmoe_combine_fwd_workspace_bytes": (_c_i64, [_c_int, _c_i64, _c_i64, _c_int]),
    "fmoe_combine_fwd": (
        _c_int,
        [_c_int, _c_vp, _c_vp, _c_int, _c_vp, _c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_int, _c_vp, _c_int, _c_i64, _c_int, _c_vp, _c_i64, _c_vp],
    ),
    "fmoe_combine_fwd_noalloc": (
        _c_int,
        [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_int, _c_vp, _c_int,
         _c_i64, _c_i64, _c_int, _c_vp, _c_int, _c_i64, _c_int, _c_vp],
    ),
    "fmoe_combine_bwd": (
        _c_int,
        [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_vp, _c_int, _c_i64, _c_vp, _c_vp, _c_int, _c_vp],
    ),
    "fmoe_combine_small_max_rows": (_c_i64, []),
    "fmoe_combine_fwd_small": (
        _c_int,
        [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_int, _c_vp, _c_int,
         _c_i64, _c_i64, _c_int, _c_vp, _c_int, _c_i64, _c_int, _c_vp, _c_vp],
    ),
    "fmoe_combine_bwd_small": (
        _c_int,
        [ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_int, _c_vp, _c_int,
         _c_i64, _c_i64, _c_int, _c_vp, _c_int, _c_i64, _c_vp, _c_vp, _c_int, _c_vp],
    ),
    "fmoe_permute_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "fmoe_permute_build": (
        _c_int,
        [_c_vp, _c_int, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
         _c_vp, _c_vp, _c_vp],
    ),
    "fmoe_permute_gather": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp]),
    "fmoe_permute_gate_grad": (_c_int, [_c_vp, _c_i64, _c_vp, _c_int, _c_vp, _c_vp]),
}

_LIB: ctypes.CDLL | None = None


class FastMoEError(RuntimeError):
    """A C-ABI call returned a negative status."""


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is missing or of another ABI version."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = Path(os.environ.get("FASTMOE_AMD_LIB", LIB_PATH))
    if not path.exists():
        raise FastMoEError(
            f"fastmoe_amd: {path} is missing; build the gfx950 kernels with "
            "`python -m fastmoe_amd.build` (there is no non-HIP fallback)"
        )
    handle = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        try:
            fn = getattr(handle, name)
        except AttributeError:
            raise FastMoEError(
                f"fastmoe_amd: {path} does not export {name} (a library built from other sources); "
                "rebuild it with `python -m fastmoe_amd.build`"
            ) from None
        fn.restype = restype
        fn.argtypes = argtypes
    ver = handle.fmoe_abi_version()
    if ver != ABI_VERSION:
        raise FastMoEError(f"fastmoe_amd: ABI version {ver} != expected {ABI_VERSION}")
    _LIB = handle
    return handle


def check(rc: int, what: str) -> None:
    """Raise FastMoEError with the library's message if ``rc`` is not FMOE_OK."""
    if rc != OK:
        msg = lib().fmoe_last_error().decode(errors="replace")
        kind = {EINVAL: ValueError, ERANGE: OverflowError}.get(rc, FastMoEError)
        if kind is FastMoEError:
            raise FastMoEError(f"{what}: status {rc}: {msg}")
        raise kind(f"{what}: {msg}")


# Mirror of the library's kernel-variant options (fmoe_set_option), so that host code can read an
# option without a library call.  Filled on first read; kept in step by set_option().
_OPTS: dict[str, int] = {}


def option(name: str) -> int:
    """Current value of a kernel-variant option (see fmoe_set_option in the header)."""
    if name not in _OPTS:
        v = ctypes.c_int64()
        check(lib().fmoe_get_option(name.encode(), ctypes.byref(v)), "fmoe_get_option")
        _OPTS[name] = v.value
    return _OPTS[name]


def set_option(name: str, value: int) -> int:
    """Set a kernel-variant option; returns its previous value."""
    prev = ctypes.c_int64()
    check(lib().fmoe_set_option(name.encode(), int(value), ctypes.byref(prev)), "fmoe_set_option")
    _OPTS[name] = int(value)
    return prev.value


@contextlib.contextmanager
def options(**values):
    """Set kernel-variant options for the duration of a ``with`` block (e.g. ``plan=1``)."""
    prev = {}
    try:
        for k, v in values.items():
            prev[k] = set_option(k, v)
        yield
    finally:
        for k, v in prev.items():
            set_option(k, v)
