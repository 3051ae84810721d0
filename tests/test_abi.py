"""The C-ABI library loads, exports exactly what include/fastmoe_amd.h declares, and rejects bad
arguments before touching the GPU (CPU only: no kernel is launched here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from fastmoe_amd import _abi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fastmoe_amd.h"


def _declared():
    text = HEADER.read_text()
    return set(re.findall(r"^FMOE_API\s+[\w\s\*]+?\b(fmoe_\w+)\s*\(", text, re.M))


def test_header_declares_the_binding_table():
    names = _declared()
    assert names == set(_abi.SIGNATURES), names ^ set(_abi.SIGNATURES)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _abi.lib()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.fmoe_abi_version() == _abi.ABI_VERSION


def test_no_other_symbols_exported():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", str(_abi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert {n for n in exported if n.startswith("fmoe_")} == _declared()
    assert not [n for n in exported if n.startswith("_ZN4fmoe")]


def test_plan_layout_functions():
    lib = _abi.lib()
    N, T = 32768, 4096
    total = lib.fmoe_plan_workspace_bytes(N, T)
    rp = lib.fmoe_plan_row_ptr_offset(N, T)
    rec = lib.fmoe_plan_records_offset(N, T)
    assert lib.fmoe_plan_status_offset() == 0
    assert rp % 256 == 0 and rec % 256 == 0
    assert rp >= 256 + 4 * (T + 1)
    assert rec >= rp + 4 * (T + 2) + 16 * N
    assert total >= rec + 16 * N
    assert lib.fmoe_plan_workspace_bytes(-1, T) < 0
    assert lib.fmoe_plan_workspace_bytes(N, 0) < 0


@pytest.mark.parametrize("case", ["zero_experts", "null_table", "negative_rows", "null_ptr_rows"])
def test_build_metadata_rejects_bad_arguments(case):
    lib = _abi.lib()
    ptrs = (ctypes.c_int64 * 2)(0x1000, 0x2000)
    rows = (ctypes.c_int64 * 2)(3, 4)
    dev = 0x10000  # never dereferenced: validation fails before any launch
    if case == "zero_experts":
        rc = lib.fmoe_build_metadata(ptrs, rows, 0, dev, dev, dev, dev, None)
    elif case == "null_table":
        rc = lib.fmoe_build_metadata(ptrs, rows, 2, None, dev, dev, dev, None)
    elif case == "negative_rows":
        rows[1] = -1
        rc = lib.fmoe_build_metadata(ptrs, rows, 2, dev, dev, dev, dev, None)
    else:
        ptrs[0] = 0
        rc = lib.fmoe_build_metadata(ptrs, rows, 2, dev, dev, dev, dev, None)
    assert rc == _abi.EINVAL
    assert lib.fmoe_last_error().decode()


def test_combine_entry_points_reject_bad_arguments():
    lib = _abi.lib()
    dev = 0x10000
    # bad mode
    rc = lib.fmoe_combine_fwd(7, dev, None, _abi.I64, None, _abi.F32, None, None, 1, 4, 4, 8,
                              _abi.F32, dev, _abi.F32, 8, 0, None, 0, None)
    assert rc == _abi.EINVAL and b"mode" in lib.fmoe_last_error()
    # det without plan
    rc = lib.fmoe_combine_fwd(_abi.MODE_DET, None, None, _abi.I64, None, _abi.F32, None, None, 1,
                              4, 4, 8, _abi.F32, dev, _abi.F32, 8, 0, None, 0, None)
    assert rc == _abi.EINVAL
    # out stride smaller than D
    rc = lib.fmoe_combine_fwd(_abi.MODE_DET, dev * 256, None, _abi.I64, None, _abi.F32, None, None,
                              1, 4, 4, 8, _abi.F32, dev, _abi.F32, 4, 0, None, 0, None)
    assert rc == _abi.EINVAL
    # too many rows for the 32-bit counters
    rc = lib.fmoe_combine_fwd(_abi.MODE_DET, dev * 256, None, _abi.I64, None, _abi.F32, None, None,
                              1, 1 << 31, 4, 8, _abi.F32, dev, _abi.F32, 8, 0, None, 0, None)
    assert rc == _abi.ERANGE
    # atomic mode with a 16-bit output: the fp32 accumulator workspace is required
    need = lib.fmoe_combine_fwd_workspace_bytes(_abi.MODE_ATOMIC, 4, 8, _abi.BF16)
    assert need == 256 and lib.fmoe_combine_fwd_workspace_bytes(_abi.MODE_DET, 4, 8, _abi.BF16) == 0
    assert lib.fmoe_combine_fwd_workspace_bytes(_abi.MODE_ATOMIC, 4, 8, _abi.F32) == 0
    assert lib.fmoe_combine_fwd_workspace_bytes(_abi.MODE_ATOMIC_PACKED, 4, 8, _abi.BF16) == 0
    for ws, nbytes in [(None, 0), (dev * 256, need - 4), (dev * 256 + 8, need)]:
        rc = lib.fmoe_combine_fwd(_abi.MODE_ATOMIC, None, dev, _abi.I64, dev, _abi.F32, dev, dev, 1,
                                  4, 4, 8, _abi.BF16, dev, _abi.BF16, 8, 0, ws, nbytes, None)
        assert rc == _abi.EINVAL and b"workspace" in lib.fmoe_last_error()
    # backward: grad_out dtype must equal the expert dtype
    rc = lib.fmoe_combine_bwd(dev * 256, 4, 4, 8, _abi.BF16, dev, _abi.F32, 8, dev, None,
                              _abi.F32, None)
    assert rc == _abi.EINVAL
    # plan: bad index dtype, unaligned workspace
    rc = lib.fmoe_build_plan(dev, _abi.F32, dev, _abi.F32, 4, 4, dev, dev, 1, 32, dev * 256, None)
    assert rc == _abi.EINVAL
    rc = lib.fmoe_build_plan(dev, _abi.I64, dev, _abi.F32, 4, 4, dev, dev, 1, 32, dev + 8, None)
    assert rc == _abi.EINVAL


def test_small_entry_points_reject_calls_beyond_their_limits():
    """fmoe_combine_fwd_small / _bwd_small check their limits on the host, before any launch."""
    lib = _abi.lib()
    dev = 0x10000
    limit = lib.fmoe_combine_small_max_rows()
    assert limit == 4096
    one = (ctypes.c_int64 * 1)(dev * 256)

    def fwd(rows, E=1, ptrs=one, status=dev, idt=_abi.I64, T=4):
        return lib.fmoe_combine_fwd_small(ptrs, rows, E, dev, idt, dev, _abi.F32, T, 8, _abi.F32,
                                          dev, _abi.F32, 8, 0, status, None)

    assert fwd((ctypes.c_int64 * 1)(limit + 1)) == _abi.ERANGE
    assert b"small path" in lib.fmoe_last_error()
    assert fwd((ctypes.c_int64 * 1)(-1)) == _abi.EINVAL
    assert fwd((ctypes.c_int64 * 1)(4), ptrs=(ctypes.c_int64 * 1)(0)) == _abi.EINVAL  # null rows
    assert fwd((ctypes.c_int64 * 1)(4), status=None) == _abi.EINVAL
    assert fwd((ctypes.c_int64 * 1)(4), idt=_abi.F32) == _abi.EINVAL
    assert fwd((ctypes.c_int64 * 1)(4), T=1 << 30) == _abi.ERANGE
    many = (ctypes.c_int64 * 257)(*([dev * 256] * 257))
    rows = (ctypes.c_int64 * 257)(*([1] * 257))
    assert fwd(rows, E=257, ptrs=many) == _abi.EINVAL
    rc = lib.fmoe_combine_bwd_small(many, rows, 257, dev, _abi.I64, dev, _abi.F32, 4, 8, _abi.F32,
                                    dev, _abi.F32, 8, dev, None, _abi.F32, None)
    assert rc == _abi.EINVAL and b"num_experts" in lib.fmoe_last_error()
    rc = lib.fmoe_combine_bwd_small(one, (ctypes.c_int64 * 1)(4), 1, dev, _abi.I64, dev, _abi.F32,
                                    4, 8, _abi.BF16, dev, _abi.F32, 8, dev, None, _abi.F32, None)
    assert rc == _abi.EINVAL and b"grad_out dtype" in lib.fmoe_last_error()


def test_metadata_and_plan_entry_points_reject_bad_arguments():
    """The one-call metadata + plan entry points check every argument on the host, including row
    totals that the kernel-argument table (32-bit offsets) cannot hold."""
    lib = _abi.lib()
    dev, ws = 0x10000, 0x10000 * 256
    ptrs = (ctypes.c_int64 * 2)(0x1000, 0x2000)

    def from_slots(rows, T, k):
        r = (ctypes.c_int64 * 2)(*rows)
        return lib.fmoe_build_metadata_and_plan_from_slots(ptrs, r, 2, dev, dev, dev, dev, dev, T,
                                                           k, dev, _abi.F32, 32, ws, None)

    # rows that each fit but sum to 2^31: not the T*k rows of the slot map
    assert from_slots([1 << 30, 1 << 30], 4, 2) == _abi.EINVAL
    assert b"slot" in lib.fmoe_last_error()
    assert from_slots([4, 4], 4, 65) == _abi.EINVAL            # top_k above 64
    assert from_slots([1 << 30, 1 << 30], 1 << 29, 4) == _abi.ERANGE   # T*k of 2^31
    assert from_slots([4, -1], 4, 2) == _abi.EINVAL

    def meta_plan(rows, idx_dtype=_abi.I64, p0=0x1000):
        r = (ctypes.c_int64 * 2)(*rows)
        pp = (ctypes.c_int64 * 2)(p0, 0x2000)
        return lib.fmoe_build_metadata_and_plan(pp, r, 2, dev, dev, dev, dev, dev, idx_dtype, dev,
                                                _abi.F32, 8, 32, ws, None)

    assert meta_plan([3, 4], p0=0) == _abi.EINVAL               # rows at a null address
    assert b"null address" in lib.fmoe_last_error()
    assert meta_plan([3, 4], idx_dtype=_abi.F32) == _abi.EINVAL  # float indices
    assert meta_plan([3, -4]) == _abi.EINVAL


def test_invert_scatter_index_rejects_bad_arguments():
    lib = _abi.lib()
    dev = 0x10000
    ws = dev * 256
    cases = {
        "num_rows": (dev, _abi.I64, -1, 4, dev, dev, ws),
        "num_tokens": (dev, _abi.I64, 4, 0, dev, dev, ws),
        "dtype": (dev, _abi.F32, 4, 4, dev, dev, ws),
        "null": (dev, _abi.I64, 4, 4, None, dev, ws),
        "aligned": (dev, _abi.I64, 4, 4, dev, dev, ws + 8),
    }
    for word, args in cases.items():
        rc = lib.fmoe_invert_scatter_index(*args, None)
        assert rc == _abi.EINVAL and word.encode() in lib.fmoe_last_error(), word
    rc = lib.fmoe_invert_scatter_index(dev, _abi.I64, 1 << 31, 4, dev, dev, ws, None)
    assert rc == _abi.ERANGE


def test_check_raises_with_library_message():
    lib = _abi.lib()
    rc = lib.fmoe_build_metadata(None, None, 0, None, None, None, None, None)
    with pytest.raises(ValueError, match="num_experts"):
        _abi.check(rc, "fmoe_build_metadata")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_abi, "_LIB", None)
    monkeypatch.setenv("FASTMOE_AMD_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(_abi.FastMoEError, match="no non-HIP fallback"):
        _abi.lib()
    monkeypatch.setattr(_abi, "_LIB", None)


def test_library_missing_a_symbol_fails_loudly(monkeypatch, tmp_path):
    """A library built from other sources (here: one exporting only the version) is refused with
    FastMoEError naming the missing entry point, not an AttributeError from ctypes."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "stub.c"
    src.write_text("int fmoe_abi_version(void) { return %d; }\n" % _abi.ABI_VERSION)
    so = tmp_path / "libstub.so"
    subprocess.run([cc, "-shared", "-fPIC", str(src), "-o", str(so)], check=True)
    monkeypatch.setattr(_abi, "_LIB", None)
    monkeypatch.setenv("FASTMOE_AMD_LIB", str(so))
    with pytest.raises(_abi.FastMoEError, match="does not export fmoe_last_error"):
        _abi.lib()
    monkeypatch.setattr(_abi, "_LIB", None)


def _documented_options():
    """Option names listed in the header's comment on fmoe_set_option (``"name" [FMOE_ENV]``
    entries, or the names of a shared line)."""
    text = HEADER.read_text()
    block = text[text.index("Kernel-variant options"): text.index("FMOE_API int fmoe_set_option")]
    return set(re.findall(r'"(\w+)"', block))


def test_every_documented_option_reads_and_sets():
    names = _documented_options()
    assert {"plan", "small", "fwd_atomic_order", "fwd_atomic_tile"} <= names
    for name in sorted(names):
        v = ctypes.c_int64(-99)
        assert _abi.lib().fmoe_get_option(name.encode(), ctypes.byref(v)) == _abi.OK, name
        prev = _abi.set_option(name, v.value + 1)
        assert prev == v.value and _abi.option(name) == v.value + 1
        _abi.set_option(name, prev)
    v = ctypes.c_int64(0)
    assert _abi.lib().fmoe_get_option(b"no_such_option", ctypes.byref(v)) == _abi.EINVAL


@pytest.mark.parametrize("N,T,auto", [(32768, 4096, 3), (49152, 8192, 3), (131072, 16384, 4),
                                      (131072, 1, 1), (131072, 100, 1), (4194304, 131071, 4),
                                      (2097152, 1048576, 1), (4194305, 131071, 1)])
def test_plan_path_reports_the_builder_taken(N, T, auto):
    """fmoe_plan_path: the automatic choice by N and T (one launch below 2^16 rows, ranged up to
    2^22 rows and 2^19 tokens, radix beyond and for tokens averaging 64 rows or more; never the
    bucketed plan), a forced path where its limits hold, and the automatic choice where they do
    not."""
    lib = _abi.lib()
    with _abi.options(plan=0):
        assert lib.fmoe_plan_path(N, T, 256) == auto
    for forced in (1, 2, 3, 4):
        with _abi.options(plan=forced):
            got = lib.fmoe_plan_path(N, T, 256)
        assert got in (forced, auto)
    with _abi.options(plan=3):
        assert lib.fmoe_plan_path(2097152, 1048576, 256) == 1  # beyond the one-launch limits
    assert lib.fmoe_plan_path(-1, 4, 1) == -1 and lib.fmoe_plan_path(4, 0, 1) == -1
