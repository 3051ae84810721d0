"""Build the gfx950 C-ABI library ``fastmoe_amd/libfastmoe_amd.so`` in-tree.

Every HIP translation unit is compiled with hipcc for gfx950 only, in parallel, then linked into
one shared library that ``fastmoe_amd._abi`` loads with ctypes.  Usage::

    python -m fastmoe_amd.build          # or: from fastmoe_amd.build import build; build()
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD_DIR = PKG / "_build"
LIB_NAME = "libfastmoe_amd.so"
LIB_PATH = PKG / LIB_NAME

# The operator layer's host helper module (fastmoe_amd._host, a CPython extension built against
# the installed torch): it reads tensor properties in C++, and is not part of the C ABI.
HOST_EXT_SOURCE = "host_ext.cpp"

HIP_SOURCES = ["metadata.hip", "plan.hip", "plan_bucket.hip", "plan_radix.hip", "combine_fwd.hip",
               "combine_bwd.hip", "permute.hip", "noalloc.hip"]
HOST_SOURCES = ["abi.cpp"]

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # The forward adds rounded fp32 products in a fixed order (bit parity with index_add_).
    "-ffp-contract=off",
    # Hardware float atomics (global_atomic_add_f32 / pk_add_bf16) on coarse-grained memory.
    "-munsafe-fp-atomics",
    # No packed-fp32 instructions anywhere in the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall"]


def source_hash() -> str:
    """sha256 (hex, 16 digits) of every source the library is built from: the HIP and host
    translation units, their headers and the C ABI header (not the Python helper module).  Measurements kept in profiles/ record
    it, so a reader (bench.py) can tell whether they describe the current kernels."""
    import hashlib

    h = hashlib.sha256()
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h"))
    files += [CSRC / s for s in HOST_SOURCES]
    files.append(PKG.parent / "include" / "fastmoe_amd.h")
    for f in files:
        h.update(f.name.encode())
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln
    )  # hipcc's host pass does not know the device feature; that warning is noise
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _host_ext_command(cxx: str):
    """g++ command of the host helper module: (command, temporary output, final path)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    path = PKG / ("_host" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = path.with_name(path.name + ".tmp")
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"]]
    libdirs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [cxx, *CXX_FLAGS, "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", str(CSRC / HOST_EXT_SOURCE),
           "-o", str(tmp), *[f"-I{i}" for i in incs], *[f"-L{d}" for d in libdirs],
           *[f"-Wl,-rpath,{d}" for d in libdirs], "-lc10", "-ltorch", "-ltorch_python"]
    return cmd, tmp, path


def build(verbose: bool = True, jobs: int | None = None, defines: list[str] | None = None,
          out: Path | None = None, build_dir: Path | None = None) -> Path:
    """Compile every translation unit and link ``libfastmoe_amd.so``; returns its path.  The
    in-tree build also compiles the host helper module ``fastmoe_amd._host``.

    ``defines`` (e.g. ``["FMOE_BWD_WAVES=8"]``) set the kernels' compile-time knobs; ``out`` and
    ``build_dir`` redirect the result (tuning builds), by default the in-tree library.
    """
    bdir = build_dir or BUILD_DIR
    lib_path = out or LIB_PATH
    bdir.mkdir(parents=True, exist_ok=True)
    dflags = [f"-D{d}" for d in (defines or [])]
    hipcc = _hipcc()
    cxx = shutil.which("g++") or "c++"
    cmds: list[list[str]] = []
    objs: list[str] = []
    for src in HIP_SOURCES:
        obj = bdir / (src + ".o")
        cmds.append([hipcc, *HIPCC_FLAGS, *dflags, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    for src in HOST_SOURCES:
        obj = bdir / (src + ".o")
        cmds.append([cxx, *CXX_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
    ext_cmd, ext_tmp, ext_path = (None, None, None) if out else _host_ext_command(cxx)
    if ext_cmd:
        cmds.append(ext_cmd)
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    if ext_cmd:
        os.replace(ext_tmp, ext_path)
    tmp = lib_path.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)])
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path}", file=sys.stderr)
    return lib_path


if __name__ == "__main__":
    build()
