"""Host-side checks of the dispatch permutation and MoE layer API (CPU only, no kernel launch)."""
from __future__ import annotations

import ctypes

import pytest
import torch

import fastmoe_amd
from fastmoe_amd import _abi
from fastmoe_amd.consts import MoEImplementation


def test_cpu_tensors_raise():
    x = torch.randn(4, 8)
    ids = torch.zeros(4, 2, dtype=torch.long)
    w = torch.ones(4, 2)
    with pytest.raises(RuntimeError, match="only on the GPU"):
        fastmoe_amd.permute_tokens(x, ids, w, 2)
    layer = fastmoe_amd.MoEFeedForward(8, 16, 2, 1)
    with pytest.raises(RuntimeError, match="only on the GPU"):
        layer(torch.randn(1, 4, 8))


def test_workspace_size():
    lib = _abi.lib()
    n = lib.fmoe_permute_workspace_bytes(32768, 256)
    nb = 32768 // 1024  # 1024-slot ranking blocks while E <= 1024
    assert n >= nb * 257 * 4 + 32768 * 4 + 257 * 4 and n % 256 == 0
    n = lib.fmoe_permute_workspace_bytes(32768, 3000)
    nb = 32768 // 256  # 256-slot blocks beyond
    assert n >= nb * 3001 * 4 + 32768 * 4 + 3001 * 4 and n % 256 == 0
    assert lib.fmoe_permute_workspace_bytes(-1, 4) < 0
    assert lib.fmoe_permute_workspace_bytes(10, 0) < 0


@pytest.mark.parametrize("case", ["no_experts", "too_many_experts", "bad_k", "bad_id_dtype",
                                  "bad_gate_dtype", "null_out", "misaligned_ws", "huge"])
def test_permute_build_rejects_bad_arguments(case):
    lib = _abi.lib()
    buf = ctypes.create_string_buffer(4096)
    ws = (ctypes.addressof(buf) + 255) // 256 * 256
    args = dict(ids=ws, idt=_abi.I64, g=ws, gdt=_abi.F32, T=4, k=2, E=4, counts=ws, offs=ws,
                rev=ws, sg=ws, pos=ws, status=ws, ws=ws)
    upd = {"no_experts": {"E": 0}, "too_many_experts": {"E": 5000}, "bad_k": {"k": 0},
           "bad_id_dtype": {"idt": _abi.F32}, "bad_gate_dtype": {"gdt": _abi.I64},
           "null_out": {"rev": None}, "misaligned_ws": {"ws": ws + 4},
           "huge": {"T": 1 << 30, "k": 8}}[case]
    args.update(upd)
    rc = lib.fmoe_permute_build(*args.values(), None)
    assert rc in (_abi.EINVAL, _abi.ERANGE), rc
    assert lib.fmoe_last_error()


def test_gather_and_gate_grad_reject_bad_arguments():
    lib = _abi.lib()
    assert lib.fmoe_permute_gather(None, 4, 2, 0, None, 0, None, None) == _abi.EINVAL
    assert lib.fmoe_permute_gather(None, 4, 2, 16, None, 16, None, None) == _abi.EINVAL
    assert lib.fmoe_permute_gather(None, 4, 2, 15, 8, 16, 8, None) == _abi.EINVAL  # odd row bytes
    assert lib.fmoe_permute_gate_grad(None, 4, None, _abi.I64, None, None) == _abi.EINVAL
    assert lib.fmoe_permute_gate_grad(None, 0, None, _abi.F32, None, None) == _abi.OK


def test_implementation_selector():
    assert MoEImplementation("fast") is MoEImplementation.FAST
    assert fastmoe_amd.MoEFeedForward(8, 16, 2, 1, "standard").implementation == "standard"
