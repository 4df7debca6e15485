"""CPU checks of the C-ABI boundary: the library builds, loads without a GPU and
exports every symbol declared in include/rte_hip.h with a binding in _lib.py."""

from __future__ import annotations

import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _declared() -> list[str]:
    text = (ROOT / "include" / "rte_hip.h").read_text()
    return sorted(set(re.findall(r"\b(rte_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from rte_amd import _lib

    assert sorted(_lib.SIGNATURES) == _declared()


def test_library_loads_and_exports_every_symbol():
    from rte_amd import _lib

    lib = _lib.load()  # dlopen only; no device call
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.rte_abi_version() == 1
    # pure host helpers work without a device
    assert lib.rte_pack_workspace_bytes(65536, 64) == 64 * 256 * 4
    assert lib.rte_rmsnorm_bwd_workspace_bytes(8192, 512) == 1024 * 512 * 4  # 8-row blocks (d <= 512)
    assert lib.rte_rmsnorm_bwd_workspace_bytes(8192, 1024) == 256 * 1024 * 4  # 32-row blocks


def test_ops_fail_loudly_without_device():
    import pytest
    import torch

    from rte_amd import _lib
    from rte_amd.kernels import hip_ops

    if _lib.device_ready():
        pytest.skip("a ROCm device is present")
    with pytest.raises(RuntimeError, match="HIP backend is required"):
        hip_ops.route_topk(torch.zeros(4, 8), 2)
