"""CPU checks of the drop-in boundary: the library builds for gfx950, loads,
and exports every symbol include/laplace_hip.h declares (no compute calls:
there is no GPU here)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "laplace_hip.h")
LIB = os.path.join(ROOT, "laplace_amd", "liblaplace_hip.so")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(lp_[a-z0-9_]+)\s*\(", text))
    return sorted(n for n in names if not n.endswith("_fn"))


def test_header_declares_entry_points():
    names = declared_symbols()
    for must in ("lp_gemm", "lp_moe_gemv", "lp_moe_gemv_multi", "lp_register_weights",
                 "lp_quantize_act", "lp_gemm_dev", "lp_block_sums_dev"):
        assert must in names


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built (python -m laplace_amd.build)")
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (lp_[a-z0-9_]+)", out))
    missing = [n for n in declared_symbols() if n not in exported]
    assert not missing, missing


def test_library_loads_and_binds_without_gpu():
    from laplace_amd import _lib
    L = _lib.lib()
    for n in declared_symbols():
        assert hasattr(L, n), n
    # pure host queries are safe without a device
    assert L.lp_act_workspace_bytes(1, 4096) >= 4096 + 3 * 128 * 4


def test_code_object_targets_gfx950_only():
    """The fat binary embedded in our own library names gfx950 and no other
    GPU target."""
    data = open(LIB, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}, targets
