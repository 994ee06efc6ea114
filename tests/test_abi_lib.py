"""The C-ABI library and the pybind11 module load on a CPU-only host and export
everything include/qwen_megakernel.h declares (no compute calls here)."""

import ctypes
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "qwen0.6b_amd", "libqwen_megakernel.so")
HEADER = os.path.join(REPO, "include", "qwen_megakernel.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^int\s+(\w+)\s*\(", text, flags=re.M)))


def test_header_declares_reference_entry_points():
    names = _declared()
    for ref in ("launch_ldg_decode_direct", "launch_ldg_generate_nosync", "launch_ldg_decode_persistent"):
        assert ref in names
    assert len(names) >= 8


def test_library_exports_every_declared_symbol():
    if not os.path.exists(LIB):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB)
    for name in _declared():
        assert hasattr(lib, name), f"{name} not exported"
    lib.qwen_abi_version.restype = ctypes.c_int
    assert lib.qwen_abi_version() == 2
    # exported with C linkage (unmangled) and as dynamic symbols
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True).stdout
    for name in _declared():
        assert re.search(rf"\bT {name}$", out, flags=re.M), name


def test_layout_checker_passes():
    exe = os.path.join(REPO, "qwen0.6b_amd", "layout_check")
    if not os.path.exists(exe):
        pytest.skip("layout checker not built")
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_pybind_module_surface():
    try:
        import qwen_megakernel_C as m
    except ImportError:
        pytest.skip("extension not built")
    assert m.abi_version() == 2
    for op in ("decode", "generate_nosync", "abi_version", "built_torch_version", "generate_ex",
               "lm_head_argmax", "mlp_block", "last_error", "generate_until", "prefill", "prefill_timestamps",
               "sample", "generate_sampled", "set_trace", "set_wait_deadline_us"):
        assert hasattr(m, op), op
    import torch

    assert m.built_torch_version().split("+")[0] == torch.__version__.split("+")[0]
