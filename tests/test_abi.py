"""The C-ABI library (CPU, no GPU calls): it loads, exports every entry point include/kv800_hip.h declares, the Python
binding's signature table covers exactly those, and host-side argument checks reject bad input before any launch."""
import ctypes
import os
import re
import subprocess

import pytest

import lfm3_kv800_amd.kv800_hip as kh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kv800_hip.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(kv800_hip_\w+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.isfile(kh.LIB):
        pytest.fail(f"{kh.LIB} not built: run __graft_entry__.build()")
    return kh.load_library()


def test_header_symbols_exported(lib):
    names = declared()
    assert len(names) >= 14
    out = subprocess.run(["nm", "-D", "--defined-only", kh.LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (kv800_hip_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        getattr(lib, n)


def test_binding_covers_header():
    assert sorted(kh.SIGNATURES) == declared()


def test_host_checks_reject_bad_arguments(lib):
    # rejected on the host: no device memory is touched
    assert lib.kv800_hip_quantize_blocks(None, None, -1, None, None) == -1
    assert b"M" in lib.kv800_hip_last_error()
    assert lib.kv800_hip_quantize_blocks(None, None, 2, None, None) == -1
    assert lib.kv800_hip_flush(None, None, 0, 0, 0, 0, 0, None, None, 0, 256, 1, None, None, 1, 1, None) == -1
    assert lib.kv800_hip_decode_merge(None, None, None, 1, 0, None, None) == -1
    assert lib.kv800_hip_quantize_blocks(None, None, 0, None, None) == 0        # empty: a no-op


def test_plan(lib):
    ns, spb = ctypes.c_int64(), ctypes.c_int64()
    assert lib.kv800_hip_plan(64, 127, ctypes.byref(ns), ctypes.byref(spb)) == 0
    assert (ns.value, spb.value) == (8, 16)
    assert lib.kv800_hip_plan(2, 19, ctypes.byref(ns), ctypes.byref(spb)) == 0
    assert ns.value * spb.value >= 19 and (ns.value - 1) * spb.value < 19
    assert lib.kv800_hip_plan(4, 0, ctypes.byref(ns), ctypes.byref(spb)) == 0 and ns.value == 0
    assert lib.kv800_hip_decode_workspace(64, 8, 0) >= 64 * 9 * 16 * 4 * 2 + 64 * 9 * 16 * 128 * 4


def test_model_header_symbols_exported_and_bound(lib):
    """include/lfm3_model.h (the engine loop's fused kernels): every declared entry point is exported by the same
    library and bound by lfm3_kv800_amd.model_ops."""
    import lfm3_kv800_amd.model_ops as mo
    src = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "lfm3_model.h")).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(lfm3_hip_\w+)\s*\(", src)))
    assert len(names) == 8
    out = subprocess.run(["nm", "-D", "--defined-only", kh.LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (lfm3_hip_\w+)", out))
    assert not [n for n in names if n not in exported]
    assert sorted(mo.SIGNATURES) == names
    for name in ("lfm3_hip_silu_mul", "lfm3_hip_argmax", "lfm3_hip_shuffle_weight", "lfm3_hip_linear"):
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = mo.SIGNATURES[name]
    assert lib.lfm3_hip_silu_mul(None, 1, 7, None, None) == -1          # F not a multiple of 8: rejected on the host
    assert lib.lfm3_hip_argmax(None, 1, 12, 12, None, None) == -1       # V not a multiple of 8
    assert lib.lfm3_hip_argmax(None, 1, 16, 8, None, None) == -1        # row stride below V
    assert lib.lfm3_hip_shuffle_weight(None, 100, 96, 128, None, None) == -1           # K not a multiple of 64
    assert lib.lfm3_hip_shuffle_weight(None, 200, 128, 128, None, None) == -1          # Npad below N
    assert lib.lfm3_hip_linear(None, 128, None, 4, 100, 128, None, 104, 1, None, 0, None) == -1   # Npad % 128
    assert lib.lfm3_hip_linear(None, 128, None, 4, 128, 128, None, 128, 3, None, 0, None) == -1   # split of K
    assert lib.lfm3_hip_linear(None, 128, None, 4, 128, 128, None, 128, 2, None, 0, None) == -1   # no workspace
    assert lib.lfm3_hip_linear(None, 128, None, 4, 128, 128, None, 64, 2, None, 1, None) == -1    # glu with split
