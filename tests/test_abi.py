"""The C-ABI libraries load and export every symbol include/dsv4_gpu.h
declares (CPU only: no compute calls)."""
import os
import re

import common

ROOT = common.ROOT


def header_symbols():
    text = open(os.path.join(ROOT, "include", "dsv4_gpu.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(dsv4_gpu_\w+)\s*\(", text))


def test_binding_covers_header():
    pkg = common.load_pkg()
    assert header_symbols() == set(pkg.SYMBOLS)


def test_hip_library_exports_every_symbol():
    pkg = common.load_pkg()
    L = pkg.lib()
    for name in header_symbols():
        assert hasattr(L, name), name


def test_stub_exports_every_symbol_and_reports_no_device():
    pkg = common.load_pkg()
    S = pkg.stub()
    for name in header_symbols():
        assert hasattr(S, name), name
    assert S.dsv4_gpu_available() == 0
    assert S.dsv4_gpu_init() == -1
    assert S.dsv4_gpu_has(None) == 0
    assert S.dsv4_gpu_free_vram() == 0
    assert S.dsv4_gpu_kv_create(4, 4, 0) is None


def test_struct_layout_matches_reference():
    """DSV4QMat is {ptr, ptr, int x5} = 36 bytes padded to 40 on LP64."""
    import ctypes
    pkg = common.load_pkg()
    assert ctypes.sizeof(pkg.DSV4QMat) == 40
    assert ctypes.sizeof(pkg.DSV4ExpertW) == 120
