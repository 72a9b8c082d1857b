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


def test_ctypes_layouts_match_the_c_header(tmp_path):
    """The binding's mirrors of the header's structs have the C sizes and
    field offsets (compiled with gcc against include/dsv4_gpu.h)."""
    import ctypes
    import shutil
    import subprocess
    import pytest
    if not shutil.which("gcc"):
        pytest.skip("gcc not available")
    pkg = common.load_pkg()
    src = tmp_path / "l.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "dsv4_gpu.h"\n'
        'int main(void){printf("%zu %zu %zu %zu %zu %zu %zu %zu\\n",'
        'sizeof(dsv4_gpu_attn_cfg), sizeof(dsv4_gpu_attn_w), sizeof(dsv4_gpu_ckpt_dims),'
        'sizeof(dsv4_gpu_layer_mats), sizeof(dsv4_gpu_ckpt_stats),'
        'offsetof(dsv4_gpu_layer_mats, gate), offsetof(dsv4_gpu_ckpt_stats, bytes),'
        'offsetof(dsv4_gpu_ckpt_dims, has_indexer));return 0;}\n')
    exe = tmp_path / "l"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    want = [ctypes.sizeof(pkg.AttnCfg), ctypes.sizeof(pkg.AttnW), ctypes.sizeof(pkg.CkptDims),
            ctypes.sizeof(pkg.LayerMats), ctypes.sizeof(pkg.CkptStats),
            pkg.LayerMats.gate.offset, pkg.CkptStats.bytes.offset,
            pkg.CkptDims.has_indexer.offset]
    assert got == want
