"""The C-ABI library (CPU only, no kernel launches): it loads, exports every entry point the header
declares, its argument structs match the header's layout, and bad arguments fail on the host."""
from __future__ import annotations

import ctypes
import re
import subprocess

import pytest

from rsna_knee_efficiency_amd import hip


def declared() -> list[str]:
    text = hip.HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(d8s_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = hip.library()
    names = declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    assert set(hip.SIGNATURES) | set(hip.STRING_FUNCS) == set(names)


def test_version_is_this_source():
    v = hip.version()
    assert v.startswith("d8s-hip 1 ") and v.endswith(" gfx950")
    assert hip.built_sha() == hip.source_sha(), "libd8s_hip.so is stale: run __graft_entry__.build()"


def test_struct_layouts_match_header(tmp_path):
    prog = tmp_path / "layout.c"
    prog.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "d8s_hip.h"\n'
        "int main(void) {\n"
        '  printf("%zu %zu %zu %zu\\n", sizeof(D8sGemmArgs), offsetof(D8sGemmArgs, wsum),'
        " offsetof(D8sGemmArgs, out), offsetof(D8sGemmArgs, G0n));\n"
        '  printf("%zu %zu %zu\\n", sizeof(D8sConv2Args), offsetof(D8sConv2Args, out),'
        " offsetof(D8sConv2Args, W));\n"
        '  printf("%zu %zu %zu\\n", sizeof(D8sStemArgs), offsetof(D8sStemArgs, out),'
        " offsetof(D8sStemArgs, flip));\n"
        '  printf("%zu %zu %zu %zu\\n", sizeof(D8sDenseArgs), offsetof(D8sDenseArgs, w2),'
        " offsetof(D8sDenseArgs, out), offsetof(D8sDenseArgs, W));\n"
        '  printf("%zu %zu %zu %zu\\n", sizeof(D8sBlockArgs), offsetof(D8sBlockArgs, layers),'
        " offsetof(D8sBlockArgs, L), sizeof(D8sLayerP));\n"
        "  return 0; }\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", f"-I{hip.HEADER.parent}", str(prog), "-o", str(exe)], check=True)
    got = [list(map(int, line.split())) for line in
           subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines()]
    G, C, S = hip.GemmArgs, hip.Conv2Args, hip.StemArgs
    assert got[0] == [ctypes.sizeof(G), G.wsum.offset, G.out.offset, G.G0n.offset]
    assert got[1] == [ctypes.sizeof(C), C.out.offset, C.W.offset]
    assert got[2] == [ctypes.sizeof(S), S.out.offset, S.flip.offset]
    D = hip.DenseArgs
    assert got[3] == [ctypes.sizeof(D), D.w2.offset, D.out.offset, D.W.offset]
    B = hip.BlockArgs
    assert got[4] == [ctypes.sizeof(B), B.layers.offset, B.L.offset, ctypes.sizeof(hip.LayerP)]


@pytest.mark.parametrize("name,args", [
    ("d8s_conv1", lambda: (None, None)),
    ("d8s_conv1_acc32", lambda: (ctypes.byref(hip.GemmArgs()), None, None)),
    ("d8s_transition", lambda: (ctypes.byref(hip.GemmArgs(1, 1, 1, 1, 1, 1, 1, 2, 3, 1, 16, 4, 16,
                                                          48, 1)), None)),
    ("d8s_conv2", lambda: (ctypes.byref(hip.Conv2Args(1, 1, 1, 1, 1, 0, 4, 4, 0)), None)),
    ("d8s_dense", lambda: (None, None)),
    ("d8s_dense_block", lambda: (None, None)),
    ("d8s_dense_block", lambda: (ctypes.byref(hip.BlockArgs(1, 1, 1, 2, 32, 32, 4, 3, 0)), None)),
    ("d8s_dense_block", lambda: (ctypes.byref(hip.BlockArgs(1, 1, 1, 2, 16, 16, 60, 8, 0)), None)),
    ("d8s_dense", lambda: (ctypes.byref(hip.DenseArgs(1, 0, 1, 1, 1, 1, 1, 1, 1, 1, 2, 3, 1, 8, 8, 0)),
                           None)),
    ("d8s_dense", lambda: (ctypes.byref(hip.DenseArgs(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 2, 600, 1, 8, 8,
                                                      0)), None)),
    ("d8s_stem", lambda: (ctypes.byref(hip.StemArgs(1, 0, 1, 1, 1, 1, 1, 8, 8, 1, 0, 0)), None)),
    ("d8s_stem", lambda: (ctypes.byref(hip.StemArgs(1, 1, 1, 1, 1, 1, 3, 8, 8, 1, 2, 0)), None)),
    ("d8s_stem", lambda: (ctypes.byref(hip.StemArgs(1, 1, 1, 1, 1, 1, 2, 8, 8, 1, 0, 0)), None)),
    ("d8s_stem", lambda: (ctypes.byref(hip.StemArgs(4, 0, 1, 1, 1, 1, 1, 8, 8, 0, 0, 0)), None)),
    ("d8s_final", lambda: (1, 20, 1, 2, 256, 1, 1, 100, None)),
    ("d8s_micro_copy", lambda: (1, 1, 17, None)),
])
def test_invalid_arguments_fail_on_the_host(name, args):
    """Every one of these is rejected before any HIP call (so it is safe without a GPU)."""
    lib = hip.library()
    rc = getattr(lib, name)(*args())
    assert rc == 1
    assert lib.d8s_last_error().decode().startswith(name)
    with pytest.raises(hip.D8sError, match=name):
        hip.call(name, *args())


def test_no_fallback_when_library_is_missing(tmp_path, monkeypatch):
    monkeypatch.setattr(hip, "_STATE", {})
    with pytest.raises(FileNotFoundError):
        hip.library(tmp_path / "libd8s_hip.so")
