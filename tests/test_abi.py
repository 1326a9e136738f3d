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


def test_stale_library_is_refused(tmp_path):
    """A library whose compiled-in source hash is not the tree's is refused at load (StaleLibrary);
    one with the tree's hash is accepted.  Stub libraries exporting only d8s_version stand in for
    builds from other sources."""
    def stub(tag: str):
        src = tmp_path / f"v_{tag}.c"
        src.write_text(f'const char* d8s_version(void) {{ return "d8s-hip 1 {tag} gfx950"; }}\n')
        so = tmp_path / f"libv_{tag}.so"
        subprocess.run(["gcc", "-shared", "-fPIC", str(src), "-o", str(so)], check=True)
        return ctypes.CDLL(str(so)), so
    lib, so = stub("0123456789ab")
    with pytest.raises(hip.StaleLibrary, match="0123456789ab"):
        hip.check_fresh(lib, so)
    lib, so = stub(hip.source_sha())
    assert hip.check_fresh(lib, so) == hip.source_sha()


def test_parts_supported_matches_the_launch():
    """d8s_parts_supported (what the runner's band options come from) and the launcher agree: a shape
    it refuses fails on the host with hipErrorInvalidValue, at the LDS limit (the 32 x 32 block with
    64 groups fits 256-pixel bands; the 128-wide map with 2-row bands does not)."""
    lib = hip.library()
    assert lib.d8s_parts_supported(32, 32, 64, 4) == 1
    assert lib.d8s_parts_supported(128, 128, 7, 64) == 0          # 256 px bands of a 128-wide map
    assert lib.d8s_parts_supported(128, 128, 7, 128) == 1
    assert lib.d8s_parts_supported(16, 16, 65, 8) == 0            # more than 64 groups
    assert lib.d8s_parts_supported(16, 16, 51, 3) == 0            # H not a multiple of parts
    lay = (hip.LayerP * 1)()
    buf = (ctypes.c_uint8 * 64)()
    args = hip.PartsArgs(ctypes.addressof(buf), ctypes.addressof(buf), ctypes.addressof(lay),
                         ctypes.addressof(buf), ctypes.addressof(buf), 1, 128, 128, 2, 6, 64)
    assert lib.d8s_dense_block_parts(ctypes.byref(args), None) == 1
    assert "LDS" in lib.d8s_last_error().decode()


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
        '  printf("%zu %zu %zu %zu\\n", sizeof(D8sPrepStack), offsetof(D8sPrepStack, K),'
        " offsetof(D8sPrepStack, r2), offsetof(D8sPrepStack, g1));\n"
        '  printf("%zu %zu %zu %zu\\n", sizeof(D8sPrepArgs), offsetof(D8sPrepArgs, kind),'
        " offsetof(D8sPrepArgs, s), sizeof(D8sPrepStat));\n"
        '  printf("%zu %zu %zu\\n", sizeof(D8sGridArgs), offsetof(D8sGridArgs, kind),'
        " offsetof(D8sGridArgs, M));\n"
        '  printf("%zu %zu %zu\\n", sizeof(D8sHeadArgs), offsetof(D8sHeadArgs, logits),'
        " offsetof(D8sHeadArgs, ctx_layers));\n"
        '  printf("%zu %zu %zu %zu %d %llu\\n", sizeof(D8sPartsArgs), offsetof(D8sPartsArgs, sync),'
        " offsetof(D8sPartsArgs, xchg), offsetof(D8sPartsArgs, parts), D8S_PARTS_SYNC_WORDS(7),"
        " (unsigned long long)D8S_PARTS_XCHG_BYTES(7, 16));\n"
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
    PS, PA = hip.PrepStack, hip.PrepArgs
    assert got[5] == [ctypes.sizeof(PS), PS.K.offset, PS.r2.offset, PS.g1.offset]
    assert got[6] == [ctypes.sizeof(PA), PA.kind.offset, PA.s.offset, ctypes.sizeof(hip.PrepStat)]
    GA = hip.GridArgs
    assert got[7] == [ctypes.sizeof(GA), GA.kind.offset, GA.M.offset]
    HA = hip.HeadArgs
    assert got[8] == [ctypes.sizeof(HA), HA.logits.offset, HA.ctx_layers.offset]
    PP = hip.PartsArgs
    assert got[9] == [ctypes.sizeof(PP), PP.sync.offset, PP.xchg.offset, PP.parts.offset,
                      hip.parts_sync_words(7), hip.parts_xchg_bytes(7, 16)]


def _prep_args(kind=0, ws_bytes=None, box=(0, 64, 0, 64), r2=None, k=(0, 1), hr=64, out=256,
               scratch_bytes=1 << 40):
    """A d8s_prep argument set that is valid except for the field a test changes (fake pointers: the
    checks run before any HIP call)."""
    a = hip.PrepArgs()
    need = ctypes.c_uint64()
    assert hip.library().d8s_prep_workspace(1, 64, ctypes.byref(need)) == 0
    a.workspace, a.ws_bytes = 1 << 20, need.value if ws_bytes is None else ws_bytes
    a.scratch, a.scratch_bytes = 1 << 24, scratch_bytes
    a.kind, a.img, a.n_stacks = kind, 64, 1
    s = a.s[0]
    s.src, s.out, s.K, s.hr, s.wr = 4096, out, 1, hr, 64
    s.y0, s.y1, s.x0, s.x1 = box
    s.k0, s.k1 = k
    k1, k2, g1, g2 = (40, 4054, 0.95, 0.05)
    s.r1, s.r2, s.g1, s.g2 = k1, k2 if r2 is None else r2, g1, g2
    return a


def _head_args(**kw):
    """d8s_head arguments valid except for the fields given (fake pointers: checked before any HIP
    call)."""
    a = hip.HeadArgs()
    for n in ("z", "slot_of", "slot_mask", "logits", "workspace", *hip.HEAD_WEIGHTS):
        setattr(a, n, 4096)
    a.B, a.W, a.D, a.S, a.CD, a.heads, a.FF, a.PER, a.T, a.ctx_layers = 1, 88, 1664, 8, 256, 4, 512, 11, 12, 1
    need = ctypes.c_uint64()
    assert hip.library().d8s_head_workspace(ctypes.byref(a), ctypes.byref(need)) == 0
    a.ws_bytes = need.value
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_prep_workspace_size():
    b1, b16 = ctypes.c_uint64(), ctypes.c_uint64()
    lib = hip.library()
    assert lib.d8s_prep_workspace(1, 512, ctypes.byref(b1)) == 0
    assert lib.d8s_prep_workspace(16, 512, ctypes.byref(b16)) == 0
    assert b16.value > b1.value > 16 * ctypes.sizeof(hip.PrepStat)
    # the stats header, then one block per stack
    assert b16.value - b1.value == 15 * (b1.value - 1024)


def _chain_args(W=32, G=10, out2=None, out1=1 << 30):
    """d8s_conv2_conv1 arguments of two 32 x 32 images (G0 8) with one field changed."""
    H, N, G0, seg = 1024 // W if W else 32, 2, 8, 4096
    rows = N * H * W
    out2 = seg + (G - 1 - G0) * rows * 32 if out2 is None else out2
    c2 = hip.Conv2Args(1 << 20, 1, 1, 1, out2, N, H, W, 0)
    c1 = hip.GemmArgs(1, seg, 1, 1, 1, 1, out1, G0, G, N, H * W, W, rows, 128, 0)
    return ctypes.byref(c2), ctypes.byref(c1), None


@pytest.mark.parametrize("H,W,G", [(64, 64, 5), (32, 32, 39), (16, 16, 64), (12, 12, 8), (32, 48, 8),
                                   (32, 128, 8), (32, 32, 65), (32, 32, 1), (8, 16, 2)])
def test_chain_supported_shapes(H, W, G):
    """The shapes d8s_conv2_conv1 takes: W in {16, 32, 64}, H W a multiple of 128, 2 <= G <= 64."""
    want = W in (16, 32, 64) and (H * W) % 128 == 0 and 2 <= G <= 64
    assert hip.library().d8s_c21_supported(H, W, G) == int(want)


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
    ("d8s_prep_workspace", lambda: (0, 512, ctypes.byref(ctypes.c_uint64()))),
    ("d8s_prep_workspace", lambda: (4, 500, ctypes.byref(ctypes.c_uint64()))),
    ("d8s_prep", lambda: (None, None)),
    ("d8s_prep", lambda: (ctypes.byref(_prep_args(kind=2)), None)),
    ("d8s_prep", lambda: (ctypes.byref(_prep_args(ws_bytes=1024)), None)),
    ("d8s_prep", lambda: (ctypes.byref(_prep_args(scratch_bytes=64 * 64 * 4 - 4)), None)),
    ("d8s_prep", lambda: (ctypes.byref(_prep_args(box=(0, 65, 0, 64))), None)),
    ("d8s_prep", lambda: (ctypes.byref(_prep_args(r2=64 * 64 - 1)), None)),
    ("d8s_prep", lambda: (ctypes.byref(_prep_args(k=(1, 1))), None)),
    ("d8s_prep", lambda: (ctypes.byref(_prep_args(box=(0, 64 * 17, 0, 64), hr=64 * 17)), None)),
    ("d8s_prep_resize", lambda: (ctypes.byref(_prep_args(kind=1)), None)),
    ("d8s_grid_sample", lambda: (None, None)),
    ("d8s_head", lambda: (None, None)),
    ("d8s_head", lambda: (ctypes.byref(_head_args(W=129)), None)),
    ("d8s_head", lambda: (ctypes.byref(_head_args(ctx_layers=2)), None)),
    ("d8s_head", lambda: (ctypes.byref(_head_args(CD=200)), None)),
    ("d8s_head", lambda: (ctypes.byref(_head_args(ws_bytes=16)), None)),
    ("d8s_head_workspace", lambda: (None, None)),
    ("d8s_grid_sample", lambda: (ctypes.byref(hip.GridArgs(src=8, grid=8, out=8, kind=2, N=1, H=4, W=4)),
                                 None)),
    ("d8s_grid_sample", lambda: (ctypes.byref(hip.GridArgs(src=8, grid=0, out=8, kind=0, N=1, H=4, W=4)),
                                 None)),
    ("d8s_grid_sample", lambda: (ctypes.byref(hip.GridArgs(src=8, slice_idx=8, lut=8, grid=8, out=8, kind=1,
                                                           N=3, H=4, W=4, B=1, SK=2, M=2)), None)),
    ("d8s_prep_resize", lambda: (ctypes.byref(_prep_args(out=8)), None)),
    ("d8s_micro_copy", lambda: (1, 1, 17, None)),
    ("d8s_linear", lambda: (None, 2, 1664, 8, 8, 8, 8, None)),
    ("d8s_linear", lambda: (8, 0, 1664, 8, 8, 8, 8, None)),
    ("d8s_linear", lambda: (8, 2, 1664, 8, 8, 5000, 8, None)),
    ("d8s_conv2_conv1", lambda: (None, None, None)),
    ("d8s_conv2_conv1", lambda: _chain_args(W=48)),                  # a width it does not take
    ("d8s_conv2_conv1", lambda: _chain_args(G=8)),                   # conv1's last group is in in0
    ("d8s_conv2_conv1", lambda: _chain_args(out2=999)),              # conv2 writes another slot
    ("d8s_conv2_conv1", lambda: _chain_args(out1=(1 << 20) + 100)),  # the two bottlenecks overlap
    ("d8s_conv2_conv1", lambda: _chain_args(G=70)),                  # more groups than the LDS takes
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


def test_kernel_variant_queries():
    """d8s_conv1 / d8s_conv2 / d8s_transition_variant: the variant a launch with v runs (v itself, or
    for 0 the choice of d8s_conv1 / d8s_conv2 / d8s_transition, here at 256 CUs), -1 where the shape
    does not take v; a launch with a variant its shape does not take fails on the host."""
    lib = hip.library()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf)

    def gemm(N, HW, W, G0, G, cout=128, G0n=0):
        return ctypes.byref(hip.GemmArgs(p, p, p, p, p, p, p, G0, G, N, HW, W, N * HW, cout, G0n))

    def trans(N, HW, W, G0, G, cout):
        return gemm(N, HW, W, G0, G, cout, cout // 32)

    def conv2(N, H, W):
        return ctypes.byref(hip.Conv2Args(p, p, p, p, p, N, H, W, 0))

    # conv1: 393216 rows -> persistent, 64-pixel tiles; 98304 -> 32-pixel tiles; 1024 -> 4 k-slices
    assert lib.d8s_conv1_variant(gemm(96, 4096, 64, 4, 10), 0) == 2
    assert lib.d8s_conv1_variant(gemm(24, 4096, 64, 4, 10), 0) == 1
    small = gemm(1, 1024, 32, 8, 10)
    assert [lib.d8s_conv1_variant(small, v) for v in range(7)] == [5, 1, 2, 3, 4, 5, -1]
    big = gemm(64, 1 << 20, 1024, 2, 3)                     # in0 of 4 GiB: no persistent form
    assert [lib.d8s_conv1_variant(big, v) for v in range(1, 6)] == [-1, -1, 3, 4, 5]
    assert lib.d8s_conv1_variant(gemm(24, 4096, 64, 4, 10, cout=256), 1) == -1
    # conv2: tiles at most the map's width wide; 0 the widest, for 32 the tallest giving 3 tiles per CU
    assert [lib.d8s_conv2_variant(conv2(96, 16, 16), v) for v in range(10)] == [4, -1, -1, -1, 4, 5, 6, 7, 8, -1]
    assert lib.d8s_conv2_variant(conv2(96, 64, 64), 0) == 1
    assert lib.d8s_conv2_variant(conv2(24, 32, 32), 0) == 3
    assert lib.d8s_conv2_variant(conv2(1, 2, 2), 0) == 7
    # transition: depth 4 for G a multiple of 4, four weight sets for 4-5 output tiles per wave; the
    # choice: depth 2 where G is even, else 1
    t = trans(24, 1024, 32, 8, 40, 640)
    assert [lib.d8s_transition_variant(t, v) for v in range(6)] == [3, 1, 2, 3, 4, -1]
    assert [lib.d8s_transition_variant(trans(24, 1024, 32, 8, 38, 640), v) for v in range(5)] == [3, -1, -1, 3, 4]
    assert [lib.d8s_transition_variant(trans(24, 4096, 64, 2, 8, 128), v) for v in range(5)] == [3, 1, -1, 3, 4]
    assert lib.d8s_transition_variant(trans(4, 1024, 32, 8, 9, 96), 0) == 4
    assert lib.d8s_transition_variant(gemm(24, 4096, 64, 2, 8, cout=128), 1) == -1      # G0n != cout / 32
    assert lib.d8s_conv2_as(conv2(96, 16, 16), 1, None) == 1
    assert "variant 1" in lib.d8s_last_error().decode()
    assert lib.d8s_transition_as(trans(24, 1024, 32, 8, 38, 640), 1, None) == 1
    assert lib.d8s_conv1_as(big, 2, None) == 1
