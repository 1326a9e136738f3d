"""ctypes binding of `libd8s_hip.so`, the gfx950 kernel library (C ABI: `include/d8s_hip.h`).

The reference compiles its CUDA source with NVRTC and launches kernels through the driver API from
ctypes (`src/knee/cudart.py:1-15,87-152`).  Here the kernels are compiled ahead of time by hipcc into
one shared library whose `extern "C"` entry points take the same by-value argument structs the
reference's kernels take (`KArg` -> `D8sGemmArgs`, `C2Arg` -> `D8sConv2Args`) and a `hipStream_t`
(a torch stream's `cuda_stream`).  Launches are asynchronous and are recorded into HIP graphs when
the stream is capturing.  A failing call raises `D8sError` carrying the HIP error code and message,
as `cudart.CudaError` carries the CUresult (`src/knee/cudart.py:29-31,57-65`).

There is no fallback: if the library is missing, `library()` raises.
"""
from __future__ import annotations

import ctypes
import hashlib
import threading
from pathlib import Path

import torch

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
SOURCE = CSRC / "d8s_kernels.hip"
# every file compiled into the library (the first is SOURCE)
SOURCES = (SOURCE, CSRC / "d8s_prep.hip", CSRC / "d8s_head.hip", CSRC / "d8s_host.h")
HEADER = PKG.parent / "include" / "d8s_hip.h"
LIB_PATH = PKG / "libd8s_hip.so"
ABI_VERSION = 1

_LOCK = threading.Lock()
_STATE: dict = {}


class D8sError(RuntimeError):
    """A failed library call: `code` is the hipError_t, the message comes from d8s_last_error()."""

    def __init__(self, what: str, code: int, msg: str) -> None:
        super().__init__(f"{what}: hipError {code}: {msg}")
        self.code = code


i32, u64, vp = ctypes.c_int32, ctypes.c_uint64, ctypes.c_void_p


class GemmArgs(ctypes.Structure):
    """`D8sGemmArgs` (the reference's `KArg`, `src/knee/dense8s.py:76-82`, plus `wsum`)."""
    _fields_ = [("in0", u64), ("seg", u64), ("w", u64), ("abh", u64), ("gd", u64), ("wsum", u64),
                ("out", u64), ("G0", i32), ("G", i32), ("N", i32), ("HW", i32), ("W", i32),
                ("rows", i32), ("cout", i32), ("G0n", i32)]


class Conv2Args(ctypes.Structure):
    """`D8sConv2Args` (the reference's `C2Arg`, `src/knee/dense8s.py:131-137`, plus `wsum`)."""
    _fields_ = [("x", u64), ("w", u64), ("sc", u64), ("wsum", u64), ("out", u64), ("N", i32),
                ("H", i32), ("W", i32), ("pad_", i32)]


class DenseArgs(ctypes.Structure):
    """`D8sDenseArgs`: a dense layer with conv1 and conv2 fused (the reference's `TileArg` + `LayerP`,
    `src/knee/dense8s.py:139-152`)."""
    _fields_ = [("in0", u64), ("seg", u64), ("w1", u64), ("abh", u64), ("gd", u64), ("w1sum", u64),
                ("w2", u64), ("sc", u64), ("w2sum", u64), ("out", u64), ("G0", i32), ("G", i32),
                ("N", i32), ("H", i32), ("W", i32), ("pad_", i32)]


class LayerP(ctypes.Structure):
    """`D8sLayerP`: one layer's tables for d8s_dense_block (the reference's `LayerP`,
    `src/knee/dense8s.py:139-143`, plus the weight sums)."""
    _fields_ = [("w1", u64), ("abh", u64), ("gd", u64), ("w1sum", u64), ("w2", u64), ("sc", u64),
                ("w2sum", u64)]


class BlockArgs(ctypes.Structure):
    """`D8sBlockArgs`: a whole dense block (the reference's `ImgArg`, `src/knee/dense8s.py:155-159`)."""
    _fields_ = [("in0", u64), ("seg", u64), ("layers", u64), ("N", i32), ("H", i32), ("W", i32),
                ("G0", i32), ("L", i32), ("pad_", i32)]


class PartsArgs(ctypes.Structure):
    """`D8sPartsArgs`: a whole dense block with every image split into row bands across workgroups."""
    _fields_ = [("in0", u64), ("seg", u64), ("layers", u64), ("sync", u64), ("xchg", u64), ("N", i32),
                ("H", i32), ("W", i32), ("G0", i32), ("L", i32), ("parts", i32)]


def parts_sync_words(nparts: int) -> int:
    """`D8S_PARTS_SYNC_WORDS`: uint32 words of d8s_dense_block_parts' synchronisation memory."""
    return 64 + 0 * nparts


def parts_xchg_bytes(nparts: int, w: int) -> int:
    """`D8S_PARTS_XCHG_BYTES`: bytes of its exchange rows."""
    return nparts * 1024 * w


PARTS_PIXELS = (32, 64, 128, 256)        # pixels per band d8s_dense_block_parts runs
C21_WIDTHS = (16, 32, 64)                # map widths d8s_conv2_conv1 runs (H * W a multiple of 128)
C21_MAX_GROUPS = 64                      # `D8S_C21_MAX_GROUPS`


class StemArgs(ctypes.Structure):
    """`D8sStemArgs`: the stem with the fused uint8 normalisation / flip of the input."""
    _fields_ = [("x", u64), ("lut", u64), ("w16", u64), ("bias", u64), ("inv", u64), ("out", u64),
                ("N", i32), ("H", i32), ("W", i32), ("kind", i32), ("flip", i32), ("pad_", i32)]


class PrepStack(ctypes.Structure):
    """`D8sPrepStack`: one stack of the preprocessing (a series at one crop scale)."""
    _fields_ = [("src", u64), ("resc", u64), ("out", u64), ("K", i32), ("hr", i32), ("wr", i32),
                ("y0", i32), ("y1", i32), ("x0", i32), ("x1", i32), ("k0", i32), ("k1", i32),
                ("flip", i32), ("r1", i32), ("r2", i32), ("g1", ctypes.c_double),
                ("g2", ctypes.c_double)]


PREP_MAX_STACKS = 16


class PrepStat(ctypes.Structure):
    """`D8sPrepStat`: the percentiles, scale and bad flag d8s_prep leaves per stack."""
    _fields_ = [("lo", ctypes.c_double), ("hi", ctypes.c_double), ("scale", ctypes.c_double),
                ("bad", i32), ("pad_", i32)]


class PrepArgs(ctypes.Structure):
    """`D8sPrepArgs`: the arguments of d8s_prep / d8s_prep_resize."""
    _fields_ = [("workspace", u64), ("ws_bytes", u64), ("scratch", u64), ("scratch_bytes", u64),
                ("kind", i32), ("img", i32),
                ("n_stacks", i32), ("pad_", i32), ("s", PrepStack * PREP_MAX_STACKS)]


class GridArgs(ctypes.Structure):
    """`D8sGridArgs`: bilinear grid sampling of fp16 images (the geometric TTA view)."""
    _fields_ = [("src", u64), ("slice_idx", u64), ("lut", u64), ("grid", u64), ("out", u64),
                ("kind", i32), ("N", i32), ("H", i32), ("W", i32), ("B", i32), ("SK", i32),
                ("M", i32), ("pad_", i32)]


HEAD_WEIGHTS = ("slot_emb", "ctx_in_w", "ctx_in_b", "ctx_pos", "in_proj_w", "in_proj_b", "out_proj_w",
                "out_proj_b", "ln1_w", "ln1_b", "ln2_w", "ln2_b", "ff1_w", "ff1_b", "ff2_w", "ff2_b",
                "ctx_out_w", "ctx_out_b", "attn_w", "attn_b", "cls_w", "cls_b")


class HeadArgs(ctypes.Structure):
    """`D8sHeadArgs`: the head after the encoder (context layer + per-finding attention pooling)."""
    _fields_ = ([("z", u64), ("slot_of", u64), ("slot_mask", u64)]
                + [(n, u64) for n in HEAD_WEIGHTS]
                + [("logits", u64), ("workspace", u64), ("ws_bytes", u64)]
                + [(n, i32) for n in ("B", "W", "D", "S", "CD", "heads", "FF", "PER", "T", "ctx_layers")])


IN_F16, IN_U8 = 0, 1

# entry point -> argument types (all return int32 status)
SIGNATURES = {
    "d8s_conv1": [ctypes.POINTER(GemmArgs), vp],
    "d8s_conv1_acc32": [ctypes.POINTER(GemmArgs), vp, vp],
    "d8s_conv1_variant": [ctypes.POINTER(GemmArgs), ctypes.c_int32],
    "d8s_conv1_as": [ctypes.POINTER(GemmArgs), ctypes.c_int32, vp],
    "d8s_conv2_variant": [ctypes.POINTER(Conv2Args), ctypes.c_int32],
    "d8s_conv2_as": [ctypes.POINTER(Conv2Args), ctypes.c_int32, vp],
    "d8s_transition_variant": [ctypes.POINTER(GemmArgs), ctypes.c_int32],
    "d8s_transition_as": [ctypes.POINTER(GemmArgs), ctypes.c_int32, vp],
    "d8s_conv2": [ctypes.POINTER(Conv2Args), vp],
    "d8s_dense": [ctypes.POINTER(DenseArgs), vp],
    "d8s_conv2_conv1": [ctypes.POINTER(Conv2Args), ctypes.POINTER(GemmArgs), vp],
    "d8s_c21_supported": [i32, i32, i32],
    "d8s_dense_block": [ctypes.POINTER(BlockArgs), vp],
    "d8s_dense_block_parts": [ctypes.POINTER(PartsArgs), vp],
    "d8s_transition": [ctypes.POINTER(GemmArgs), vp],
    "d8s_final": [vp, i32, vp, i32, i32, vp, vp, i32, vp],
    "d8s_final_checked": [vp, i32, vp, i32, i32, vp, vp, i32, vp, vp, vp],
    "d8s_host_mapped": [vp, ctypes.POINTER(vp)],
    "d8s_parts_supported": [i32, i32, i32, i32],
    "d8s_linear": [vp, i32, i32, vp, vp, i32, vp, vp],
    "d8s_stem": [ctypes.POINTER(StemArgs), vp],
    "d8s_stem_pair": [ctypes.POINTER(StemArgs), ctypes.POINTER(StemArgs), vp],
    "d8s_conv1_pair": [ctypes.POINTER(GemmArgs), ctypes.POINTER(GemmArgs), vp],
    "d8s_conv2_pair": [ctypes.POINTER(Conv2Args), ctypes.POINTER(Conv2Args), vp],
    "d8s_dense_pair": [ctypes.POINTER(DenseArgs), ctypes.POINTER(DenseArgs), vp],
    "d8s_dense_block_pair": [ctypes.POINTER(BlockArgs), ctypes.POINTER(BlockArgs), vp],
    "d8s_transition_pair": [ctypes.POINTER(GemmArgs), ctypes.POINTER(GemmArgs), vp],
    "d8s_prep_workspace": [i32, i32, ctypes.POINTER(ctypes.c_uint64)],
    "d8s_prep": [ctypes.POINTER(PrepArgs), vp],
    "d8s_prep_resize": [ctypes.POINTER(PrepArgs), vp],
    "d8s_grid_sample": [ctypes.POINTER(GridArgs), vp],
    "d8s_head_workspace": [ctypes.POINTER(HeadArgs), ctypes.POINTER(ctypes.c_uint64)],
    "d8s_head": [ctypes.POINTER(HeadArgs), vp],
    "d8s_head_noalloc": [ctypes.POINTER(HeadArgs), vp],
    "d8s_micro_copy": [vp, vp, ctypes.c_size_t, vp],
    "d8s_micro_mfma": [i32, i32, vp, vp],
    "d8s_probe_mfma_i8": [vp, vp, vp, vp],
    "d8s_probe_mfma_f16": [vp, vp, vp, vp],
}
STRING_FUNCS = ("d8s_version", "d8s_last_error")


def source_sha() -> str:
    """Hash of the kernel source and header: the build's `kernels_sha` (`src/knee/dense8s.py:781-783`)."""
    h = hashlib.sha1()
    for f in SOURCES:
        h.update(f.read_bytes())
    h.update(HEADER.read_bytes())
    return h.hexdigest()[:12]


class StaleLibrary(D8sError):
    """The library on disk was built from other sources than the ones beside it."""


def check_fresh(lib: ctypes.CDLL, where: Path) -> str:
    """The source hash compiled into `lib`; raises StaleLibrary when the kernel sources are present and
    hash otherwise -- the library would run kernels other than the ones in the tree (the reference
    checks its package's cubin against `kernels_sha` and recompiles, `src/knee/dense8s.py:883-908`;
    here rebuilding is `__graft_entry__.build()`, outside the runtime)."""
    fn = lib.d8s_version
    fn.argtypes, fn.restype = [], ctypes.c_char_p
    fields = fn().decode().split()
    built = fields[2] if len(fields) >= 3 else ""
    if all(f.is_file() for f in SOURCES) and HEADER.is_file():
        want = source_sha()
        if built != want:
            raise StaleLibrary("library", 0, f"{where} was built from sources {built or '?'}, the tree's "
                                             f"hash {want}: run __graft_entry__.build()")
    return built


def library(path: Path | None = None) -> ctypes.CDLL:
    """The loaded library (once per process), checked against the kernel sources (`check_fresh`).
    Raises FileNotFoundError / OSError if it is missing: the encoder has no other implementation.
    """
    with _LOCK:
        lib = _STATE.get("lib")
        if lib is not None:
            return lib
        p = Path(path or LIB_PATH)
        if not p.is_file():
            raise FileNotFoundError(f"{p}: the HIP kernel library is not built "
                                    f"(run __graft_entry__.build())")
        lib = ctypes.CDLL(str(p))
        check_fresh(lib, p)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int32
        for name in STRING_FUNCS:
            fn = getattr(lib, name)
            fn.argtypes = []
            fn.restype = ctypes.c_char_p
        _STATE["lib"] = lib
        return lib


def version() -> str:
    return library().d8s_version().decode()


def built_sha() -> str:
    """The source hash compiled into the loaded library."""
    parts = version().split()
    return parts[2] if len(parts) >= 3 else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise D8sError(what, int(rc), library().d8s_last_error().decode())


def call(name: str, *args) -> None:
    """Calls entry point `name` and raises D8sError on a non-zero status."""
    check(getattr(library(), name)(*args), name)


def written(*tensors) -> None:
    """Marks tensors a kernel wrote through a raw pointer as modified: bumps their version counter
    (shared with their base and views), as an in-place torch op would, so a later consumer that
    keys on (storage, version) sees new contents."""
    for t in tensors:
        if t is not None:
            torch.autograd.graph.increment_version(t)
