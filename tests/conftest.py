"""pytest setup: the `gpu` marker, the package (directory `rsna-knee-efficiency_amd/` imported as
`rsna_knee_efficiency_amd`) and the repository root on sys.path (for `oracle`)."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built HIP library")


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from rsna_knee_efficiency_amd import hip
    hip.library()          # raises if the HIP library is missing (no fallback) or stale
    assert hip.built_sha() == hip.source_sha(), "libd8s_hip.so is not built from the tree's sources"
    print(f"\nlibrary {hip.version()}", flush=True)
    return torch.device("cuda:0")
