"""Shared test setup: the `gpu` marker, the product package (loaded by path,
its directory name has a hyphen) and the CPU oracle (test infrastructure)."""
from __future__ import annotations

import importlib.util
import os
import pathlib
import sys

import pytest
import torch  # noqa: F401  -- imported at collection: the first import on a fresh box is slow

REPO = pathlib.Path(__file__).resolve().parents[1]
PKG_DIR = REPO / "rich-triplet_amd"
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def load_pkg():
    if "rich_triplet_amd" in sys.modules:
        return sys.modules["rich_triplet_amd"]
    spec = importlib.util.spec_from_file_location("rich_triplet_amd", PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["rich_triplet_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through librt_hip.so on cuda:0)")


@pytest.fixture(scope="session")
def rt():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test scheduled on a host without a GPU")
    return torch.device("cuda:0")


def to_dev(arr, device):
    """numpy array -> torch tensor on `device` (same bytes)."""
    import numpy as np
    import torch
    t = torch.from_numpy(np.ascontiguousarray(arr))
    return t.to(device)


def rel_l2(got, ref) -> float:
    import numpy as np
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))
