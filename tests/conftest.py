"""Shared fixtures. GPU tests are marked `gpu`; CPU tests cover the oracle, the
host logic and the C-ABI library's exported symbols."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through libythip.so)")
    config.addinivalue_line("markers", "slow: large CPU oracle work (full-size configs)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible (gpu tests run on the MI355X box)")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle.oracle()


@pytest.fixture(scope="session")
def ref():
    import oracle
    r = oracle.reference()
    if r is None:
        pytest.skip("compiled reference (oracle/_ref) not built here")
    return r


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def yt():
    import ytensor_amd
    ytensor_amd.load()
    return ytensor_amd


def rel_err(g: np.ndarray, r: np.ndarray) -> float:
    """max|g - r| / max|r| (the parity bar's relative error)."""
    g = g.astype(np.float64)
    r = r.astype(np.float64)
    den = np.abs(r).max()
    return float(np.abs(g - r).max() / (den if den > 0 else 1.0))


def mae(g: np.ndarray, r: np.ndarray) -> float:
    return float(np.abs(g.astype(np.float64) - r.astype(np.float64)).mean())
