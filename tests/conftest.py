"""Shared fixtures. GPU tests carry @pytest.mark.gpu and run on an MI355X."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


_CACHE: dict[str, str] = {}


@pytest.fixture(scope="session")
def synth(model_dir):
    """synth(name) -> path of that workload's GGUF (written once per session)."""
    from chonklm_amd import write_synthetic_gguf

    def make(name: str) -> str:
        if name not in _CACHE:
            path = str(model_dir / f"{name}.gguf")
            write_synthetic_gguf(name, path, threads=min(16, os.cpu_count() or 4))
            _CACHE[name] = path
        return _CACHE[name]

    return make


def rel_err(a: np.ndarray, b: np.ndarray) -> float:
    """max |a - b| / max |b| (the parity metric for fp32 outputs)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))
