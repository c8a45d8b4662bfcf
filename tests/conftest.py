"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on the
CPU (oracle pinning, host logic, ABI exports)."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o  # test infrastructure (oracle/oracle.py)

    return o


@pytest.fixture(scope="session")
def ctx():
    """Device context; fails (never skips) when the library or GPU is missing."""
    import wohper_amd

    c = wohper_amd.Context(0)
    yield c
    c.close()


def lcg_bytes(seed: int, count: int):
    """E/compute.rs:7396-7404"""
    out = []
    state = seed & 0xFFFFFFFF
    for _ in range(count):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out.append(state >> 24)
    return out


def lcg_f32(seed: int, count: int):
    """E/compute.rs:7406-7414"""
    import numpy as np

    out = []
    state = seed & 0xFFFFFFFF
    for _ in range(count):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out.append(np.float32(np.float32(state >> 16) / np.float32(65536.0)) - np.float32(0.5))
    return np.array(out, np.float32)
