"""Shared pytest configuration.

Marker `gpu`: needs an MI355X and the built libspock_hip.so; run with -m gpu.
Everything else runs on the CPU (oracle pinning, host logic, ABI surface).
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: requires an MI355X GPU and the built HIP library")


def max_rel(a, b):
    """|a-b| / max(1, |b|), the reference probes' metric
    (apps/spock-deltanet-chunk-prefill-tiled-probe.cpp:286)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b) / np.maximum(1.0, np.abs(b)))) if a.size else 0.0


def fp16_ulp(a, b):
    """Per-element fp16 ULP distance (diary/0089_fp16_ulp_tolerance_policy.md:30-37):
    0 for equal bits or +-0, 65535 for opposite signs, else |bits(a)-bits(b)|."""
    a = np.asarray(a, dtype=np.uint16).astype(np.int32)
    b = np.asarray(b, dtype=np.uint16).astype(np.int32)
    ma, mb = a & 0x7FFF, b & 0x7FFF
    d = np.abs(ma - mb)
    opp = ((a >> 15) != (b >> 15)) & ~((ma == 0) & (mb == 0))
    d[opp] = 65535
    return d


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    oracle_lib.lib()
    return oracle_lib


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from spock_amd import _lib
    _lib.lib()  # fail loudly if the HIP library is missing
    return torch.device("cuda:0")
