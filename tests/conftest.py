"""pytest setup: import paths, the `gpu` marker, shared fixtures.

Tests marked `gpu` run on an MI355X through the C ABI of libgemma_hip; they
fail (never skip) when no device is visible, so a CPU fallback can never pass
for them.  Unmarked tests run on the CPU: the oracle against the reference's
golden vectors, host logic, and the library's exported symbols.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "gemma.hs_amd", REPO / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libgemma_hip)")


def load_ref_golden(name: str) -> np.ndarray:
    """A tensor of the reference's test/golden-values fixtures (key 'output')."""
    from safetensors.numpy import load_file
    return load_file(str(GOLDEN / "reference" / f"{name}.safetensors"))["output"]


def rel_err(a, b) -> float:
    """max |a-b| / max |b|: the relative error used for activation parity."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = max(float(np.max(np.abs(b))), 1e-30)
    return float(np.max(np.abs(a - b))) / den


@pytest.fixture(scope="session")
def ctx():
    import gemma_hip as gh
    n = gh.device_count()
    if n == 0:
        pytest.fail("gpu test but no HIP device is visible (no CPU fallback exists)")
    c = gh.Context(0)
    yield c
    c.close()
