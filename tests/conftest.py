"""Shared test setup: import paths, the `gpu` marker, common fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "disk-streaming-moe-engine_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def block():
    """One device context shared by the GPU tests (fails loudly without the library)."""
    from dismoen import MoEBlock
    b = MoEBlock(0)
    yield b
    b.close()


def f10(ref, cand):
    """The reference's F10 metrics of a candidate against a reference output
    (tools/dismoen-tools/src/compare.rs:648-700: delta_max = max |c - r|,
    epsilon_rel = sqrt(sum (c - r)^2 / sum r^2), float64) and its G-M3-1 gate
    for MoE-layer outputs (compare.rs:1041-1043: delta_max <= 1e-3 and
    epsilon_rel <= 1e-4)."""
    import numpy as np
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    c = np.asarray(cand, dtype=np.float64).reshape(-1)
    assert r.size == c.size and r.size > 0
    assert np.isfinite(r).all() and np.isfinite(c).all()
    d = np.abs(c - r)
    dmax = float(d.max())
    eps = float(np.sqrt(np.sum(d * d) / np.sum(r * r))) if np.any(r) else 0.0
    return dmax, eps, dmax <= 1e-3 and eps <= 1e-4


def tol_check(y, ref, factor=1e-3):
    """The parity bar: max-abs-err <= factor * RMS(ref) on the no-residual output."""
    import numpy as np
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref * ref)))
    err = float(np.max(np.abs(y - ref)))
    return err, rms, err <= factor * rms
