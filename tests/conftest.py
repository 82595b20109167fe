"""Shared test setup.

Markers: `gpu` tests need an MI355X and call the HIP library through its C ABI;
everything else runs on the CPU (oracle pins, host logic, ABI exports).
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vestra-engine_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

SEED = 20260812


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


def parity_report(got, ref, atol, rtol):
    """da-parity compare semantics (da-parity/src/lib.rs:64-129): pass iff
    |got - ref| <= atol + rtol*|ref| element-wise; empty or size mismatch fail.
    One deliberate difference: a NaN on either side fails here, where the
    reference's `d > tol` test lets it pass."""
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    ref = np.asarray(ref, dtype=np.float64).reshape(-1)
    if got.size != ref.size or got.size == 0:
        return False, float("inf"), 0
    d = np.abs(got - ref)
    worst = int(np.argmax(d))
    ok = bool(np.all(d <= atol + rtol * np.abs(ref)))
    return ok, float(d[worst]), worst


def assert_parity(got, ref, atol, rtol, label=""):
    ok, max_abs, worst = parity_report(got, ref, atol, rtol)
    if not ok:
        g = np.asarray(got).reshape(-1)
        r = np.asarray(ref).reshape(-1)
        detail = "" if g.size != r.size or g.size == 0 else \
            f" worst@{worst} got={g[worst]!r} ref={r[worst]!r}"
        raise AssertionError(f"[{label}] parity FAIL max|d|={max_abs:.3e}{detail} "
                             f"(atol={atol}, rtol={rtol})")


# F32 parity bar (rtol 1e-5 with a stated atol 1e-6) and the F16-stored-weight
# bar (rtol 2e-3, atol 2e-3; da-parity's default manifest tolerance).
F32_RTOL, F32_ATOL = 1e-5, 1e-6
W16_RTOL, W16_ATOL = 2e-3, 2e-3


@pytest.fixture
def rng():
    return np.random.default_rng(SEED)


@pytest.fixture(scope="session")
def rt():
    import vestra_hip
    r = vestra_hip.Runtime(0)
    yield r
    r.synchronize()
