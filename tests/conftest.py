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


# ---------------------------------------------------------------- parity margins
# What a passing comparison leaves of its bar: tests record them under a
# group name, and the session ends with the worst record of every group
# (also written as JSON to $VK_MARGINS_OUT when that is set).
_MARGINS = {}


def record_margin(group, got, ref, tol=None, atol=None, rtol=None, label=""):
    """Record max |got - ref|, the mean |got - ref|, the largest relative
    error over |ref| >= 1e-3 and the share of the bound used (max of
    |got - ref| / tol, tol = the given bound array or atol + rtol*|ref|)
    under `group`; returns the record."""
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    r = np.asarray(ref, dtype=np.float64).reshape(-1)
    d = np.abs(g - r)
    if tol is None:
        tol = (atol or 0.0) + (rtol or 0.0) * np.abs(r)
    tol = np.asarray(tol, dtype=np.float64)
    tol = tol.reshape(-1) if tol.size == d.size else np.broadcast_to(tol, d.shape)
    big = np.abs(r) >= 1e-3
    rec = {"label": label or group, "n": int(d.size),
           "max_abs": float(d.max()) if d.size else 0.0,
           "mae": float(d.mean()) if d.size else 0.0,
           "max_rel_ref_ge_1e-3": float((d[big] / np.abs(r[big])).max()) if big.any() else 0.0,
           "bound_used": float((d / np.where(tol > 0, tol, np.inf)).max()) if d.size else 0.0}
    _MARGINS.setdefault(group, []).append(rec)
    return rec


def pytest_terminal_summary(terminalreporter):
    if not _MARGINS:
        return
    terminalreporter.section("parity margins (worst per group: max|d|, mean|d|, max rel "
                             "where |ref|>=1e-3, share of the bar used)")
    for group in sorted(_MARGINS):
        recs = _MARGINS[group]
        w = max(recs, key=lambda r: r["bound_used"])
        terminalreporter.write_line(
            f"{group}: max|d| {max(r['max_abs'] for r in recs):.2e}  "
            f"mae {max(r['mae'] for r in recs):.2e}  "
            f"rel {max(r['max_rel_ref_ge_1e-3'] for r in recs):.2e}  "
            f"bar {100 * w['bound_used']:.1f}% ({w['label']}; {len(recs)} cases)")
    out = os.environ.get("VK_MARGINS_OUT")
    if out:
        import json
        with open(out, "w") as f:
            json.dump(_MARGINS, f, indent=1)


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
