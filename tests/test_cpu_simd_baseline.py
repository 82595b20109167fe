"""The SIMD CPU baseline (oracle/cpu_simd.c) against the scalar oracle.

The baseline is what bench.py times as the reference's AVX-512 CPU path; it
must compute the same functions: rtol 1e-5 / atol 1e-6 where its row sums
run 16 lanes wide or its GELU takes its own exp, bit-exact for LayerScale +
residual (no reduction, the same two roundings).
"""
import numpy as np
import pytest

import oracle
from conftest import F32_ATOL, F32_RTOL, assert_parity

simd = pytest.importorskip("oracle.simd")
pytestmark = pytest.mark.skipif(not simd.available(), reason="host lacks AVX-512")


def test_layernorm(rng):
    for rows, cols in ((866, 768), (37, 1024), (5, 40)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        g = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
        b = (0.02 * rng.standard_normal(cols)).astype(np.float32)
        out = np.empty_like(x)
        simd.layernorm_into(x, out, g, b, 1e-6)
        assert_parity(out, oracle.layernorm(x, g, b, 1e-6), F32_ATOL, F32_RTOL, f"ln {cols}")


def test_gelu_including_tails(rng):
    x = np.concatenate([rng.standard_normal(866 * 3072).astype(np.float32) * 3,
                        np.array([0.0, -0.0, 10.0, -10.0, 20.0, -20.0, 1e-8, -1e-8, 5.5],
                                 np.float32)])
    y = x.copy()
    simd.gelu_(y)
    assert_parity(y, oracle.gelu(x), F32_ATOL, F32_RTOL, "gelu")


def test_layerscale_residual_bit_exact(rng):
    x = rng.standard_normal((866, 768)).astype(np.float32)
    y = rng.standard_normal((866, 768)).astype(np.float32)
    g = rng.uniform(0, 0.1, 768).astype(np.float32)
    out = x.copy()
    simd.layerscale_residual_(out, y, g)
    assert np.array_equal(out, oracle.layerscale_residual(x, y, g))


def test_qk_norm_rope(rng):
    heads, n_special, gh, gw = 12, 2, 24, 36
    n = n_special + gh * gw
    q = rng.standard_normal((heads, n, 64)).astype(np.float32)
    k = rng.standard_normal((heads, n, 64)).astype(np.float32)
    qg, qb, kg, kb = [(s + 0.02 * rng.standard_normal(64)).astype(np.float32)
                      for s in (1.0, 0.0, 1.0, 0.0)]
    pos = oracle.rope_positions(n_special, gh, gw, 1, False)
    qo, ko = q.copy(), k.copy()
    simd.qk_norm_rope_(qo, ko, qg, qb, kg, kb, pos, heads, n)
    rq, rk = oracle.qk_norm_rope(q, k, qg, qb, kg, kb, pos, heads, n)
    assert_parity(qo, rq, F32_ATOL, F32_RTOL, "q")
    assert_parity(ko, rk, F32_ATOL, F32_RTOL, "k")
