"""The SIMD CPU baseline (cpu_simd.c): AVX-512 + OpenMP restatement of the
fused per-token operations.

TEST AND BENCHMARK INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it
beside the GPU, and tests/test_cpu_simd_baseline.py checks it against the
scalar oracle.  The product path never imports it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import _HERE, build

LIB_PATH = os.path.join(_HERE, "libvestra_cpu_simd.so")
if not os.path.exists(LIB_PATH):
    build()
lib = C.CDLL(LIB_PATH)

_vp, _sz, _f, _i = C.c_void_p, C.c_size_t, C.c_float, C.c_int
for _n, (_a, _r) in {
    "cs_available": ([], _i),
    "cs_set_threads": ([_i], None),
    "cs_layernorm_f32": ([_vp, _vp, _sz, _sz, _vp, _vp, _f], None),
    "cs_gelu_f32": ([_vp, _sz], None),
    "cs_layerscale_residual_f32": ([_vp, _vp, _vp, _sz, _sz], None),
    "cs_qk_norm_rope_f32": ([_vp] * 7 + [_sz, _sz, _f, _f], None),
}.items():
    _fn = getattr(lib, _n)
    _fn.argtypes = _a
    _fn.restype = _r


def available() -> bool:
    """The host has AVX-512 F/BW/DQ/VL."""
    return bool(lib.cs_available())


def set_threads(n: int) -> None:
    lib.cs_set_threads(int(n))


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def layernorm_into(x, out, gamma, beta, eps: float) -> None:
    cols = x.shape[-1]
    lib.cs_layernorm_f32(_p(x), _p(out), x.size // cols, cols, _p(gamma), _p(beta), eps)


def gelu_(x) -> None:
    lib.cs_gelu_f32(_p(x), x.size)


def layerscale_residual_(x, y, gamma) -> None:
    cols = x.shape[-1]
    lib.cs_layerscale_residual_f32(_p(x), _p(y), _p(gamma), x.size // cols, cols)


def qk_norm_rope_(q, k, qg, qb, kg, kb, pos_yx, heads: int, n: int, base: float = 100.0,
                  eps: float = 1e-5) -> None:
    lib.cs_qk_norm_rope_f32(_p(q), _p(k), _p(qg), _p(qb), _p(kg), _p(kb), _p(pos_yx), heads, n,
                            base, eps)
