"""Seeded synthetic inputs shared by bench.py and tests (CPU, numpy).

The reference has no normal generator, so this one is frozen here:
splitmix64 used as a counter-based stream per tensor, element i drawing
mix(seed + (i+1)*0x9E3779B97F4A7C15); uniforms are (z >> 40) * 2^-24;
normals come from Box-Muller in float64 over consecutive uniform pairs and are
rounded to float32 after scaling.  Seeds are 0x51C0DE00 + 16*config + tensor_id.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def seed_for(config: int, tensor_id: int) -> int:
    return 0x51C0DE00 + 16 * config + tensor_id


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, count: int) -> np.ndarray:
    """float64 uniforms in [0, 1 - 2^-24], multiples of 2^-24."""
    return (splitmix64(seed, count) >> np.uint64(40)).astype(np.float64) * 2.0 ** -24


def normal(seed: int, count: int, sigma: float = 1.0, chunk: int = 1 << 22) -> np.ndarray:
    """float32 N(0, sigma^2) by Box-Muller over uniform pairs (2i, 2i+1)."""
    out = np.empty(count, dtype=np.float32)
    pairs = (count + 1) // 2
    for p0 in range(0, pairs, chunk):
        p1 = min(pairs, p0 + chunk)
        z = splitmix64(seed, 2 * (p1 - p0), offset=2 * p0)
        u = (z >> np.uint64(40)).astype(np.float64) * 2.0 ** -24
        r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        t = 2.0 * np.pi * u[1::2]
        v = np.empty(2 * (p1 - p0), dtype=np.float64)
        v[0::2] = r * np.cos(t)
        v[1::2] = r * np.sin(t)
        lo, hi = 2 * p0, min(count, 2 * p1)
        out[lo:hi] = (v[: hi - lo] * sigma).astype(np.float32)
    return out


def activations_with_outliers(config: int, m: int, k: int) -> np.ndarray:
    """x ~ N(0,1) with an independent 0.1% of entries multiplied by 20."""
    x = normal(seed_for(config, 1), m * k)
    hit = uniform(seed_for(config, 2), m * k) < 0.001
    x[hit] *= np.float32(20.0)
    return x.reshape(m, k)


# --- fast path: the same streams from csrc/synth.c (OpenMP), bit-identical --
_clib = None


def _c():
    global _clib
    if _clib is None:
        import ctypes
        import os
        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqcsynth.so")
        if not os.path.exists(path):
            return None
        lib = ctypes.CDLL(path)
        lib.qcs_normal.argtypes = [ctypes.c_uint64, ctypes.c_longlong, ctypes.c_double,
                                   ctypes.c_void_p]
        lib.qcs_uniform.argtypes = [ctypes.c_uint64, ctypes.c_longlong, ctypes.c_void_p]
        _clib = lib
    return _clib


def normal_fast(seed: int, count: int, sigma: float = 1.0) -> np.ndarray:
    lib = _c()
    if lib is None:
        return normal(seed, count, sigma)
    out = np.empty(count, dtype=np.float32)
    lib.qcs_normal(seed, count, sigma, out.ctypes.data)
    return out


def uniform_fast(seed: int, count: int) -> np.ndarray:
    lib = _c()
    if lib is None:
        return uniform(seed, count)
    out = np.empty(count, dtype=np.float64)
    lib.qcs_uniform(seed, count, out.ctypes.data)
    return out


def weights(config: int, n: int, k: int, tensor_id: int = 0, sigma: float = 0.02) -> np.ndarray:
    """f32 weights [n, k] ~ N(0, sigma^2)."""
    return normal_fast(seed_for(config, tensor_id), n * k, sigma).reshape(n, k)


def activations(config: int, m: int, k: int, tensor_id: int = 1) -> np.ndarray:
    """f32 activations [m, k] ~ N(0, 1)."""
    return normal_fast(seed_for(config, tensor_id), m * k).reshape(m, k)


def activations_outliers_fast(config: int, m: int, k: int) -> np.ndarray:
    x = normal_fast(seed_for(config, 1), m * k)
    x[uniform_fast(seed_for(config, 2), m * k) < 0.001] *= np.float32(20.0)
    return x.reshape(m, k)
