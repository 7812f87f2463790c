"""rew's keyed host generators over librew_mi355x.

Same names and meaning as the reference:

* ``initKey`` / ``split`` / ``foldIn`` -- src/rew/rng.nim:57-80 (Threefry-2x32,
  four rounds, as rew defines it at rng.nim:39-55)
* ``uniformF32`` / ``normalF32``       -- src/rew/nn/init.nim:19-51 (24-bit
  uniforms, Box-Muller on ``foldIn(key, i)`` pairs)
* ``xavierUniformF32``                 -- src/rew/nn/init.nim:93-97

The samplers run in the native library (multi-threaded over disjoint index
ranges, so the values do not depend on the thread count).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

Key = tuple  # (a, b) uint32 halves, rng.nim Key


def initKey(seed: int) -> Key:
    """Low and high 32-bit halves of the 64-bit seed (rng.nim:57-63)."""
    return (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)


def split(key: Key, n: int = 2) -> list:
    """n child keys: threefry(key, (i, 0)) (rng.nim:65-73)."""
    if n <= 0:
        return []
    out = (C.c_uint32 * (2 * n))()
    _lib.load().rew_mi355x_rng_split(key[0], key[1], n, out)
    return [(out[2 * i], out[2 * i + 1]) for i in range(n)]


def foldIn(key: Key, data: int) -> Key:
    """threefry(key, (lo32(data), hi32(data))) (rng.nim:75-80)."""
    out = (C.c_uint32 * 2)()
    _lib.load().rew_mi355x_rng_fold_in(key[0], key[1], data, out)
    return (out[0], out[1])


def uniformF32(key: Key, count: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.float32)
    _lib.load().rew_mi355x_rng_uniform_f32(key[0], key[1], count, lo, hi,
                                           out.ctypes.data_as(C.c_void_p))
    return out


def normalF32(key: Key, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.float32)
    _lib.load().rew_mi355x_rng_normal_f32(key[0], key[1], count, mean, std,
                                          out.ctypes.data_as(C.c_void_p))
    return out


def xavierUniformF32(key: Key, fanIn: int, fanOut: int) -> np.ndarray:
    """U(-b, b) with b = sqrt(6 / (fanIn + fanOut)) computed in float32."""
    bound = float(np.sqrt(np.float32(6.0) / np.float32(fanIn + fanOut)))
    return uniformF32(key, fanIn * fanOut, -bound, bound)


def tokenIds(key: Key, count: int, vocab: int) -> np.ndarray:
    """Uniform token ids: ``foldIn(key, i).a mod vocab`` as int32."""
    ids = np.empty(count, np.int32)
    for i in range(count):
        ids[i] = foldIn(key, i)[0] % vocab
    return ids
