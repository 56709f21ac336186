"""numpy restatement of libhwk's synthetic draws (hwnpu_amd/csrc/synth.h), to check them and to
make small inputs on the host: splitmix64 at state key + (i+1)*gamma, Box-Muller in float64."""
from __future__ import annotations

import numpy as np

from hwnpu_amd.synth import key_of

GAMMA = np.uint64(0x9E3779B97F4A7C15)


def splitmix_at(key: int, idx: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(key) + (idx.astype(np.uint64) + np.uint64(1)) * GAMMA
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def bytes_(n: int, name: str, seed: int = 0) -> np.ndarray:
    return (splitmix_at(key_of(name, seed), np.arange(n, dtype=np.uint64)) & np.uint64(0xFF)).astype(np.uint8)


def uniform_int(n: int, lo: int, span: int, name: str, seed: int = 0) -> np.ndarray:
    top = splitmix_at(key_of(name, seed), np.arange(n, dtype=np.uint64)) >> np.uint64(32)
    return (lo + ((top * np.uint64(span)) >> np.uint64(32)).astype(np.int64)).astype(np.int64)


def normal64(n: int, name: str, seed: int = 0, first: int = 0) -> np.ndarray:
    """float64 normals of elements first .. first+n-1."""
    key = key_of(name, seed)
    i = np.arange(first, first + n, dtype=np.uint64)
    p = i & ~np.uint64(1)
    u1 = (splitmix_at(key, p) >> np.uint64(11)).astype(np.float64) * 2.0**-53
    u2 = (splitmix_at(key, p + np.uint64(1)) >> np.uint64(11)).astype(np.float64) * 2.0**-53
    r = np.sqrt(-2.0 * np.log(1.0 - u1))
    t = 6.283185307179586 * u2
    return np.where((i & np.uint64(1)) == 1, r * np.sin(t), r * np.cos(t))


def normal32(n: int, name: str, std: float = 1.0, seed: int = 0, first: int = 0) -> np.ndarray:
    return (normal64(n, name, seed, first) * np.float64(np.float32(std))).astype(np.float32)


def normal16(n: int, name: str, std: float = 1.0, seed: int = 0) -> np.ndarray:
    return normal32(n, name, std, seed).astype(np.float16)


def mxfp4_uniform(rows: int, k: int, name: str, seed: int = 0, emin: int = -4, emax: int = 2):
    w = bytes_(rows * (k // 2), name + ".blocks", seed).reshape(rows, k // 2)
    e = (uniform_int(rows * (k // 32), 127 + emin, emax - emin + 1, name + ".scales", seed)
         .astype(np.uint8).reshape(rows, k // 32))
    return w, e
