"""Synthetic inputs and weights: one documented counter-based generator.

The reference seeds ``System.Random``, which cannot be reproduced outside .NET, so every tensor of
the benchmark configurations comes from this generator instead (the same definition is used by the
tests, the benchmark and the CPU baseline):

  word(seed, tensor_id, i) = mix(mix(seed * G + tensor_id) + (i + 1) * G)
      mix = SplitMix64's finaliser, G = 0x9E3779B97F4A7C15 (Steele et al., 2014)
  uniform(a, b)[i]  = a + (b - a) * (word >> 40) / 2^24                       (top 24 bits)
  normal(0, s)[i]   = s * sqrt(-2 ln u1) * cos(2 pi u2), Box-Muller in float64, with
                      u1 = ((word(2i) >> 11) + 1) / 2^53, u2 = (word(2i+1) >> 11) / 2^53
  all cast to float32 at the end.
"""
from __future__ import annotations

import hashlib

import numpy as np

_G = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def words(seed: int, tensor_id: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        key = _mix(np.array([(seed * 0x9E3779B97F4A7C15 + tensor_id) & 0xFFFFFFFFFFFFFFFF], np.uint64))[0]
        i = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(key + i * _G)


def uniform(seed: int, tensor_id: int, shape, a: float, b: float) -> np.ndarray:
    n = int(np.prod(shape))
    w = words(seed, tensor_id, n)
    u = (w >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    return (a + (b - a) * u).astype(np.float32).reshape(shape)


def normal(seed: int, tensor_id: int, shape, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    w = words(seed, tensor_id, 2 * n)
    u1 = ((w[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) / float(1 << 53)
    u2 = (w[1::2] >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (std * z).astype(np.float32).reshape(shape)


def he_normal(seed: int, tensor_id: int, shape) -> np.ndarray:
    """He-normal weights N(0, sqrt(2 / fan_in)) for an ONNX conv / gemm weight."""
    fan_in = int(np.prod(shape[1:])) if len(shape) == 4 else int(shape[0])
    return normal(seed, tensor_id, shape, float(np.sqrt(2.0 / fan_in)))


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()
