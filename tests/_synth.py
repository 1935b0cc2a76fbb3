"""Seeded synthetic inputs shared by the golden-vector script and the tests.

Every tensor is drawn from numpy's PCG64 generator keyed by (seed, tag), so a
test can regenerate exactly the inputs a fixture was made from; fixtures also
store a SHA-256 of the regenerated inputs, checked before any comparison.
fp16 tensors are IEEE round-to-nearest-even of the fp32 draw (numpy's cast,
pinned to the oracle's own RNE in tests/test_oracle.py).
"""
from __future__ import annotations

import hashlib
import zlib

import numpy as np

SEED = 42  # reference c/Makefile:33 ORACLE_SEED


def rng(seed: int, tag: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(tag.encode())])


def normal(seed: int, tag: str, shape, scale: float = 1.0) -> np.ndarray:
    x = rng(seed, tag).standard_normal(size=shape, dtype=np.float64) * scale
    return x.astype(np.float32)


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def digest(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def outlier_keys(seed: int, tag: str, shape, channels: int = 3, spike: float = 20.0) -> np.ndarray:
    """K ~ N(0,1) plus +-`spike` on a fixed set of `channels` channels per KV head
    (random sign per element), the config-5 stress pattern.  shape = [..., kv, d]."""
    k = normal(seed, tag, shape)
    d = shape[-1]
    kv = shape[-2]
    r = rng(seed, tag + "/outliers")
    for h in range(kv):
        ch = r.choice(d, size=channels, replace=False)
        signs = r.choice(np.array([-1.0, 1.0], dtype=np.float32), size=shape[:-2] + (channels,))
        k[..., h, ch] += spike * signs
    return k
