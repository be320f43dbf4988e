"""Test infrastructure (the oracle): a numpy restatement of Philox4x32-10.

J. K. Salmon, M. A. Moraes, R. O. Dror, D. E. Shaw, "Parallel Random Numbers: As Easy
as 1, 2, 3", SC 2011: ten rounds of
    (hi0, lo0) = mulhilo(0xD2511F53, c0); (hi1, lo1) = mulhilo(0xCD9E8D57, c2)
    c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0); k += (0x9E3779B9, 0xBB67AE85)
with the key bumped between rounds.  ``seeded_uniform`` is the sampler's use of it: the
counter (step low, step high, 0x4E53534D, 0) under the key (seed low, seed high), first
output word >> 8, times 2^-24.  Pinned by the generator's published known-answer vectors
and by rocRAND's engine (tests/test_philox.py); only tests import this module.
"""
from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
TAG = 0x4E53534D
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr, key):
    """Vectorised: ctr (..., 4) and key (..., 2) uint32 arrays -> (..., 4) uint32."""
    c = np.asarray(ctr, dtype=np.uint32).copy()
    k = np.asarray(key, dtype=np.uint32).copy()
    c0, c1, c2, c3 = (c[..., i].astype(np.uint64) for i in range(4))
    k0, k1 = k[..., 0].astype(np.uint64), k[..., 1].astype(np.uint64)
    for r in range(10):
        p0 = M0 * c0
        p1 = M1 * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK32
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
        if r < 9:
            k0 = (k0 + np.uint64(W0)) & MASK32
            k1 = (k1 + np.uint64(W1)) & MASK32
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def seeded_uniform(seeds, steps):
    """float32 uniforms of the sampler's seeded rows (see the module docstring)."""
    seeds = [seeds] if isinstance(seeds, (int, np.integer)) else list(seeds)   # Python ints: no float detour
    steps = [steps] if isinstance(steps, (int, np.integer)) else list(steps)
    s = np.array([int(x) & 0xFFFFFFFFFFFFFFFF for x in seeds], dtype=np.uint64)
    t = np.array([int(x) for x in steps], dtype=np.int64).astype(np.uint64)
    ctr = np.stack([t & MASK32, t >> np.uint64(32), np.full_like(t, TAG), np.zeros_like(t)], axis=-1)
    key = np.stack([s & MASK32, s >> np.uint64(32)], axis=-1)
    x0 = philox4x32_10(ctr.astype(np.uint32), key.astype(np.uint32))[..., 0]
    return ((x0 >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)
