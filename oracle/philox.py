"""numpy restatement of the weight generator — TEST INFRASTRUCTURE ONLY.

Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy
as 1, 2, 3", SC'11): 10 rounds of the 4x32 Philox S-box with multipliers
0xD2511F53 / 0xCD9E8D57 and Weyl key increments 0x9E3779B9 / 0xBB67AE85.
Pinned by the Random123 known-answer vectors in tests/test_oracle_philox.py.

Element i of a tensor uses block counter (i//2, 0, 0) under the tensor key;
words 0 and 1 give u1 = (w0+1)/2^32 in (0,1] and u2 = w1/2^32 in [0,1); the
Box-Muller pair sqrt(-2 ln u1) * (cos, sin)(2 pi u2) is evaluated in f64; the
even element takes the cosine branch.  value = bf16(f32(std * z)).
"""

from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(c0, c1, c2, c3, k0: int, k1: int):
    """Vectorised Philox4x32-10 over uint32 arrays; returns four uint32 arrays."""
    c0 = np.asarray(c0, np.uint32).copy()
    c1 = np.asarray(c1, np.uint32).copy()
    c2 = np.asarray(c2, np.uint32).copy()
    c3 = np.asarray(c3, np.uint32).copy()
    key0 = np.uint32(k0)
    key1 = np.uint32(k1)
    with np.errstate(over="ignore"):
        for r in range(10):
            if r:
                key0 = np.uint32(key0 + W0)
                key1 = np.uint32(key1 + W1)
            p0 = M0 * c0.astype(np.uint64)
            p1 = M1 * c2.astype(np.uint64)
            hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
            lo0 = (p0 & MASK32).astype(np.uint32)
            hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
            lo1 = (p1 & MASK32).astype(np.uint32)
            c0, c1, c2, c3 = hi1 ^ c1 ^ key0, lo1, hi0 ^ c3 ^ key1, lo0
    return c0, c1, c2, c3


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & np.uint64(0x7FFFFFFF)) > np.uint64(0x7F800000)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    r = np.where(nan, (u >> np.uint64(16)) | np.uint64(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16_bits(n: int, key: int, std: float, start: int = 0) -> np.ndarray:
    """bf16 bit patterns of elements [start, start+n) of a tensor with this key."""
    if n == 0:
        return np.zeros(0, np.uint16)
    first_pair = start // 2
    last_pair = (start + n - 1) // 2
    j = np.arange(first_pair, last_pair + 1, dtype=np.uint64)
    w0, w1, _, _ = philox4x32_10(
        (j & MASK32).astype(np.uint32), (j >> np.uint64(32)).astype(np.uint32), 0, 0,
        key & 0xFFFFFFFF, (key >> 32) & 0xFFFFFFFF,
    )
    u1 = (w0.astype(np.float64) + 1.0) / 4294967296.0
    u2 = w1.astype(np.float64) / 4294967296.0
    rad = np.sqrt(-2.0 * np.log(u1))
    ang = 6.283185307179586476925286766559 * u2
    z = np.empty(2 * len(j), np.float64)
    z[0::2] = rad * np.cos(ang)
    z[1::2] = rad * np.sin(ang)
    off = start - 2 * first_pair
    vals = (float(std) * z[off : off + n]).astype(np.float32)
    return f32_to_bf16_bits(vals)


def fnv1a64(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_key(seed: int, name: str) -> int:
    """64-bit Philox key of one named tensor under a model seed."""
    return fnv1a64(name.encode()) ^ ((seed * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)
