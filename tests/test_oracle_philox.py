"""CPU: the numpy weight generator (oracle/philox.py) against published known
answers and the properties its construction fixes.

* Philox4x32-10: the Random123 known-answer vectors (kat_vectors, "philox4x32
  10" lines: zero counter/key, all-ones, and the pi-digit counter/key).
* FNV-1a 64: the published test vectors of the hash ("", "a", "foobar").
* f32 -> bf16: torch's own conversion (an independent implementation),
  including exact ties, infinities and NaN.
* normal_bf16_bits: each (cos, sin) pair satisfies z0^2 + z1^2 = -2 ln u1 with
  u1 from the Philox word it was built from; an odd start offset selects the
  same elements as the full tensor; a large draw has mean 0 / std `std` and
  passes a Kolmogorov-Smirnov test against N(0, std).
"""

import math

import numpy as np
import pytest
import torch
from scipy import stats

from oracle import philox

KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expect", KAT)
def test_philox_known_answers(ctr, key, expect):
    got = philox.philox4x32_10(*[np.array([c], np.uint32) for c in ctr], key[0], key[1])
    assert tuple(int(w[0]) for w in got) == expect


def test_philox_vectorised_equals_scalar_calls():
    rng = np.random.default_rng(7)
    c = rng.integers(0, 2**32, size=(4, 16), dtype=np.uint64).astype(np.uint32)
    vec = philox.philox4x32_10(c[0], c[1], c[2], c[3], 0x1234, 0x5678)
    for i in range(16):
        one = philox.philox4x32_10(c[0, i:i + 1], c[1, i:i + 1], c[2, i:i + 1], c[3, i:i + 1], 0x1234, 0x5678)
        assert all(int(v[i]) == int(o[0]) for v, o in zip(vec, one))


@pytest.mark.parametrize("text,expect", [("", 0xCBF29CE484222325), ("a", 0xAF63DC4C8601EC8C),
                                         ("foobar", 0x85944171F73967E8)])
def test_fnv1a64_published_vectors(text, expect):
    assert philox.fnv1a64(text.encode()) == expect


def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 20000),
        np.array([1.0, 1.00390625, 1.01171875, -2.5, 0.0, -0.0, np.inf, -np.inf, 3.0e38, 1e-40], np.float32),
    ]).astype(np.float32)
    got = philox.f32_to_bf16_bits(x)
    exp = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, exp)
    # exact ties go to even: 1 + 2^-8 -> 1.0 (0x3F80), 1 + 3*2^-8 -> 1 + 2^-6 (0x3F82)
    assert philox.f32_to_bf16_bits(np.array([1.00390625, 1.01171875], np.float32)).tolist() == [0x3F80, 0x3F82]
    nan = philox.f32_to_bf16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_bf16_round_trip_is_identity_on_bf16_values():
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7F80) != 0x7F80
    f = philox.bf16_bits_to_f32(bits[finite])
    assert np.array_equal(philox.f32_to_bf16_bits(f), bits[finite])


def test_normal_pairs_follow_box_muller_radius():
    key = philox.tensor_key(3, "layers.0.q_proj")
    n = 4096
    z = philox.bf16_bits_to_f32(philox.normal_bf16_bits(n, key, 1.0)).astype(np.float64)
    j = np.arange(n // 2, dtype=np.uint64)
    w0, _, _, _ = philox.philox4x32_10(j.astype(np.uint32), np.zeros(n // 2, np.uint32), 0, 0,
                                       key & 0xFFFFFFFF, key >> 32)
    u1 = (w0.astype(np.float64) + 1.0) / 2.0**32
    r2 = z[0::2] ** 2 + z[1::2] ** 2
    # each z is one bf16 rounding (relative 2^-9) away from the exact value
    assert np.all(np.abs(r2 - (-2.0 * np.log(u1))) <= 2.0 ** -7 * (-2.0 * np.log(u1)) + 1e-30)


def test_normal_offset_window_matches_full_tensor():
    key = philox.tensor_key(0, "embed")
    full = philox.normal_bf16_bits(1001, key, 0.02)
    for start, n in ((0, 10), (1, 10), (7, 33), (500, 501), (999, 2)):
        assert np.array_equal(philox.normal_bf16_bits(n, key, 0.02, start=start), full[start:start + n])
    assert philox.normal_bf16_bits(0, key, 0.02).size == 0


def test_normal_distribution():
    z = philox.bf16_bits_to_f32(philox.normal_bf16_bits(200000, philox.tensor_key(1, "x"), 0.02)).astype(np.float64)
    assert abs(z.mean()) < 0.02 * 5 / math.sqrt(z.size)
    assert abs(z.std() / 0.02 - 1.0) < 0.01
    assert stats.kstest(z / 0.02, "norm").pvalue > 1e-3


def test_tensor_keys_differ_by_name_and_seed():
    keys = {philox.tensor_key(s, n) for s in (0, 1, 3) for n in ("embed", "norm", "layers.0.q_proj")}
    assert len(keys) == 9
    assert philox.tensor_key(0, "embed") == philox.fnv1a64(b"embed")
