"""The host restatement of the synthetic-input generator (oracle/synth.c; the
device side is gp_fill_normal): Philox-4x32-10 against its published
known-answer vectors, each fp32 transform against its closed form, the
Box-Muller composition and element order against an independent float64
computation from the Philox words, offsets, the 16-bit roundings and the
moments of the stream."""
import math

import numpy as np
import pytest

import oracle

# Known-answer vectors of Philox-4x32-10 (Salmon et al., SC 2011; Random123's
# kat_vectors): counter, key, output.
PHILOX_KAT = [
    ([0x00000000] * 4, [0x00000000] * 2, [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(ctr, key, want):
    assert [int(v) for v in oracle.philox4x32_10(ctr, key)] == want


def test_log_unit_closed_form():
    rng = np.random.default_rng(0)
    us = np.concatenate([(np.arange(1, 2 ** 12) * 2.0 ** -12), rng.random(20000) + 2.0 ** -24,
                         [2.0 ** -24, 1.0 - 2.0 ** -24, 1.0, 0.5, 0.70710677, 0.70710683]]).astype(np.float32)
    for u in us:
        got, want = oracle.log_unit(u), math.log(float(u))
        assert abs(got - want) <= 4e-7 * max(1.0, abs(want)), (float(u), got, want)


def test_sqrt_and_sincos_closed_forms():
    for v in np.linspace(0.0, 34.0, 5001, dtype=np.float32):
        assert abs(oracle.sqrt_small(v) - math.sqrt(float(v))) <= 3e-7 * max(1.0, math.sqrt(float(v))), float(v)
    for a in np.linspace(0.0, math.pi / 2, 5001, dtype=np.float32):
        s, c = oracle.sincos_quarter(a)
        assert abs(s - math.sin(float(a))) <= 3e-7 and abs(c - math.cos(float(a))) <= 3e-7, float(a)


def test_box_muller_against_float64():
    """Element 4g + 2p + j is the j-th output (cos, sin) of Box-Muller on words
    (2p, 2p + 1) of Philox counter g under key seed, with u1 = ((x >> 8) + 1) / 2^24
    and u2 = (x >> 8) / 2^24."""
    for seed in (0, 7, 0x123456789ABCDEF):
        n, off = 4000, 13
        got = oracle.normal(n, seed=seed, offset=off)
        key = [seed & 0xFFFFFFFF, seed >> 32]
        for i in range(n):
            e = off + i
            g, r = divmod(e, 4)
            x = oracle.philox4x32_10([g & 0xFFFFFFFF, g >> 32, 0, 0], key)
            p, j = divmod(r, 2)
            u1 = ((int(x[2 * p]) >> 8) + 1) / 2.0 ** 24
            u2 = (int(x[2 * p + 1]) >> 8) / 2.0 ** 24
            rad = math.sqrt(-2.0 * math.log(u1))
            want = rad * (math.cos if j == 0 else math.sin)(2.0 * math.pi * u2)
            assert abs(float(got[i]) - want) <= 2e-6 * max(1.0, abs(want)), (seed, e, float(got[i]), want)


def test_offsets_and_seeds():
    full = oracle.normal(10007, seed=3)
    for off in (0, 1, 2, 3, 4, 5, 999):
        part = oracle.normal(10007 - off, seed=3, offset=off)
        assert np.array_equal(part.view(np.uint32), full[off:].view(np.uint32)), off
    assert not np.array_equal(oracle.normal(64, seed=4), oracle.normal(64, seed=3))


def test_sixteen_bit_roundings():
    z = oracle.normal(200003, seed=11)
    h = oracle.normal(200003, seed=11, dtype="f16")
    assert np.array_equal(h, z.astype(np.float16).view(np.uint16))  # numpy: round to nearest even
    b = oracle.normal(200003, seed=11, dtype="bf16")
    u = z.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(b, want)


def test_moments():
    n = 1 << 22
    z = oracle.normal(n, seed=0).astype(np.float64)
    se = 1.0 / math.sqrt(n)
    assert abs(z.mean()) <= 5 * se
    assert abs(z.var() - 1.0) <= 5 * math.sqrt(2.0) * se
    for k, p in ((1.0, 0.6826894921), (2.0, 0.9544997361), (3.0, 0.9973002039)):
        frac = np.mean(np.abs(z) < k)
        assert abs(frac - p) <= 5 * math.sqrt(p * (1 - p)) * se, (k, frac)
