"""fp16 pack/unpack of the oracle, pinned by IEEE binary16 (numpy) and the reference's own packer."""
import numpy as np
import pytest

import oracle


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    # NaN keeps its payload shifted into the f32 mantissa (ptq_decode.h:66-72)
    nan_h = h[~fin].astype(np.uint32)
    expect = ((nan_h & 0x8000) << 16) | 0x7F800000 | ((nan_h & 0x3FF) << 13)
    assert np.array_equal(got[~fin].view(np.uint32), expect.astype(np.uint32))


def _probe_floats():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=400000, dtype=np.uint64).astype(np.uint32)
    # every f32 exponent, with mantissas at/around the 13-bit rounding boundary (ties and carries)
    ex = np.arange(256, dtype=np.uint32) << 23
    mant = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x2000, 0x3000, 0x7FE000, 0x7FF000, 0x7FFFFF,
                     0x7FEFFF, 0x400000, 0x401000, 0x403000], dtype=np.uint32)
    grid = (ex[:, None] | mant[None, :]).ravel()
    # half-subnormal ties: k * 2^-25 for odd k (exact midpoints between subnormal steps)
    ties = (np.arange(1, 4096, 2, dtype=np.float64) * 2.0**-25).astype(np.float32).view(np.uint32)
    allb = np.concatenate([bits, grid, ties])
    allb = np.concatenate([allb, allb | np.uint32(0x80000000)])
    return allb.view(np.float32)


def test_f32_to_f16_matches_ieee_rne():
    x = _probe_floats()
    got = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    # any NaN -> quiet sign|0x7E00 (f16_rne_host.h:38)
    sign = (x[nan].view(np.uint32) >> 16) & 0x8000
    assert np.array_equal(got[nan], (sign | 0x7E00).astype(np.uint16))


def test_f32_to_f16_special_values():
    cases = [(0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (65504.0, 0x7BFF), (65520.0, 0x7C00),
             (65519.99, 0x7BFF), (2.0**-24, 0x0001), (2.0**-25, 0x0000), (3 * 2.0**-26, 0x0001), (3 * 2.0**-25, 0x0002), (5 * 2.0**-25, 0x0002),
             (float("inf"), 0x7C00), (-float("inf"), 0xFC00), (1e-40, 0x0000), (-1e-40, 0x8000)]
    for v, h in cases:
        assert oracle.lib().bko_f32_to_f16(v) == h, (v, hex(h))


def test_f16_against_reference_packer():
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    x = _probe_floats()[::7]
    got = oracle.f32_to_f16(x)
    want = np.array([R.ref_f32_to_f16_bits(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)
    h = np.arange(0, 65536, 3, dtype=np.uint32).astype(np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]          # NaN payloads do not survive ctypes' float return
    g2 = oracle.f16_to_f32(h)
    w2 = np.array([R.ref_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    assert np.array_equal(g2.view(np.uint32), w2.view(np.uint32))
