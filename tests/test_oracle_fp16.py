"""Pins the oracle's IEEE binary16 conversions against numpy's float16 casts (a library routine
implementing IEEE 754 round-to-nearest-even), exhaustively where the domain allows."""
import numpy as np


def test_fp16_to_fp32_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp32_to_fp16_all_halves_and_midpoints(orc):
    # every finite half, the midpoints between neighbours (ties) and one float32 ulp either side
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    v = h.view(np.float16).astype(np.float64)
    nxt = np.append(v[1:], 65520.0)
    mid = ((v + nxt) / 2).astype(np.float32)
    cand = np.concatenate([
        v.astype(np.float32), mid,
        np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)),
    ])
    cand = np.concatenate([cand, -cand])
    got = orc.f32_to_f16(cand)
    want = cand.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_fp32_to_fp16_random_and_specials(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    got = orc.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 2.0**-24, 2.0**-25,
                         2.0**-25 * 1.0000001, 6.1e-5, 5.96e-8], dtype=np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(orc.f32_to_f16(specials), specials.astype(np.float16).view(np.uint16))
    # NaN stays NaN
    assert np.isnan(orc.f16_to_f32(orc.f32_to_f16(np.array([np.nan], dtype=np.float32))))[0]
