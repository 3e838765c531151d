"""Pins the oracle's ggml block formats, *_ref quantizers and dequantizers.

The reference holds no golden vectors (it ships no tests and does not vendor ggml), so the checks
here are (a) known answers derived by hand from the block definitions (byte positions, nibble
order, qh bit order, code offsets), (b) invariants of the _ref quantizers that a dropped term,
wrong sign or swapped nibble would break, (c) an independent vectorised unpacker of the
documented layout over every fp16 scale, and (d) the committed fixture tests/golden/blocks.npz.
"""
import os

import numpy as np
import pytest

from _ties import tie_cases, tie_q8_0_cpu_case
from oracle.oracle import F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, QUANT_TYPES, TYPE_BYTES

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def h(x):
    return int(np.float16(x).view(np.uint16))


def half_bytes(x):
    v = h(x)
    return [v & 0xFF, v >> 8]


# ------------------------------------------------------------------------------------------
# (a) known answers from the layout definitions
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("j", [0, 5, 15, 16, 21, 31])
def test_quantize_single_spike_known_bytes(orc, j):
    x = np.zeros(32, dtype=np.float32)
    x[j] = 1.0
    # q8_0: d = 1/127, spike -> +127, everything else 0
    b = orc.quantize_flat(Q8_0, x)
    assert list(b[:2]) == half_bytes(np.float32(1.0) / np.float32(127.0))
    want = [0] * 32
    want[j] = 127
    assert list(b[2:].view(np.int8)) == want
    # q4_0: max = +1 -> d = -1/8; spike code (int8)(-8+8.5)=0, others (int8)(8.5)=8
    b = orc.quantize_flat(Q4_0, x)
    assert list(b[:2]) == half_bytes(-0.125)
    qs = [0x88] * 16
    qs[j % 16] = 0x80 if j < 16 else 0x08
    assert list(b[2:]) == qs
    # q5_0: d = -1/16; spike code 0, others 16 = nibble 0 with the high bit set
    b = orc.quantize_flat(Q5_0, x)
    assert list(b[:2]) == half_bytes(-0.0625)
    qh = int.from_bytes(bytes(b[2:6]), "little")
    assert qh == (0xFFFFFFFF & ~(1 << j))
    assert list(b[6:]) == [0] * 16
    # q4_1: min 0, max 1 -> d = 1/15, m = 0; spike code 15
    b = orc.quantize_flat(Q4_1, x)
    assert list(b[:2]) == half_bytes(np.float32(1.0) / np.float32(15.0))
    assert list(b[2:4]) == [0, 0]
    qs = [0] * 16
    qs[j % 16] = 0x0F if j < 16 else 0xF0
    assert list(b[4:]) == qs
    # q5_1: d = 1/31, spike code 31 = nibble 15 + high bit j
    b = orc.quantize_flat(Q5_1, x)
    assert list(b[:2]) == half_bytes(np.float32(1.0) / np.float32(31.0))
    assert list(b[2:4]) == [0, 0]
    assert int.from_bytes(bytes(b[4:8]), "little") == (1 << j)
    qs = [0] * 16
    qs[j % 16] = 0x0F if j < 16 else 0xF0
    assert list(b[8:]) == qs


def test_zero_block_scales_keep_ieee_sign(orc):
    """0 / -8 and 0 / -16 are -0.0 in IEEE arithmetic, so all-zero q4_0/q5_0 blocks store d = -0."""
    x = np.zeros(32, dtype=np.float32)
    assert list(orc.quantize_flat(Q4_0, x)[:2]) == [0x00, 0x80]
    assert list(orc.quantize_flat(Q5_0, x)[:2]) == [0x00, 0x80]
    assert list(orc.quantize_flat(Q8_0, x)[:2]) == [0x00, 0x00]  # 0 / 127 = +0
    assert list(orc.quantize_flat(Q4_1, x)[:4]) == [0, 0, 0, 0]


def test_quantize_negative_spike_and_sign_of_d(orc):
    x = np.zeros(32, dtype=np.float32)
    x[3] = -2.0
    b = orc.quantize_flat(Q4_0, x)
    assert list(b[:2]) == half_bytes(0.25)  # d = max/-8 with max = -2
    assert b[2 + 3] & 0x0F == 0  # the max-|x| element maps to code 0 (value -8*d = -2)
    b = orc.quantize_flat(Q8_0, x)
    assert b[2 + 3].view(np.int8) == -127


def _hand_blocks():
    """Hand-built blocks with hand-computed dequantized values."""
    ks = np.arange(16)
    qs = (ks | ((15 - ks) << 4)).astype(np.uint8)
    qh_bits = 0xAAAAAAAA  # odd element indices carry the 5th bit
    out = {}
    # q8_0: d = 0.5, qs[j] = j-16
    b = bytes(half_bytes(0.5)) + bytes(((np.arange(32) - 16).astype(np.int8)).view(np.uint8))
    out[Q8_0] = (b, (np.arange(32) - 16) * 0.5)
    # q4_0: d = 0.25: y[k] = (k-8)/4, y[k+16] = (7-k)/4
    b = bytes(half_bytes(0.25)) + bytes(qs)
    out[Q4_0] = (b, np.concatenate([(ks - 8) * 0.25, (7 - ks) * 0.25]))
    # q4_1: d = 0.5, m = -1: y[k] = k/2 - 1, y[k+16] = (15-k)/2 - 1
    b = bytes(half_bytes(0.5) + half_bytes(-1.0)) + bytes(qs)
    out[Q4_1] = (b, np.concatenate([ks * 0.5 - 1, (15 - ks) * 0.5 - 1]))
    code_lo = ks + 16 * (ks & 1)
    code_hi = (15 - ks) + 16 * (ks & 1)
    # q5_0: d = 1: y = code - 16
    b = bytes(half_bytes(1.0)) + qh_bits.to_bytes(4, "little") + bytes(qs)
    out[Q5_0] = (b, np.concatenate([code_lo - 16, code_hi - 16]).astype(np.float64))
    # q5_1: d = 0.5, m = 2: y = code/2 + 2
    b = bytes(half_bytes(0.5) + half_bytes(2.0)) + qh_bits.to_bytes(4, "little") + bytes(qs)
    out[Q5_1] = (b, np.concatenate([code_lo * 0.5 + 2, code_hi * 0.5 + 2]))
    return out


@pytest.mark.parametrize("t", QUANT_TYPES)
def test_dequantize_hand_blocks(orc, t):
    b, want = _hand_blocks()[t]
    assert len(b) == TYPE_BYTES[t]
    got = orc.dequantize(t, np.frombuffer(b, dtype=np.uint8), 32)
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("t", QUANT_TYPES)
def test_quantize_exact_ties_known_codes(orc, t):
    """Inputs on exact rounding ties (|id| = 1): the codes of each *_ref tie rule, written out by
    hand in tests/_ties.py.  The |x - deq| <= d/2 invariants below hold under any tie rule; these
    do not (rint instead of roundf, or roundf instead of the +0.5 truncation, changes them)."""
    for x, want in tie_cases()[t]:
        got = orc.quantize_flat(t, x)
        assert list(got) == list(want), (t, list(got), list(want))


def test_cpu_q8_0_variant_ties_to_even(orc):
    x, want = tie_q8_0_cpu_case()
    assert list(orc.quantize_q8_0_cpu(x)) == list(want)


# ------------------------------------------------------------------------------------------
# (b) invariants of the _ref quantizers on random blocks
# ------------------------------------------------------------------------------------------
def _random_blocks(rng, n=4000):
    x = rng.standard_normal((n, 32)).astype(np.float32)
    scale = np.exp(rng.uniform(-8, 8, size=(n, 1))).astype(np.float32)
    x = x * scale
    x[::17] = np.round(x[::17] * 2) / 2  # ties
    return x


def _codes(t, b):
    """Unsigned codes of each element (independent numpy unpacker of the documented layout)."""
    n = b.shape[0]
    if t == Q8_0:
        return b[:, 2:34].view(np.int8).astype(np.int32)
    qs_off = {Q4_0: 2, Q4_1: 4, Q5_0: 6, Q5_1: 8}[t]
    qs = b[:, qs_off:qs_off + 16].astype(np.int32)
    code = np.concatenate([qs & 15, qs >> 4], axis=1)
    if t in (Q5_0, Q5_1):
        qh_off = 2 if t == Q5_0 else 4
        qh = b[:, qh_off:qh_off + 4].copy().view("<u4").reshape(n).astype(np.int64)
        bits = (qh[:, None] >> np.arange(32)[None, :]) & 1
        code = code | (bits.astype(np.int32) << 4)
    return code


def _f16(b, off):
    return b[:, off:off + 2].copy().view(np.float16).reshape(-1).astype(np.float32)


def test_q8_0_invariants(orc, rng):
    x = _random_blocks(rng)
    b = orc.quantize(Q8_0, x)
    c = _codes(Q8_0, b)
    amax = np.abs(x).max(axis=1)
    d32 = amax / np.float32(127)
    assert np.array_equal(_f16(b, 0), d32.astype(np.float16).astype(np.float32))
    assert c.min() >= -127 and c.max() <= 127
    am = np.abs(x).argmax(axis=1)
    nz = amax > 0  # an all-zero block has d = 0 and all codes 0
    assert np.all(c[~nz] == 0)
    assert np.array_equal(np.abs(c[np.arange(len(x)), am])[nz], np.full(int(nz.sum()), 127))
    assert np.all(np.sign(c) * np.sign(x) >= 0)
    err = np.abs(x - c * d32[:, None])
    assert np.all(err <= d32[:, None] * 0.5 * (1 + 1e-5) + 1e-30)


@pytest.mark.parametrize("t,levels,off", [(Q4_0, 8, 8), (Q5_0, 16, 16)])
def test_symmetric_4_5_bit_invariants(orc, rng, t, levels, off):
    x = _random_blocks(rng)
    b = orc.quantize(t, x)
    c = _codes(t, b)
    am = np.abs(x).argmax(axis=1)  # first maximum, like the reference loop
    mx = x[np.arange(len(x)), am]
    d32 = mx / np.float32(-levels)
    assert np.array_equal(_f16(b, 0), d32.astype(np.float16).astype(np.float32))
    nz = mx != 0
    assert np.array_equal(c[np.arange(len(x)), am][nz], np.zeros(int(nz.sum()), dtype=np.int32))
    assert np.all(c[~nz] == off)
    assert c.min() >= 0 and c.max() <= 2 * levels - 1
    val = (c - off) * d32[:, None]
    err = np.abs(x - val)
    # the top code saturates (x*id + off >= 2*levels happens only on the side opposite the max)
    clamped = c == 2 * levels - 1
    bound = np.broadcast_to(np.abs(d32)[:, None], err.shape)
    assert np.all((err <= bound * 0.5 * (1 + 1e-5) + 1e-30) | clamped)
    assert np.all(err[clamped] <= bound[clamped] * (1 + 1e-5))


@pytest.mark.parametrize("t,levels", [(Q4_1, 15), (Q5_1, 31)])
def test_affine_4_5_bit_invariants(orc, rng, t, levels):
    x = _random_blocks(rng)
    b = orc.quantize(t, x)
    c = _codes(t, b)
    mn, mxv = x.min(axis=1), x.max(axis=1)
    d32 = (mxv - mn) / np.float32(levels)
    assert np.array_equal(_f16(b, 0), d32.astype(np.float16).astype(np.float32))
    assert np.array_equal(_f16(b, 2), mn.astype(np.float16).astype(np.float32))
    assert c.min() >= 0 and c.max() <= levels
    r = np.arange(len(x))
    nz = mxv > mn
    assert np.all(c[r, x.argmin(axis=1)] == 0)
    assert np.all(c[r, x.argmax(axis=1)][nz] == levels)
    err = np.abs(x - (c * d32[:, None] + mn[:, None]))
    assert np.all(err <= d32[:, None] * 0.5 * (1 + 1e-4) + np.abs(mn)[:, None] * 1e-6 + 1e-30)


def test_cpu_q8_0_variant_within_one_code(orc, rng):
    x = _random_blocks(rng, 2000)
    ref = _codes(Q8_0, orc.quantize(Q8_0, x))
    cpu = np.stack([_codes(Q8_0, orc.quantize_q8_0_cpu(x[i])[None, :])[0] for i in range(len(x))])
    assert np.abs(ref - cpu).max() <= 1


# ------------------------------------------------------------------------------------------
# (c) every fp16 scale: the oracle's dequantizer vs an independent vectorised unpacker
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("t", QUANT_TYPES)
def test_dequantize_every_scale(orc, t):
    rng = np.random.default_rng(t)
    d_all = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    n = d_all.size
    tb = TYPE_BYTES[t]
    b = rng.integers(0, 256, size=(n, tb), dtype=np.uint8)
    b[:, 0] = (d_all & 0xFF).astype(np.uint8)
    b[:, 1] = (d_all >> 8).astype(np.uint8)
    if t in (Q4_1, Q5_1):  # m: every half as well, in another order
        m_all = np.roll(d_all, 12345)
        b[:, 2] = (m_all & 0xFF).astype(np.uint8)
        b[:, 3] = (m_all >> 8).astype(np.uint8)
    d = d_all.view(np.float16).astype(np.float32)
    c = _codes(t, b)
    with np.errstate(invalid="ignore", over="ignore"):
        if t in (Q4_1, Q5_1):
            m = np.roll(d_all, 12345).view(np.float16).astype(np.float32)
            want = c.astype(np.float32) * d[:, None] + m[:, None]
        else:
            off = {Q8_0: 0, Q4_0: 8, Q5_0: 16}[t]
            want = (c - off).astype(np.float32) * d[:, None]
    got = orc.dequantize(t, b.ravel(), n * 32).reshape(n, 32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_rows_roundtrip(orc, rng):
    x = rng.standard_normal(4096).astype(np.float32)
    b = orc.quantize_flat(F16, x)
    assert np.array_equal(b.view(np.uint16), x.astype(np.float16).view(np.uint16))
    assert np.array_equal(orc.dequantize(F16, b, x.size), x.astype(np.float16).astype(np.float32))


# ------------------------------------------------------------------------------------------
# (d) committed fixture
# ------------------------------------------------------------------------------------------
def test_golden_blocks(orc):
    g = np.load(os.path.join(GOLDEN, "blocks.npz"))
    x = g["x"]
    for t in QUANT_TYPES:
        b = orc.quantize(t, x)
        assert np.array_equal(b, g[f"bytes_{t}"]), t
        deq = np.stack([orc.dequantize(t, b[i], 32) for i in range(len(x))])
        assert np.array_equal(deq.view(np.uint32), g[f"deq_{t}"].view(np.uint32)), t
