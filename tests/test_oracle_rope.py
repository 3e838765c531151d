"""Pins of the oracle's ggml_rope_ext restatement (or_rope_f32), CPU only.

The callers rotate Q and K before attention: NEOX over each 64-dim head with the GGUF theta
(src/cosyvoice-llm.cpp:56-57) and NORMAL over the first 64 dims of a 1024-wide row with base
10000 (src/cosyvoice-graph.cpp:351-352).  Each check below fails for a plausible slip in the
restatement (wrong pairing, sign of the sine term, angle index or base, touched tail dims).
"""
import ctypes
import ctypes.util
import math

import numpy as np
import pytest

from oracle.oracle import ROPE_NEOX, ROPE_NORMAL

MODES = [ROPE_NORMAL, ROPE_NEOX]

# the C library's powf (numpy's float32 power can differ from it in the last bit, and ggml's CPU
# rope takes theta_scale from powf)
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def theta_scale(base, n_dims):
    return np.float32(_libm.powf(np.float32(base), np.float32(-2.0) / np.float32(n_dims)))


def f32_angles(p, n_dims, base, scale=1.0):
    """theta_k as float32 arithmetic produces it: p, then times powf(base, -2/n) per pair."""
    ts = theta_scale(base, n_dims)
    th = np.float32(p)
    out = []
    for _ in range(n_dims // 2):
        out.append(np.float32(np.float32(scale) * th))
        th = np.float32(th * ts)
    return np.array(out, dtype=np.float32)


def pairs(mode, n_dims):
    half = n_dims // 2
    if mode == ROPE_NEOX:
        return [(k, k + half) for k in range(half)]
    return [(2 * k, 2 * k + 1) for k in range(half)]


@pytest.mark.parametrize("mode", MODES)
def test_position_zero_is_identity(orc, rng, mode):
    x = rng.standard_normal((5, 64)).astype(np.float32)
    y = orc.rope(x, np.zeros(5, np.int32), 64, mode, 1e6)
    assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("mode", MODES)
def test_known_answer_unit_vector(orc, mode):
    # one pair: x = (1, 0) at p = 1 rotates to (cos 1, sin 1) -- the sign convention
    x = np.array([[1.0, 0.0]], dtype=np.float32)
    y = orc.rope(x, [1], 2, mode, 10000.0)
    assert abs(float(y[0, 0]) - math.cos(1.0)) < 1e-7
    assert abs(float(y[0, 1]) - math.sin(1.0)) < 1e-7
    # x = (0, 1) rotates to (-sin 1, cos 1)
    y = orc.rope(np.array([[0.0, 1.0]], np.float32), [1], 2, mode, 10000.0)
    assert abs(float(y[0, 0]) + math.sin(1.0)) < 1e-7
    assert abs(float(y[0, 1]) - math.cos(1.0)) < 1e-7


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("base,n_dims,ne0", [(1e6, 64, 64), (10000.0, 64, 1024), (10000.0, 32, 96)])
def test_float64_rotation_by_float32_angles(orc, rng, mode, base, n_dims, ne0):
    pos = np.array([0, 1, 2, 7, 100, 1023, 4095, 8191], np.int32)
    x = rng.standard_normal((len(pos), ne0)).astype(np.float32)
    y = orc.rope(x, pos, n_dims, mode, base)
    for r, p in enumerate(pos):
        th = f32_angles(int(p), n_dims, base).astype(np.float64)
        for k, (a, b) in enumerate(pairs(mode, n_dims)):
            c, s = math.cos(th[k]), math.sin(th[k])
            x0, x1 = float(x[r, a]), float(x[r, b])
            # cosf/sinf are within an ulp; products and the sum round once each
            tol = 4e-7 * (abs(x0) + abs(x1)) + 1e-12
            assert abs(float(y[r, a]) - (x0 * c - x1 * s)) <= tol
            assert abs(float(y[r, b]) - (x0 * s + x1 * c)) <= tol
        # dims from n_dims on are copied bit for bit
        assert np.array_equal(x[r, n_dims:].view(np.uint32), y[r, n_dims:].view(np.uint32))


@pytest.mark.parametrize("base,n_dims", [(1e6, 64), (10000.0, 64), (500000.0, 128)])
def test_angles_against_closed_form(base, n_dims):
    # the iterated float32 angle stays within k+1 roundings of p * base^(-2k/n)
    for p in (1, 3, 4096, 8191):
        th = f32_angles(p, n_dims, base).astype(np.float64)
        for k in range(n_dims // 2):
            exact = p * base ** (-2.0 * k / n_dims)
            assert abs(th[k] - exact) <= (k + 2) * 2.0 ** -23 * exact


@pytest.mark.parametrize("mode", MODES)
def test_pair_norms_preserved(orc, rng, mode):
    pos = rng.integers(0, 8192, 16).astype(np.int32)
    x = rng.standard_normal((16, 64)).astype(np.float32)
    y = orc.rope(x, pos, 64, mode, 1e6).astype(np.float64)
    x = x.astype(np.float64)
    for a, b in pairs(mode, 64):
        nx = np.hypot(x[:, a], x[:, b])
        ny = np.hypot(y[:, a], y[:, b])
        assert np.all(np.abs(nx - ny) <= 1e-6 * (1 + nx))


@pytest.mark.parametrize("mode", MODES)
def test_scores_depend_on_position_difference(orc, rng, mode):
    q = rng.standard_normal(64).astype(np.float32)
    k = rng.standard_normal(64).astype(np.float32)
    base = 10000.0
    for p1, p2 in ((5, 2), (40, 33), (100, 0)):
        ref = None
        for d in (0, 1, 17, 250):
            qa = orc.rope(q[None], [p1 + d], 64, mode, base)[0].astype(np.float64)
            ka = orc.rope(k[None], [p2 + d], 64, mode, base)[0].astype(np.float64)
            s = float(qa @ ka)
            if ref is None:
                ref = s
            assert abs(s - ref) <= 2e-4 * (1 + abs(ref))


def test_neox_is_normal_under_pairing_permutation(orc, rng):
    # NEOX pairs (k, k+n/2); NORMAL pairs (2k, 2k+1): permuting dims maps one onto the other
    n = 64
    perm = np.empty(n, np.int64)
    perm[0::2] = np.arange(n // 2)
    perm[1::2] = np.arange(n // 2) + n // 2
    pos = rng.integers(0, 8192, 9).astype(np.int32)
    x = rng.standard_normal((9, n)).astype(np.float32)
    y_neox = orc.rope(x, pos, n, ROPE_NEOX, 1e6)
    y_norm = orc.rope(x[:, perm], pos, n, ROPE_NORMAL, 1e6)
    assert np.array_equal(y_neox[:, perm].view(np.uint32), y_norm.view(np.uint32))


def test_freq_scale_scales_angles(orc, rng):
    # freq_scale multiplies every angle: scale 0.5 at position 2p equals scale 1 at p
    x = rng.standard_normal((4, 64)).astype(np.float32)
    pos = np.array([2, 10, 64, 300], np.int32)
    a = orc.rope(x, pos, 64, ROPE_NORMAL, 10000.0, 0.5)
    b = orc.rope(x, pos // 2, 64, ROPE_NORMAL, 10000.0, 1.0)
    assert np.max(np.abs(a - b)) < 2e-5


def test_rejects_bad_arguments(orc):
    x = np.zeros((1, 64), np.float32)
    for n_dims, mode in ((63, ROPE_NORMAL), (66, ROPE_NORMAL), (64, 1)):
        with pytest.raises(ValueError):
            orc.rope(x, [0], n_dims, mode, 10000.0)
