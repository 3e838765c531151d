"""GPU parity of the block formats: the in-register dequantizer the attention kernels use
(cvattn_dequantize) and the quantize-on-write KV update (cvattn_set_rows) against the oracle,
bit for bit."""
import os

import numpy as np
import pytest
import torch

import cvattn
from _gpu import dev, host
from _ties import tie_cases
from oracle.oracle import F16, F32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, QUANT_TYPES, TYPE_BYTES, row_bytes

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def gpu_dequant(eng, t, b: np.ndarray, n: int) -> np.ndarray:
    src = dev(b)
    out = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda:0")
    rc = eng.dequantize(t, src.data_ptr(), out.data_ptr(), n)
    assert rc == cvattn.OK
    return host(out)


def same_bits(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.mark.parametrize("t", QUANT_TYPES)
def test_dequant_every_fp16_scale_bit_exact(eng, orc, t, cuda):
    rng = np.random.default_rng(100 + t)
    n = 65536
    b = rng.integers(0, 256, size=(n, TYPE_BYTES[t]), dtype=np.uint8)
    d_all = np.arange(n, dtype=np.uint32).astype(np.uint16)
    b[:, 0] = (d_all & 0xFF).astype(np.uint8)
    b[:, 1] = (d_all >> 8).astype(np.uint8)
    got = gpu_dequant(eng, t, b.ravel(), n * 32)
    want = orc.dequantize(t, b.ravel(), n * 32)
    assert same_bits(got, want)


def test_dequant_golden_blocks(eng, orc, cuda):
    g = np.load(os.path.join(GOLDEN, "blocks.npz"))
    for t in QUANT_TYPES:
        b = g[f"bytes_{t}"]
        got = gpu_dequant(eng, t, b.ravel(), b.shape[0] * 32)
        assert same_bits(got, g[f"deq_{t}"].ravel()), t


def test_dequant_f16_f32(eng, orc, cuda):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(1000).astype(np.float32)  # not a multiple of 32
    h = x.astype(np.float16)
    assert same_bits(gpu_dequant(eng, F16, h.view(np.uint8), 1000), h.astype(np.float32))
    assert same_bits(gpu_dequant(eng, F16, h[:992].view(np.uint8), 992), h[:992].astype(np.float32))
    assert same_bits(gpu_dequant(eng, F32, x.view(np.uint8), 1000), x)


def quant_inputs(rng, rows, ne0):
    x = rng.standard_normal((rows, ne0)).astype(np.float32)
    x *= np.exp(rng.uniform(-6, 6, size=(rows, 1))).astype(np.float32)
    x[::7] = np.round(x[::7] * 2) / 2  # exact ties for the rounding paths
    x[3] = 0.0
    x[5, :] = 1.25
    return x


@pytest.mark.parametrize("t", [F32, F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1])
def test_set_rows_bit_exact(eng, orc, t, cuda):
    """Positions written as cosyvoice_kv_cache::update_cache does (src/cosyvoice-kv-cache.cpp:316)."""
    rng = np.random.default_rng(200 + t)
    max_seq, ne0, n = 300, 128, 64
    rb = row_bytes(t, ne0)
    cache = rng.integers(0, 256, size=(max_seq, rb), dtype=np.uint8)
    src = quant_inputs(rng, n, ne0)
    idx = rng.permutation(max_seq)[:n].astype(np.int32)
    want = cache.copy()
    orc.set_rows(want, t, rb, max_seq, src, idx)
    d_cache, d_src, d_idx = dev(cache), dev(src), dev(idx)
    dt = cvattn.contiguous(d_cache.data_ptr(), t, [ne0, max_seq, 1, 1])
    st = cvattn.contiguous(d_src.data_ptr(), F32, [ne0, n, 1, 1])
    it = cvattn.contiguous(d_idx.data_ptr(), cvattn.I32, [n, 1, 1, 1])
    assert eng.set_rows(dt, st, it) == cvattn.OK
    assert np.array_equal(host(d_cache), want)


def test_set_rows_dit_batch_index(eng, orc, cuda):
    """DiT cache write: k [1024, T, 2] with 2-D position ids [T, 2] (src/cosyvoice-graph.cpp:363-365,
    src/cosyvoice-kv-cache.cpp:104-119 with batch 2)."""
    rng = np.random.default_rng(9)
    ne0, T, B, max_seq, t = 1024, 50, 2, 200, Q8_0
    rb = row_bytes(t, ne0)
    cache = np.zeros((B, max_seq, rb), dtype=np.uint8)
    src = rng.standard_normal((B, T, ne0)).astype(np.float32)
    pos = np.stack([np.arange(T) + 100, np.arange(T) + 100], axis=1).astype(np.int32)  # [T, B] -> ne=[T, 2]
    pos_dev = np.ascontiguousarray(pos.T)  # ggml [T, 2]: row b holds batch b's positions
    want = cache.copy()
    for b in range(B):
        orc.set_rows(want[b], t, rb, max_seq, src[b], pos_dev[b])
    d_cache, d_src, d_idx = dev(cache), dev(src), dev(pos_dev)
    dt = cvattn.contiguous(d_cache.data_ptr(), t, [ne0, max_seq, B, 1])
    st = cvattn.contiguous(d_src.data_ptr(), F32, [ne0, T, B, 1])
    it = cvattn.contiguous(d_idx.data_ptr(), cvattn.I32, [T, B, 1, 1])
    assert eng.set_rows(dt, st, it) == cvattn.OK
    assert np.array_equal(host(d_cache), want)


@pytest.mark.parametrize("t", QUANT_TYPES)
def test_set_rows_exact_ties_known_codes(eng, t, cuda):
    """The quantize-on-write on inputs that land exactly on rounding ties (|id| = 1), against the
    codes written out by hand from each *_ref tie rule (tests/_ties.py), not against the oracle."""
    cases = tie_cases()[t]
    x = np.stack([c[0] for c in cases]).astype(np.float32)      # one 32-element row per case
    want = np.stack([c[1] for c in cases])
    n = x.shape[0]
    cache = np.full((n + 3, TYPE_BYTES[t]), 0xA5, dtype=np.uint8)
    idx = (np.arange(n, dtype=np.int32) * 2 + 1) % (n + 3)
    d_cache, d_src, d_idx = dev(cache), dev(x), dev(idx)
    dt = cvattn.contiguous(d_cache.data_ptr(), t, [32, n + 3, 1, 1])
    st = cvattn.contiguous(d_src.data_ptr(), F32, [32, n, 1, 1])
    it = cvattn.contiguous(d_idx.data_ptr(), cvattn.I32, [n, 1, 1, 1])
    assert eng.set_rows(dt, st, it) == cvattn.OK
    got = host(d_cache)
    for i in range(n):
        assert list(got[idx[i]]) == list(want[i]), (t, i)
