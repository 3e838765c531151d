"""RoPE on the GPU against the oracle's ggml_rope_ext restatement, and the KV write with RoPE fused
in front against oracle rope followed by oracle set_rows.

Rotations are floating point: the device cosf/sinf and the C library's differ by about an ulp, so
rotated values agree within 2e-6 (N(0,1) inputs) and the dims the rope does not rotate are copied
bit for bit.  Quantized writes are compared through their codes: the inputs to the quantizer
differ by an ulp at most, which moves a code across a rounding boundary rarely; the test requires
every block scale and at least 99.9% of codes to match and every dequantized value to lie within
one quantization step of the oracle's.
"""
import numpy as np
import pytest

import cvattn
from _gpu import dev, host
from cvattn import F16, F32, I32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, ROPE_NEOX, ROPE_NORMAL
from oracle.oracle import row_bytes

pytestmark = pytest.mark.gpu

ROT_TOL = 2e-6


def oracle_rope_rows(orc, x, pos_rows, head, n_dims, mode, base):
    """x[..., ne0] with one position per row; ropes each `head`-wide input of a row."""
    shp = x.shape
    segs = x.reshape(-1, shp[-1] // head, head)
    p = np.repeat(np.asarray(pos_rows, np.int32).reshape(-1), shp[-1] // head)
    return orc.rope(segs.reshape(-1, head), p, n_dims, mode, base).reshape(shp)


@pytest.mark.parametrize("mode,n_dims,ne0,ne1,base", [
    (ROPE_NEOX, 64, 64, 14, 1e6),      # LLM query heads (src/cosyvoice-llm.cpp:56)
    (ROPE_NORMAL, 64, 1024, 1, 1e4),   # DiT query row, 64 of 1024 dims (src/cosyvoice-graph.cpp:351)
    (ROPE_NEOX, 32, 96, 3, 1e4),       # partial rotation, odd head count
])
def test_rope_matches_oracle(eng, orc, cuda, mode, n_dims, ne0, ne1, base):
    rng = np.random.default_rng(31 + n_dims + ne1)
    n_tok = 37
    x = rng.standard_normal((n_tok, ne1, ne0)).astype(np.float32)
    pos = (np.arange(n_tok) + 4090).astype(np.int32)
    want = orc.rope(x, pos[:, None], n_dims, mode, base)
    dx, dp = dev(x), dev(pos)
    out = cvattn_empty(x.shape)
    sd = cvattn.contiguous(dx.data_ptr(), F32, [ne0, ne1, n_tok, 1])
    od = cvattn.contiguous(out.data_ptr(), F32, [ne0, ne1, n_tok, 1])
    pd = cvattn.contiguous(dp.data_ptr(), I32, [n_tok, 1, 1, 1])
    assert eng.rope(od, sd, pd, n_dims, mode, base) == cvattn.OK
    got = host(out)
    assert np.max(np.abs(got[..., :n_dims] - want[..., :n_dims])) <= ROT_TOL
    assert np.array_equal(got[..., n_dims:].view(np.uint32), x[..., n_dims:].view(np.uint32))


def cvattn_empty(shape):
    import torch
    return torch.full(shape, float("nan"), dtype=torch.float32, device="cuda:0")


def test_rope_strided_in_place(eng, orc, cuda):
    """The permuted/strided views the graphs hand over, rotated in place (dst aliases src)."""
    rng = np.random.default_rng(5)
    T, B, ne0 = 40, 2, 1024
    buf = rng.standard_normal((B * T, ne0 + 64)).astype(np.float32)   # padded rows
    pos = np.tile(np.arange(T) + 1000, B).astype(np.int32)
    want = buf.copy()
    want[:, :ne0] = orc.rope(buf[:, :ne0], pos, 64, ROPE_NORMAL, 1e4)
    d = dev(buf)
    dp = dev(pos)
    rb = (ne0 + 64) * 4
    view = cvattn.tensor(d.data_ptr(), F32, [ne0, 1, B * T, 1], [4, rb, rb, rb * B * T])
    pd = cvattn.contiguous(dp.data_ptr(), I32, [B * T, 1, 1, 1])
    assert eng.rope(view, view, pd, 64, ROPE_NORMAL, 1e4) == cvattn.OK
    got = host(d)
    assert np.max(np.abs(got[:, :64] - want[:, :64])) <= ROT_TOL
    assert np.array_equal(got[:, 64:].view(np.uint32), want[:, 64:].view(np.uint32))


def block_fields(t, rows):
    """(scale bytes, code bytes) views of rows of ggml blocks of type t."""
    nbk = {Q8_0: 34, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24}[t]
    hdr = {Q8_0: 2, Q4_0: 2, Q4_1: 4, Q5_0: 2, Q5_1: 4}[t]
    b = rows.reshape(-1, nbk)
    return b[:, :hdr], b[:, hdr:]


def compare_written(orc, t, got, want, ne0):
    if t == F32:
        assert np.max(np.abs(got.view(np.float32) - want.view(np.float32))) <= ROT_TOL
        return
    if t == F16:
        g = got.view(np.uint16).astype(np.int32)
        w = want.view(np.uint16).astype(np.int32)
        assert np.max(np.abs(g - w)) <= 1   # one fp16 ulp, same sign (N(0,1) data)
        return
    sg, cg = block_fields(t, got)
    sw, cw = block_fields(t, want)
    assert np.array_equal(sg, sw), "block scales differ"
    assert np.mean(cg == cw) >= 0.999
    dg = orc.dequantize(t, got.reshape(-1), got.size // row_bytes(t, ne0) * ne0)
    dw = orc.dequantize(t, want.reshape(-1), want.size // row_bytes(t, ne0) * ne0)
    step = np.abs(orc.f16_to_f32(sw[:, :2].copy().view(np.uint16)).reshape(-1))
    err = np.abs(dg - dw).reshape(-1, 32).max(axis=1)
    assert np.all(err <= step + 1e-7)


@pytest.mark.parametrize("t", [F32, F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1])
def test_rope_set_rows_llm(eng, orc, cuda, t):
    """K of one Qwen2 layer: [64, 2, n] NEOX with theta 1e6, written at position_ids
    (src/cosyvoice-llm.cpp:57-59, src/cosyvoice-kv-cache.cpp:316)."""
    rng = np.random.default_rng(700 + t)
    max_seq, n, ne0 = 4200, 9, 128
    rb = row_bytes(t, ne0)
    cache = rng.integers(0, 256, size=(max_seq, rb), dtype=np.uint8)
    src = rng.standard_normal((n, ne0)).astype(np.float32)
    posv = (np.arange(n) + 4090).astype(np.int32)
    roped = oracle_rope_rows(orc, src, posv, 64, 64, ROPE_NEOX, 1e6)
    want = cache.copy()
    orc.set_rows(want, t, rb, max_seq, roped, posv)
    d_cache, d_src, d_pos = dev(cache), dev(src), dev(posv)
    dt = cvattn.contiguous(d_cache.data_ptr(), t, [ne0, max_seq, 1, 1])
    st = cvattn.contiguous(d_src.data_ptr(), F32, [ne0, n, 1, 1])
    it = cvattn.contiguous(d_pos.data_ptr(), I32, [n, 1, 1, 1])
    assert eng.rope_set_rows(dt, st, it, it, 64, 64, ROPE_NEOX, 1e6) == cvattn.OK
    got = host(d_cache)
    untouched = np.setdiff1d(np.arange(max_seq), posv)
    assert np.array_equal(got[untouched], cache[untouched])
    compare_written(orc, t, got[posv], want[posv], ne0)


@pytest.mark.parametrize("t", [F16, Q8_0, Q4_0])
def test_rope_set_rows_dit(eng, orc, cuda, t):
    """DiT streaming chunk: k [1024, T, 2] rotated NORMAL on its first 64 dims (base 10000) and
    written at 2-D position ids [T, 2] (src/cosyvoice-graph.cpp:352,363-365)."""
    rng = np.random.default_rng(90 + t)
    ne0, T, B, max_seq, cur = 1024, 50, 2, 1100, 1000
    rb = row_bytes(t, ne0)
    cache = np.zeros((B, max_seq, rb), dtype=np.uint8)
    src = rng.standard_normal((B, T, ne0)).astype(np.float32)
    pos = np.stack([np.arange(T) + cur] * B).astype(np.int32)  # ggml [T, B]: row b = batch b
    want = cache.copy()
    for b in range(B):
        roped = oracle_rope_rows(orc, src[b], pos[b], 1024, 64, ROPE_NORMAL, 1e4)
        orc.set_rows(want[b], t, rb, max_seq, roped, pos[b])
    d_cache, d_src, d_pos = dev(cache), dev(src), dev(pos)
    dt = cvattn.contiguous(d_cache.data_ptr(), t, [ne0, max_seq, B, 1])
    st = cvattn.contiguous(d_src.data_ptr(), F32, [ne0, T, B, 1])
    it = cvattn.contiguous(d_pos.data_ptr(), I32, [T, B, 1, 1])
    assert eng.rope_set_rows(dt, st, it, it, 1024, 64, ROPE_NORMAL, 1e4) == cvattn.OK
    got = host(d_cache)
    assert not got[:, :cur].any() and not got[:, cur + T:].any()
    for b in range(B):
        compare_written(orc, t, got[b, cur:cur + T], want[b, cur:cur + T], ne0)


def test_llm_layer_write_then_decode(eng, orc, cuda):
    """One Qwen2 layer's attention path end to end on the device: Q rotated by cvattn_rope, K
    rotated and written (q8_0) by cvattn_rope_set_rows, V written (q4_0) by cvattn_set_rows,
    then the decode attention over the cache -- against the same chain in the oracle
    (src/cosyvoice-llm.cpp:56-62, src/cosyvoice-kv-cache.cpp:316-324,379-386)."""
    from oracle.oracle import view
    from _gpu import check_close, empty_f32, run_fa
    rng = np.random.default_rng(77)
    H, Hkv, D, n_kv, max_seq, theta = 14, 2, 64, 700, 768, 1e6
    ne0 = Hkv * D
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    k = rng.standard_normal((n_kv, ne0)).astype(np.float32)
    v = rng.standard_normal((n_kv, ne0)).astype(np.float32)
    posv = np.arange(n_kv, dtype=np.int32)
    qpos = np.array([n_kv - 1], np.int32)
    # oracle chain
    q_r = orc.rope(q, np.full((1, H), n_kv - 1, np.int32), D, ROPE_NEOX, theta)
    rbk, rbv = row_bytes(Q8_0, ne0), row_bytes(Q4_0, ne0)
    kc = np.zeros((max_seq, rbk), np.uint8)
    vc = np.zeros((max_seq, rbv), np.uint8)
    orc.set_rows(kc, Q8_0, rbk, max_seq, oracle_rope_rows(orc, k, posv, D, D, ROPE_NEOX, theta), posv)
    orc.set_rows(vc, Q4_0, rbv, max_seq, v, posv)
    kv_ne = [D, n_kv, Hkv, 1]
    want = orc.fa_f64(view(np.ascontiguousarray(q_r), F32, [D, 1, H, 1], [4, 4 * D * H, 4 * D, 4 * D * H]),
                      view(kc, Q8_0, kv_ne, [34, rbk, rbk // Hkv, rbk * max_seq]),
                      view(vc, Q4_0, kv_ne, [18, rbv, rbv // Hkv, rbv * max_seq]), None, 0.125, (1, 1, H, D))
    # device chain
    dq, dk, dv, dp, dqp = dev(q), dev(k), dev(v), dev(posv), dev(qpos)
    dkc, dvc = dev(np.zeros((max_seq, rbk), np.uint8)), dev(np.zeros((max_seq, rbv), np.uint8))
    qt = cvattn.contiguous(dq.data_ptr(), F32, [D, H, 1, 1])
    assert eng.rope(qt, qt, cvattn.contiguous(dqp.data_ptr(), I32, [1, 1, 1, 1]), D, ROPE_NEOX, theta) == cvattn.OK
    it = cvattn.contiguous(dp.data_ptr(), I32, [n_kv, 1, 1, 1])
    assert eng.rope_set_rows(cvattn.contiguous(dkc.data_ptr(), Q8_0, [ne0, max_seq, 1, 1]),
                             cvattn.contiguous(dk.data_ptr(), F32, [ne0, n_kv, 1, 1]), it, it, D, D, ROPE_NEOX,
                             theta) == cvattn.OK
    assert eng.set_rows(cvattn.contiguous(dvc.data_ptr(), Q4_0, [ne0, max_seq, 1, 1]),
                        cvattn.contiguous(dv.data_ptr(), F32, [ne0, n_kv, 1, 1]), it) == cvattn.OK
    out = empty_f32(1, 1, H, D)
    run_fa(eng, cvattn.llm_q_view(dq.data_ptr(), D, H, 1), cvattn.llm_kv_view(dkc.data_ptr(), Q8_0, D, Hkv, n_kv, max_seq),
           cvattn.llm_kv_view(dvc.data_ptr(), Q4_0, D, Hkv, n_kv, max_seq), None,
           cvattn.out_view(out.data_ptr(), D, H, 1))
    compare_written(orc, Q8_0, host(dkc)[:n_kv], kc[:n_kv], ne0)
    check_close(host(out), want, what="rope + write + decode")
