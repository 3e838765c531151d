"""The DiT streaming cache on the GPU: the device-built step inputs against the oracle (chunk
mask, positions, v_idxs -- bit-exact), offload/load round trips through pinned host memory, and
two streaming chunks run end to end through the cache's slots and views against the oracle
(src/cosyvoice-token2wav.cpp:265-412, src/cosyvoice-kv-cache.cpp:148-290,309-355,379-395)."""
import numpy as np
import pytest
import torch

import cvattn
from _gpu import check_close, dev, empty_f32, host, workspace
from cvattn import F16, F32, I32, Q4_0, Q8_0, ROPE_NORMAL
from oracle.oracle import row_bytes, v_idxs, view

pytestmark = pytest.mark.gpu
D, H = 64, 16


@pytest.mark.parametrize("n,bounds", [(1050, [1000, 1025, 1050]), (300, [25, 50, 75, 100, 125, 150, 175, 200]),
                                      (64, []), (90, [90]), (40, [10, 10, 30])])
def test_chunk_mask_matches_oracle(eng, orc, cuda, n, bounds):
    d = dev(np.full((n, n), 0x1234, np.uint16))
    assert eng.chunk_mask(cvattn.contiguous(d.data_ptr(), F16, [n, n, 1, 1]), bounds) == cvattn.OK
    assert np.array_equal(host(d), orc.chunk_mask(n, bounds))


def test_chunk_mask_padded_rows(eng, orc, cuda):
    # a mask tensor with padded rows: only the [n_cols] of each row are written
    n, pad = 120, 8
    d = dev(np.full((n, n + pad), 0x1234, np.uint16))
    m = cvattn.tensor(d.data_ptr(), F16, [n, n, 1, 1], [2, 2 * (n + pad), 2 * (n + pad) * n, 2 * (n + pad) * n])
    assert eng.chunk_mask(m, [30, 70]) == cvattn.OK
    got = host(d)
    assert np.array_equal(got[:, :n], orc.chunk_mask(n, [30, 70]))
    assert np.all(got[:, n:] == 0x1234)


def test_positions_and_v_idxs(eng, cuda):
    T, B, base, n_embd, max_seq = 50, 2, 1000, 1024, 1100
    p = dev(np.zeros((B, T), np.int32))
    assert eng.fill_positions(cvattn.contiguous(p.data_ptr(), I32, [T, B, 1, 1]), base) == cvattn.OK
    pos = host(p)
    assert np.array_equal(pos, np.tile(np.arange(T, dtype=np.int32) + base, (B, 1)))
    idx = dev(np.zeros(T * B * n_embd, np.int32))
    assert eng.v_idxs(idx.data_ptr(), p.data_ptr(), T * B, T, n_embd, max_seq) == cvattn.OK
    assert np.array_equal(host(idx), v_idxs(pos[0], T * B, T, n_embd, max_seq))


def make_cache(eng, **kw):
    p = cvattn.DitCacheParams()
    d = dict(layers=3, heads=H, head_dim=D, max_seq=200, batch=2, k_type=Q8_0, v_type=Q4_0, n_slots=3,
             n_host_slots=2, flash_attn=1)
    d.update(kw)
    for k, v in d.items():
        setattr(p, k, v)
    dev_bytes, host_bytes = eng.dit_cache_bytes(p)
    dbuf = torch.empty(dev_bytes, dtype=torch.uint8, device="cuda:0")
    hbuf = torch.empty(max(host_bytes, 1), dtype=torch.uint8, pin_memory=True)
    rc, c = eng.dit_cache_create(p, dbuf.data_ptr(), dev_bytes, hbuf.data_ptr(), host_bytes)
    assert rc == cvattn.OK
    return p, c, dbuf, hbuf


@pytest.mark.parametrize("flash", [1, 0])
def test_offload_load_round_trip(eng, cuda, flash):
    """offload_slot / load_slot: the first n rows of every layer of the bound slot survive a
    trip through a host slot; the rest of the slot and the other slots are untouched."""
    kw = {} if flash else dict(v_type=F16, flash_attn=0)
    p, c, dbuf, hbuf = make_cache(eng, **kw)
    L = eng.L
    try:
        g = torch.Generator(device="cuda:0").manual_seed(5)
        dbuf.copy_(torch.randint(0, 256, dbuf.shape, dtype=torch.uint8, device="cuda:0", generator=g))
        before = host(dbuf).copy()
        n = 77
        assert L.cvattn_dit_cache_bind_slot(c, 1) == cvattn.OK
        assert L.cvattn_dit_cache_offload(c, 1, n, None) == cvattn.OK
        torch.cuda.synchronize()
        # clobber slot 1 entirely, then load it back
        per_slot = dbuf.numel() // p.n_slots
        dbuf[per_slot:2 * per_slot].fill_(0xAB)
        assert L.cvattn_dit_cache_load(c, 1, None) == cvattn.OK
        assert L.cvattn_dit_cache_len(c) == n
        after = host(dbuf)
        # the restored rows equal the originals; the other slots never changed
        assert np.array_equal(after[:per_slot], before[:per_slot])
        assert np.array_equal(after[2 * per_slot:], before[2 * per_slot:])
        for layer in range(p.layers):
            rc, (kc, vc, _, _) = eng.dit_cache_layer(c, layer, n)
            for t, is_v in ((kc, False), (vc, True)):
                off = t.data - dbuf.data_ptr()
                if not is_v or flash:
                    rb = t.nb[1]
                    for b in range(p.batch):
                        lo = off + b * t.nb[2]
                        assert np.array_equal(after[lo:lo + rb * n], before[lo:lo + rb * n])
                        assert np.all(after[lo + rb * n:lo + rb * p.max_seq] == 0xAB)
                else:   # transposed: the first n tokens of each of the 1024*2 feature columns
                    col = t.nb[1]
                    cols = np.arange(H * D * p.batch)
                    a = after[off:off + col * len(cols)].reshape(len(cols), col)
                    b0 = before[off:off + col * len(cols)].reshape(len(cols), col)
                    assert np.array_equal(a[:, :2 * n], b0[:, :2 * n])
                    assert np.all(a[:, 2 * n:] == 0xAB)
    finally:
        L.cvattn_dit_cache_destroy(c)


def test_two_streaming_chunks_end_to_end(eng, orc, cuda):
    """Chunk 1 (60 frames) then chunk 2 (40 frames) of one cached DiT step and layer: positions
    built on the device, K rotated and written with cvattn_rope_set_rows, V with set_rows, the
    slot offloaded to a host slot and loaded back between the chunks, Q rotated with cvattn_rope,
    and chunk 2 attends over the 100 cached frames through the cache's views -- against the
    oracle's rope, quantizers and fp64 attention (src/cosyvoice-graph.cpp:345-377)."""
    p, c, dbuf, hbuf = make_cache(eng, layers=1, max_seq=160, n_slots=2, n_host_slots=1)
    L = eng.L
    rng = np.random.default_rng(21)
    B, T1, T2 = 2, 60, 40
    xk = rng.standard_normal((B, T1 + T2, H * D)).astype(np.float32)
    xv = rng.standard_normal((B, T1 + T2, H * D)).astype(np.float32)
    xq = rng.standard_normal((B, T2, H * D)).astype(np.float32)
    try:
        def write_chunk(t0, T):
            pos = torch.zeros((B, T), dtype=torch.int32, device="cuda:0")
            pd = cvattn.contiguous(pos.data_ptr(), I32, [T, B, 1, 1])
            assert eng.fill_positions(pd, t0) == cvattn.OK
            rc, (kc, vc, _, _) = eng.dit_cache_layer(c, 0, t0 + T)
            k = dev(xk[:, t0:t0 + T])
            v = dev(xv[:, t0:t0 + T])
            src = lambda d: cvattn.contiguous(d.data_ptr(), F32, [H * D, T, B, 1])
            assert eng.rope_set_rows(kc, src(k), pd, pd, H * D, D, ROPE_NORMAL, 1e4) == cvattn.OK
            assert eng.set_rows(vc, src(v), pd) == cvattn.OK
            torch.cuda.synchronize()
            return pos

        write_chunk(0, T1)
        assert L.cvattn_dit_cache_offload(c, 0, T1, None) == cvattn.OK
        torch.cuda.synchronize()
        dbuf.fill_(0x5A)                         # the staging slot is reused by another step
        assert L.cvattn_dit_cache_load(c, 0, None) == cvattn.OK
        assert L.cvattn_dit_cache_len(c) == T1
        pos2 = write_chunk(T1, T2)
        # queries of chunk 2, rotated in place: [1024, 1, T2*B] rows at positions T1..
        q = dev(xq)
        qd = cvattn.contiguous(q.data_ptr(), F32, [H * D, 1, T2 * B, 1])
        assert eng.rope(qd, qd, cvattn.contiguous(pos2.data_ptr(), I32, [T2 * B, 1, 1, 1]), D, ROPE_NORMAL,
                        1e4) == cvattn.OK
        rc, (_, _, kv, vv) = eng.dit_cache_layer(c, 0, T1 + T2)
        out = empty_f32(B, T2, H, D)
        qv = cvattn.tensor(q.data_ptr(), F32, [D, T2, H, B], [4, 4 * H * D, 4 * D, 4 * H * D * T2])
        ws = workspace(eng.flash_attn_ext_workspace(qv, kv, vv, None))
        assert eng.flash_attn_ext(qv, kv, vv, None, cvattn.out_view(out.data_ptr(), D, H, T2, B), 0.125,
                                  ws.data_ptr(), ws.numel()) == cvattn.OK
        got = host(out)
    finally:
        L.cvattn_dit_cache_destroy(c)
    # oracle: rope K (first 64 dims of the 1024-wide rows) and Q, quantize K q8_0 / V q4_0
    allpos = np.arange(T1 + T2, dtype=np.int32)
    kr = np.stack([orc.rope(xk[b], allpos, D, ROPE_NORMAL, 1e4) for b in range(B)])
    qr = np.stack([orc.rope(xq[b], allpos[T1:], D, ROPE_NORMAL, 1e4) for b in range(B)])
    n = T1 + T2
    kb = orc.quantize_flat(Q8_0, kr.reshape(-1)).reshape(B, n, row_bytes(Q8_0, H * D))
    vb = orc.quantize_flat(Q4_0, xv.reshape(-1)).reshape(B, n, row_bytes(Q4_0, H * D))
    rk, rv = row_bytes(Q8_0, H * D), row_bytes(Q4_0, H * D)
    want = orc.fa_f64(view(np.ascontiguousarray(qr), F32, [D, T2, H, B], [4, 4 * H * D, 4 * D, 4 * H * D * T2]),
                      view(kb, Q8_0, [D, n, H, B], [34, rk, rk // H, rk * n]),
                      view(vb, Q4_0, [D, n, H, B], [18, rv, rv // H, rv * n]), None, 0.125, (B, T2, H, D))
    check_close(got, want, what="two streaming chunks")
