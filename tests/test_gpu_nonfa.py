"""GPU parity of the non-flash-attention path (--llm-flash-attn 0 / --flow-flash-attn 0):
cvattn_attn_nonfa over the transposed V cache against the oracle's soft_max restatement
(or_attn_nonfa_f64), and the transposed V write (cvattn_set_rows with ne0 = 1 and v_idxs).
  LLM   src/cosyvoice-kv-cache.cpp:104-108 (V cache [max_seq, H_kv*D]), :326-348 (scatter), :387-395
  DiT   src/cosyvoice-graph.cpp:378-388 (no cache: V made contiguous after permute(1,0,2,3))
Bar: the attention bar (max-abs 2e-3, mean-abs 2e-4) against fp64; the scatter is bit-exact."""
import numpy as np
import pytest

import cvattn
from _gpu import check_close, dev, empty_f32, host, workspace
from oracle.oracle import F16, F32, Q4_0, Q8_0, TYPE_BYTES, row_bytes, v_idxs, view

pytestmark = pytest.mark.gpu
D = 64


def run_nonfa(eng, q, k, vt, mask, dst, scale=0.125):
    ws_bytes = eng.attn_nonfa_workspace(q, k, vt, mask)
    ws = workspace(ws_bytes)
    rc = eng.attn_nonfa(q, k, vt, mask, dst, scale, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK, eng.status_string(rc)
    host(ws)  # synchronise
    return ws


class Held:
    def __init__(self):
        self.keep = []

    def pair(self, arr, ttype, ne, nb):
        arr = np.ascontiguousarray(arr)
        d = dev(arr)
        self.keep += [arr, d]
        return view(arr, ttype, ne, nb), cvattn.tensor(d.data_ptr(), ttype, ne, nb)


def llm_nonfa(orc, rng, *, nq, nkv, kt, vtype, max_seq, mask=None, H=14, Hkv=2):
    """Q (rope output view), the K cache as in flash mode, the V cache transposed."""
    h = Held()
    q = rng.standard_normal((nq, H, D)).astype(np.float32)
    qh, qd = h.pair(q, F32, [D, nq, H, 1], [4, 4 * D * H, 4 * D, 4 * D * H * nq])
    kx = rng.standard_normal((max_seq, Hkv * D)).astype(np.float32)
    kb = orc.quantize_flat(kt, kx.reshape(-1)).reshape(max_seq, row_bytes(kt, Hkv * D))
    rb = row_bytes(kt, Hkv * D)
    kh, kd = h.pair(kb, kt, [D, nkv, Hkv, 1], [TYPE_BYTES[kt], rb, rb // Hkv, rb * max_seq])
    es = 4 if vtype == F32 else 2
    vx = rng.standard_normal((Hkv * D, max_seq)).astype(np.float32)       # [feature][token]
    vbuf = vx if vtype == F32 else orc.f32_to_f16(vx)
    vne = [nkv, D, Hkv, 1]
    vnb = [es, es * max_seq, es * max_seq * D, es * max_seq * D * Hkv]
    vh, vd = h.pair(vbuf, vtype, vne, vnb)
    mh = md = None
    if mask is not None:
        mh, md = h.pair(mask, F16, [mask.shape[1], mask.shape[0], 1, 1],
                        [2, 2 * mask.shape[1], 2 * mask.size, 2 * mask.size])
    out = empty_f32(1, nq, H, D)
    return h, (qh, kh, vh, mh), (qd, kd, vd, md), out, (1, nq, H, D)


@pytest.mark.parametrize("kt,vtype,nkv,max_seq", [(F16, F16, 1500, 1600), (Q8_0, F16, 1500, 1600),
                                                  (Q4_0, F32, 1500, 1600), (F32, F32, 1500, 1600),
                                                  (Q8_0, F16, 1501, 1600),   # odd n_kv: row ends mid-dword
                                                  (Q8_0, F16, 777, 801)])    # odd max_seq: 2-byte rows
def test_llm_decode_nonfa(eng, orc, rng, cuda, kt, vtype, nkv, max_seq):
    h, ho, dv, out, shape = llm_nonfa(orc, rng, nq=1, nkv=nkv, kt=kt, vtype=vtype, max_seq=max_seq)
    run_nonfa(eng, dv[0], dv[1], dv[2], None, cvattn.out_view(out.data_ptr(), D, 14, 1))
    want = orc.attn_nonfa_f64(*ho, 0.125, shape)
    check_close(host(out), want, what=f"nonfa decode k{kt} v{vtype}")


@pytest.mark.parametrize("nq,nkv", [(100, 356), (33, 33), (7, 4100)])
def test_llm_prefill_nonfa_causal(eng, orc, rng, cuda, nq, nkv):
    mask = orc.causal_mask(nq, nkv)
    h, ho, dv, out, shape = llm_nonfa(orc, rng, nq=nq, nkv=nkv, kt=Q8_0, vtype=F16, max_seq=nkv + 30, mask=mask)
    run_nonfa(eng, dv[0], dv[1], dv[2], dv[3], cvattn.out_view(out.data_ptr(), D, 14, nq))
    want = orc.attn_nonfa_f64(*ho, 0.125, shape)
    check_close(host(out), want, what=f"nonfa prefill {nq}x{nkv}")


@pytest.mark.parametrize("T", [300, 301])
def test_dit_nonfa_no_cache(eng, orc, rng, cuda, T):
    """DiT without cache: q/k the f32 [64, T, 16, 2] views, V transposed by the ggml_cont of
    permute(1, 0, 2, 3) into [T, 64, 16, 2] (src/cosyvoice-graph.cpp:380-381).  Both are copied
    to fp16 first; an odd T pads the copied V rows."""
    B, H = 2, 16
    h = Held()
    x = rng.standard_normal((3, B, T, H * D)).astype(np.float32)
    ne = [D, T, H, B]
    nb = [4, 4 * H * D, 4 * D, 4 * H * D * T]
    qh, qd = h.pair(x[0], F32, ne, nb)
    kh, kd = h.pair(x[1], F32, ne, nb)
    vt = np.ascontiguousarray(x[2].reshape(B, T, H, D).transpose(0, 2, 3, 1))  # [B][H][D][T]
    vh, vd = h.pair(vt, F32, [T, D, H, B], [4, 4 * T, 4 * T * D, 4 * T * D * H])
    out = empty_f32(B, T, H, D)
    run_nonfa(eng, qd, kd, vd, None, cvattn.out_view(out.data_ptr(), D, H, T, B))
    want = orc.attn_nonfa_f64(qh, kh, vh, None, 0.125, (B, T, H, D))
    check_close(host(out), want, what="dit nonfa")


def test_dit_nonfa_stream_cache_chunk_mask(eng, orc, rng, cuda):
    """DiT streaming step in non-flash mode: f16 V^T cache [max_seq, 1024, 2] of one layer, the
    chunk mask, 50 query rows over 1050 keys (src/cosyvoice-kv-cache.cpp:104-108,345)."""
    nq, nkv, max_seq, H, B = 50, 1050, 1100, 16, 2
    h = Held()
    q = rng.standard_normal((B, nq, H * D)).astype(np.float32)
    qh, qd = h.pair(q, F32, [D, nq, H, B], [4, 4 * H * D, 4 * D, 4 * H * D * nq])
    kx = rng.standard_normal((B, max_seq, H * D)).astype(np.float32)
    kb = orc.quantize_flat(Q8_0, kx.reshape(-1)).reshape(B, max_seq, row_bytes(Q8_0, H * D))
    rb = row_bytes(Q8_0, H * D)
    kh, kd = h.pair(kb, Q8_0, [D, nkv, H, B], [34, rb, rb // H, rb * max_seq])
    vx = orc.f32_to_f16(rng.standard_normal((B, H * D, max_seq)).astype(np.float32))
    vh, vd = h.pair(vx, F16, [nkv, D, H, B], [2, 2 * max_seq, 2 * max_seq * D, 2 * max_seq * D * H])
    full = orc.chunk_mask(nkv, [1000, 1025, 1050])
    mask = np.ascontiguousarray(full[nkv - nq:, :])
    mh, md = h.pair(mask, F16, [nkv, nq, 1, 1], [2, 2 * nkv, 2 * nkv * nq, 2 * nkv * nq])
    out = empty_f32(B, nq, H, D)
    run_nonfa(eng, qd, kd, vd, md, cvattn.out_view(out.data_ptr(), D, H, nq, B))
    want = orc.attn_nonfa_f64(qh, kh, vh, mh, 0.125, (B, nq, H, D))
    check_close(host(out), want, what="dit stream nonfa")


def test_fully_masked_row_is_nan(eng, orc, rng, cuda):
    """soft_max over a row whose keys are all -inf gives NaN in ggml; other rows are unaffected."""
    nq, nkv = 4, 70
    mask = np.zeros((nq, nkv), np.uint16)
    mask[2, :] = 0xFC00
    h, ho, dv, out, shape = llm_nonfa(orc, rng, nq=nq, nkv=nkv, kt=F16, vtype=F16, max_seq=80, mask=mask)
    run_nonfa(eng, dv[0], dv[1], dv[2], dv[3], cvattn.out_view(out.data_ptr(), D, 14, nq))
    got = host(out)
    assert np.all(np.isnan(got[0, 2]))
    want = orc.attn_nonfa_f64(*ho, 0.125, shape)
    keep = [0, 1, 3]
    check_close(got[:, keep], want[:, keep], what="rows beside the masked one")


@pytest.mark.parametrize("vtype", [F16, F32])
def test_transposed_v_write_v_idxs(eng, orc, cuda, vtype):
    """The non-flash V write: V [n_embd, n] flattened to [1, N] and scattered through v_idxs
    into the flattened [max_seq, n_embd, batch] cache with cvattn_set_rows (ne0 = 1);
    bit-exact against the oracle's transposed write."""
    rng = np.random.default_rng(11 + vtype)
    n_embd, max_seq, T, B = 1024, 120, 50, 2
    pos = np.arange(T) + 60
    idx = v_idxs(pos, B * T, T, n_embd, max_seq)
    es = 4 if vtype == F32 else 2
    cache = rng.integers(0, 256, size=B * n_embd * max_seq * es, dtype=np.uint8)
    src = rng.standard_normal((B * T, n_embd)).astype(np.float32)
    flat_want = cache.copy().view(np.float32 if vtype == F32 else np.uint16)
    flat_want[idx] = src.reshape(-1) if vtype == F32 else orc.f32_to_f16(src.reshape(-1))
    d_cache, d_src, d_idx = dev(cache), dev(src), dev(idx)
    N = idx.size
    dt = cvattn.contiguous(d_cache.data_ptr(), vtype, [1, B * n_embd * max_seq, 1, 1])
    st = cvattn.contiguous(d_src.data_ptr(), F32, [1, N, 1, 1])
    it = cvattn.contiguous(d_idx.data_ptr(), cvattn.I32, [N, 1, 1, 1])
    assert eng.set_rows(dt, st, it) == cvattn.OK
    assert np.array_equal(host(d_cache), flat_want.view(np.uint8))


def test_nonfa_after_transposed_write(eng, orc, rng, cuda):
    """A decode step of the non-flash LLM path on device: V written through v_idxs, then
    cvattn_attn_nonfa over the cache it produced (src/cosyvoice-kv-cache.cpp:326-348,387-395)."""
    Hkv, H, n_embd, max_seq, n_kv = 2, 14, 128, 512, 300
    v_rows = rng.standard_normal((n_kv, n_embd)).astype(np.float32)
    idx = v_idxs(np.arange(n_kv), n_kv, n_kv, n_embd, max_seq)
    d_cache = dev(np.zeros(n_embd * max_seq, np.uint16))
    d_src, d_idx = dev(v_rows), dev(idx)
    assert eng.set_rows(cvattn.contiguous(d_cache.data_ptr(), F16, [1, n_embd * max_seq, 1, 1]),
                        cvattn.contiguous(d_src.data_ptr(), F32, [1, idx.size, 1, 1]),
                        cvattn.contiguous(d_idx.data_ptr(), cvattn.I32, [idx.size, 1, 1, 1])) == cvattn.OK
    h = Held()
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    qh, qd = h.pair(q, F32, [D, 1, H, 1], [4, 4 * D * H, 4 * D, 4 * D * H])
    kx = orc.f32_to_f16(rng.standard_normal((max_seq, n_embd)).astype(np.float32))
    kh, kd = h.pair(kx, F16, [D, n_kv, Hkv, 1], [2, 2 * n_embd, 2 * D, 2 * n_embd * max_seq])
    vne, vnb = [n_kv, D, Hkv, 1], [2, 2 * max_seq, 2 * max_seq * D, 2 * max_seq * n_embd]
    vd = cvattn.tensor(d_cache.data_ptr(), F16, vne, vnb)
    vcache = orc.f32_to_f16(np.zeros(n_embd * max_seq, np.float32))
    vcache[idx] = orc.f32_to_f16(v_rows.reshape(-1))
    vh = view(vcache, F16, vne, vnb)
    out = empty_f32(1, 1, H, D)
    run_nonfa(eng, qd, kd, vd, None, cvattn.out_view(out.data_ptr(), D, H, 1))
    want = orc.attn_nonfa_f64(qh, kh, vh, None, 0.125, (1, 1, H, D))
    check_close(host(out), want, what="write then nonfa")
