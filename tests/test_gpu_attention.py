"""GPU parity of cvattn_flash_attn_ext (the GGML_OP_FLASH_ATTN_EXT node) against the fp64 oracle,
with the exact tensor views the reference builds:
  LLM decode/prefill  src/cosyvoice-kv-cache.cpp:316-324, src/cosyvoice-llm.cpp:56-60
  DiT (no cache)      src/cosyvoice-graph.cpp:357-377
  DiT (stream cache)  src/cosyvoice-graph.cpp:363-367 -> kv-cache views with batch 2
Bar: max-abs <= 2e-3 and mean-abs <= 2e-4 vs the fp64 oracle on identical (bit-exact) inputs."""
import os

import numpy as np
import pytest
import torch

import cvattn
from _gpu import check_close, dev, empty_f32, host, run_fa, workspace
from oracle.oracle import F16, F32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, TYPE_BYTES, row_bytes, view

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
D = 64
ALL_TYPES = [F32, F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1]


class Case:
    """One attention problem held twice: host buffers for the oracle, device buffers for the engine,
    both described with the same ne/nb."""

    def __init__(self):
        self.keep = []

    def add(self, name, arr, ttype, ne, nb):
        arr = np.ascontiguousarray(arr)
        d = dev(arr)
        self.keep += [arr, d]
        setattr(self, name + "_h", view(arr, ttype, ne, nb))
        setattr(self, name + "_d", cvattn.tensor(d.data_ptr(), ttype, ne, nb))
        setattr(self, name + "_dev", d)


def kv_bytes(orc, t, x):
    """[..., rows, H_kv*D] float32 -> [..., rows, row_bytes] cache bytes."""
    lead = x.shape[:-1]
    flat = orc.quantize_flat(t, x.reshape(-1))
    return flat.reshape(*lead, row_bytes(t, x.shape[-1]))


def llm_case(orc, rng, *, H=14, Hkv=2, nq=1, nkv=512, kt=F16, vt=F16, B=1, kB=None, max_seq=None,
             mask=None, qscale=1.0, kvscale=1.0):
    kB = kB or B
    max_seq = max_seq or nkv
    c = Case()
    q = (qscale * rng.standard_normal((B, nq, H, D))).astype(np.float32)
    c.add("q", q, F32, [D, nq, H, B], [4, 4 * D * H, 4 * D, 4 * D * H * nq])
    for name, t in (("k", kt), ("v", vt)):
        x = (kvscale * rng.standard_normal((kB, max_seq, Hkv * D))).astype(np.float32)
        b = kv_bytes(orc, t, x)
        rb = row_bytes(t, Hkv * D)
        c.add(name, b, t, [D, nkv, Hkv, kB], [TYPE_BYTES[t], rb, rb // Hkv, rb * max_seq])
    c.mask_h = c.mask_d = None
    if mask is not None:
        m = np.ascontiguousarray(mask)
        ne = [m.shape[-1], m.shape[-2], m.shape[-3] if m.ndim > 2 else 1, m.shape[-4] if m.ndim > 3 else 1]
        nb = [2, 2 * ne[0], 2 * ne[0] * ne[1], 2 * ne[0] * ne[1] * ne[2]]
        c.add("mask", m, F16, ne, nb)
    c.out_shape = (B, nq, H, D)
    c.dst = empty_f32(*c.out_shape)
    c.dst_d = cvattn.out_view(c.dst.data_ptr(), D, H, nq, B)
    return c


def run_case(eng, orc, c, scale=0.125, what=""):
    run_fa(eng, c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d, scale)
    got = host(c.dst)
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, scale, c.out_shape)
    return check_close(got, want, what=what), got, want


# ------------------------------------------------------------------------------------------
# committed fixtures
# ------------------------------------------------------------------------------------------
def test_golden_decode_512_f16(eng, cuda):
    """Single-layer Qwen2 decode: 14/2 heads, f16 KV, n_kv 512, scale 1/8, no mask."""
    g = np.load(os.path.join(GOLDEN, "attn_decode_512_f16.npz"))
    q, kh, vh = g["q"], g["k_f16"], g["v_f16"]
    dq, dk, dv = dev(q), dev(kh), dev(vh)
    qd = cvattn.llm_q_view(dq.data_ptr(), D, 14, 1)
    kd = cvattn.llm_kv_view(dk.data_ptr(), F16, D, 2, 512, 512)
    vd = cvattn.llm_kv_view(dv.data_ptr(), F16, D, 2, 512, 512)
    out = empty_f32(14, D)
    run_fa(eng, qd, kd, vd, None, cvattn.out_view(out.data_ptr(), D, 14, 1))
    check_close(host(out), g["out"], what="decode 512 f16 fixture")


def test_golden_prefill_small(eng, cuda):
    g = np.load(os.path.join(GOLDEN, "attn_prefill_small.npz"))
    nq, nkv = 8, 40
    dq, dk, dv, dm = dev(g["q"]), dev(g["k_q8_0"]), dev(g["v_q4_0"]), dev(g["mask"])
    qd = cvattn.llm_q_view(dq.data_ptr(), D, 14, nq)
    kd = cvattn.llm_kv_view(dk.data_ptr(), Q8_0, D, 2, nkv, nkv)
    vd = cvattn.llm_kv_view(dv.data_ptr(), Q4_0, D, 2, nkv, nkv)
    md = cvattn.mask_view(dm.data_ptr(), nkv, nq)
    out = empty_f32(nq, 14, D)
    run_fa(eng, qd, kd, vd, md, cvattn.out_view(out.data_ptr(), D, 14, nq))
    check_close(host(out), g["out"].reshape(nq, 14, D), what="prefill_small")


def test_golden_dit_small(eng, cuda):
    g = np.load(os.path.join(GOLDEN, "attn_dit_small.npz"))
    T, B = 40, 2
    q, k, v = (g[n].astype(np.float32) for n in ("q", "k", "v"))
    dq, dk, dv, dm = dev(q), dev(k), dev(v), dev(g["mask"])
    qd = cvattn.dit_view(dq.data_ptr(), T, B)
    kd = cvattn.dit_view(dk.data_ptr(), T, B)
    vd = cvattn.dit_view(dv.data_ptr(), T, B)
    md = cvattn.mask_view(dm.data_ptr(), T, T)
    out = empty_f32(B, T, 16, D)
    run_fa(eng, qd, kd, vd, md, cvattn.out_view(out.data_ptr(), D, 16, T, B))
    check_close(host(out), g["out"], what="dit_small")


# ------------------------------------------------------------------------------------------
# every K/V type pair the loader can choose
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("kt", ALL_TYPES)
@pytest.mark.parametrize("vt", ALL_TYPES)
def test_decode_type_pairs(eng, orc, rng, kt, vt, cuda):
    c = llm_case(orc, rng, nq=1, nkv=301, kt=kt, vt=vt, max_seq=320)
    run_case(eng, orc, c, what=f"k{kt} v{vt}")


@pytest.mark.parametrize("kt,vt", [(Q8_0, Q4_0), (Q8_0, Q8_0), (F16, F16), (Q5_1, Q5_1)])
def test_decode_4096_token_layer(eng, orc, rng, kt, vt, cuda):
    """One Qwen2 layer over a full 4096-row cache (n_kv 4096), 14/2 heads (split over the chip)."""
    c = llm_case(orc, rng, nq=1, nkv=4096, kt=kt, vt=vt, max_seq=4096)
    run_case(eng, orc, c, what="cfg2 layer")


@pytest.mark.parametrize("nkv", [1, 2, 31, 32, 33, 127, 129, 1000])
def test_decode_ragged_lengths(eng, orc, rng, nkv, cuda):
    c = llm_case(orc, rng, nq=1, nkv=nkv, kt=Q8_0, vt=Q4_0, max_seq=nkv + 40)
    run_case(eng, orc, c, what=f"nkv {nkv}")


@pytest.mark.parametrize("H,Hkv,nq,B,kB", [(6, 3, 1, 1, 1),     # odd kv heads: one head per workgroup
                                            (8, 4, 1, 2, 1),     # two head pairs, K/V broadcast over batch
                                            (16, 2, 1, 1, 1),    # 8 rows per head: full head slots
                                            (4, 2, 3, 1, 1),     # 6 rows per head over 3 query tokens
                                            (18, 2, 1, 1, 1)])   # 9 rows per head: no pairing
def test_decode_head_grouping(eng, orc, rng, H, Hkv, nq, B, kB, cuda):
    """Kv-head pairing of the decode kernel (two heads of <= 8 rows share a 16-row tile) and the
    fallbacks around it, with splits over several workgroups (n_kv 2500)."""
    for kt, vt in ((Q8_0, Q4_0), (F16, Q5_1)):
        c = llm_case(orc, rng, H=H, Hkv=Hkv, nq=nq, nkv=2500, kt=kt, vt=vt, B=B, kB=kB, max_seq=2600)
        run_case(eng, orc, c, what=f"H {H} Hkv {Hkv} nq {nq} B {B} k{kt} v{vt}")


def test_several_row_groups_over_long_cache_split(eng, orc, rng, cuda):
    """50 query rows per kv head (four 16-row groups, as a DiT streaming chunk) over 9000 cached
    f16 tokens: the decode kernel with several row groups and token splits merged in-kernel."""
    c = llm_case(orc, rng, H=16, Hkv=16, nq=50, nkv=9000, kt=F16, vt=F16, max_seq=9000)
    p = cvattn.FaProblem()
    p.q, p.k, p.v, p.dst = c.q_d, c.k_d, c.v_d, c.dst_d
    ws = workspace(eng.fa_batch_workspace([p]))
    rc, plan = eng.fa_batch_prepare([p], 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
    check_close(host(c.dst), want, what="50 rows x 9000 tokens, batch")
    single = empty_f32(*c.out_shape)
    run_fa(eng, c.q_d, c.k_d, c.v_d, None, cvattn.out_view(single.data_ptr(), D, 16, 50))
    check_close(host(single), want, what="50 rows x 9000 tokens, single call")


def test_decode_two_query_tokens(eng, orc, rng, cuda):
    c = llm_case(orc, rng, nq=2, nkv=700, kt=Q8_0, vt=Q4_0, max_seq=1024)
    run_case(eng, orc, c, what="nq 2")


# ------------------------------------------------------------------------------------------
# prefill with the reference's causal mask (src/cosyvoice-llm.cpp:20-29, 101-108)
# ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("nq,nkv,kt,vt", [(256, 256, F16, F16), (256, 768, F16, F16), (37, 100, Q8_0, Q4_0),
                                          (3, 60, F16, F16), (256, 512, Q8_0, Q8_0)])
def test_prefill_causal(eng, orc, rng, nq, nkv, kt, vt, cuda):
    mask = orc.causal_mask(nq, nkv)
    c = llm_case(orc, rng, nq=nq, nkv=nkv, kt=kt, vt=vt, max_seq=nkv + 16, mask=mask, qscale=0.5, kvscale=0.5)
    run_case(eng, orc, c, what=f"prefill {nq}x{nkv}")


def test_mask_rows_wider_than_nkv_and_all_masked_row(eng, orc, rng, cuda):
    nq, nkv = 5, 70
    mask = np.zeros((nq + 3, nkv + 9), dtype=np.uint16)  # padded mask: only [:nq, :nkv] is read
    mask[:, nkv:] = 0x7C00  # +inf beyond n_kv would poison the result if read
    mask[2, :] = 0xFC00     # a row with every key masked -> 0
    mask[3, ::2] = 0xFC00
    c = llm_case(orc, rng, nq=nq, nkv=nkv, kt=Q8_0, vt=Q4_1, mask=mask, max_seq=80)
    (_, _), got, _ = run_case(eng, orc, c, what="padded mask")
    assert np.all(got[0, 2] == 0)


def test_mask_broadcast_over_heads_and_batch(eng, orc, rng, cuda):
    nq, nkv, H, B = 4, 90, 14, 2
    mask = np.where(rng.random((1, 7, nq, nkv)) < 0.3, 0xFC00, 0).astype(np.uint16)  # ne2 = 7 heads, ne3 = 1
    mask = (mask.view(np.uint16) | np.where(mask == 0, rng.integers(0, 0x3C00, size=mask.shape), 0)).astype(np.uint16)
    c = llm_case(orc, rng, nq=nq, nkv=nkv, H=H, B=B, kt=F16, vt=Q8_0, mask=mask, max_seq=96)
    run_case(eng, orc, c, what="mask broadcast")


def test_kv_broadcast_over_batch(eng, orc, rng, cuda):
    c = llm_case(orc, rng, nq=3, nkv=200, B=3, kB=1, kt=Q4_0, vt=Q5_0)
    run_case(eng, orc, c, what="kv batch broadcast")


def test_scale_and_large_logits(eng, orc, rng, cuda):
    c = llm_case(orc, rng, nq=1, nkv=500, kt=F16, vt=F16, qscale=4.0)
    run_case(eng, orc, c, scale=0.3, what="large logits")


# ------------------------------------------------------------------------------------------
# DiT (src/cosyvoice-graph.cpp:326-398)
# ------------------------------------------------------------------------------------------
def dit_case(orc, rng, *, T, B=2, H=16, Tq=None, mask=None, ttype=F32):
    Tq = Tq or T
    c = Case()
    es = 4 if ttype == F32 else 2
    npt = np.float32 if ttype == F32 else np.float16
    for name, n in (("q", Tq), ("k", T), ("v", T)):
        x = rng.standard_normal((B, n, H * D)).astype(npt)
        arr = x if ttype == F32 else x.view(np.uint16)
        row = es * H * D
        c.add(name, arr, ttype, [D, n, H, B], [es, row, es * D, row * n])
    c.mask_h = c.mask_d = None
    if mask is not None:
        c.add("mask", mask, F16, [mask.shape[1], mask.shape[0], 1, 1],
              [2, 2 * mask.shape[1], 2 * mask.size, 2 * mask.size])
    c.out_shape = (B, Tq, H, D)
    c.dst = empty_f32(*c.out_shape)
    c.dst_d = cvattn.out_view(c.dst.data_ptr(), D, H, Tq, B)
    return c


@pytest.mark.parametrize("T", [50, 300, 1500])
def test_dit_bidirectional_f32(eng, orc, rng, T, cuda):
    c = dit_case(orc, rng, T=T)
    run_case(eng, orc, c, what=f"dit T={T}")


def test_dit_f16_inputs(eng, orc, rng, cuda):
    c = dit_case(orc, rng, T=333, ttype=F16)
    run_case(eng, orc, c, what="dit f16")


@pytest.mark.parametrize("T", [400, 1500])
@pytest.mark.parametrize("kt,vt", [(F32, F16), (F16, F32)])
def test_dit_one_fp32_side(eng, orc, rng, kt, vt, T, cuda):
    """Only one of K/V fp32: that side alone is copied to fp16 before the kernel runs (at T=1500
    the kernel is the wide form: 192-row workgroups)."""
    B, H = 2, 16
    c = Case()
    for name, t, n in (("q", F32, T), ("k", kt, T), ("v", vt, T)):
        x = rng.standard_normal((B, n, H * D)).astype(np.float32)
        es = 4 if t == F32 else 2
        arr = x if t == F32 else orc.f32_to_f16(x)
        c.add(name, arr, t, [D, n, H, B], [es, es * H * D, es * D, es * H * D * n])
    c.mask_h = c.mask_d = None
    c.out_shape = (B, T, H, D)
    c.dst = empty_f32(*c.out_shape)
    c.dst_d = cvattn.out_view(c.dst.data_ptr(), D, H, T, B)
    run_case(eng, orc, c, what=f"dit T={T} k{kt} v{vt}")


def test_dit_fp32_head_major_k_view(eng, orc, rng, cuda):
    """fp32 K laid out head-major ([B][H][T][D]: nb1 = 256, nb2 = 256 T) and fp32 V token-major, an
    odd T: the fp16 copies index both views through their own strides (row, head and batch
    decomposition of the copy kernel)."""
    T, B, H = 333, 2, 16
    c = Case()
    q = rng.standard_normal((B, T, H * D)).astype(np.float32)
    c.add("q", q, F32, [D, T, H, B], [4, 4 * H * D, 4 * D, 4 * H * D * T])
    k = rng.standard_normal((B, H, T, D)).astype(np.float32)
    c.add("k", k, F32, [D, T, H, B], [4, 4 * D, 4 * D * T, 4 * D * T * H])
    v = rng.standard_normal((B, T, H * D)).astype(np.float32)
    c.add("v", v, F32, [D, T, H, B], [4, 4 * H * D, 4 * D, 4 * H * D * T])
    c.mask_h = c.mask_d = None
    c.out_shape = (B, T, H, D)
    c.dst = empty_f32(*c.out_shape)
    c.dst_d = cvattn.out_view(c.dst.data_ptr(), D, H, T, B)
    run_case(eng, orc, c, what="dit head-major fp32 K")


def test_dit_chunk_mask(eng, orc, rng, cuda):
    T = 250
    mask = orc.chunk_mask(T, [50, 100, 150, 200])
    c = dit_case(orc, rng, T=T, mask=mask)
    run_case(eng, orc, c, what="dit chunk mask")


def test_dit_cut_len_query_subset(eng, orc, rng, cuda):
    """Last block with cut_len: n_q = T - cut < n_kv = T, one shared mask indexed by local row
    (src/cosyvoice-graph.cpp:337-343, 453-465)."""
    T, cut = 180, 60
    mask = orc.chunk_mask(T, [60, 120])
    c = dit_case(orc, rng, T=T, Tq=T - cut, mask=mask)
    run_case(eng, orc, c, what="dit cut_len")


@pytest.mark.parametrize("kt,vt", [(F16, F16), (Q8_0, Q4_0)])
def test_dit_streaming_cache(eng, orc, rng, kt, vt, cuda):
    """Streaming: a 50-frame chunk over a cached 1000-frame prefix plus itself, cache rows of
    1024 elements with batch 2 (src/cosyvoice-kv-cache.cpp:104-119, 316-324)."""
    nq, nkv, max_seq, H, B = 50, 1050, 1200, 16, 2
    c = Case()
    q = rng.standard_normal((B, nq, H * D)).astype(np.float32)
    c.add("q", q, F32, [D, nq, H, B], [4, 4 * H * D, 4 * D, 4 * H * D * nq])
    for name, t in (("k", kt), ("v", vt)):
        x = rng.standard_normal((B, max_seq, H * D)).astype(np.float32)
        b = kv_bytes(orc, t, x)
        rb = row_bytes(t, H * D)
        c.add(name, b, t, [D, nkv, H, B], [TYPE_BYTES[t], rb, rb // H, rb * max_seq])
    c.mask_h = c.mask_d = None
    c.out_shape = (B, nq, H, D)
    c.dst = empty_f32(*c.out_shape)
    c.dst_d = cvattn.out_view(c.dst.data_ptr(), D, H, nq, B)
    run_case(eng, orc, c, what="dit stream")


# ------------------------------------------------------------------------------------------
# batched launches (many FA nodes, ragged KV lengths)
# ------------------------------------------------------------------------------------------
def test_batch_ragged_matches_single_calls_and_oracle(eng, orc, rng, cuda):
    lens = [256, 4000, 17, 8192, 1000, 64, 3333, 512]
    cases = [llm_case(orc, rng, nq=1, nkv=n, kt=Q8_0, vt=Q8_0, max_seq=n + 8) for n in lens]
    probs = []
    for c in cases:
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.dst = c.q_d, c.k_d, c.v_d, c.dst_d
        probs.append(p)
    wsb = eng.fa_batch_workspace(probs)
    ws = workspace(wsb)
    rc, plan = eng.fa_batch_prepare(probs, 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    for _ in range(2):  # a prepared plan can be launched repeatedly
        assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    for c, n in zip(cases, lens):
        got = host(c.dst)
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
        check_close(got, want, what=f"batch nkv {n}")
        single = empty_f32(*c.out_shape)
        run_fa(eng, c.q_d, c.k_d, c.v_d, None, cvattn.out_view(single.data_ptr(), D, 14, 1))
        check_close(host(single), got, max_abs=1e-5, mean_abs=1e-6, what="batch vs single")


def test_batch_prefill_with_masks(eng, orc, rng, cuda):
    cases = []
    for nkv in (64, 300):
        mask = orc.causal_mask(16, nkv)
        cases.append(llm_case(orc, rng, nq=16, nkv=nkv, kt=F16, vt=F16, mask=mask, max_seq=nkv))
    probs = []
    for c in cases:
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.mask, p.dst = c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d
        probs.append(p)
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare(probs, 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    for c in cases:
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, 0.125, c.out_shape)
        check_close(host(c.dst), want, what="batch prefill")


def one_allocation(cases, names=("q", "k", "v", "mask")):
    """Move the cases' tensors into one device allocation per tensor kind, problem i at a fixed
    byte stride past problem i-1 (the layers of one cache buffer), and return their problems."""
    keep = []
    for name in names:
        if getattr(cases[0], name + "_d", None) is None:
            continue
        big = torch.stack([getattr(c, name + "_dev") for c in cases])
        keep.append(big)
        for i, c in enumerate(cases):
            t = getattr(c, name + "_d")
            setattr(c, name + "_d", cvattn.tensor(big[i].data_ptr(), t.type, list(t.ne), list(t.nb)))
    out = empty_f32(len(cases), *cases[0].out_shape)
    keep.append(out)
    for i, c in enumerate(cases):
        c.dst = out[i]
        B, nq, H, _ = c.out_shape
        c.dst_d = cvattn.out_view(out[i].data_ptr(), D, H, nq, B)
    probs = []
    for c in cases:
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.dst = c.q_d, c.k_d, c.v_d, c.dst_d
        if c.mask_d is not None:
            p.mask = c.mask_d
        probs.append(p)
    return probs, keep


def launch_batch(eng, probs):
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare(probs, 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    for _ in range(2):  # the merging workgroups leave the arrival counters at zero
        assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    return ws


@pytest.mark.parametrize("order", ["forward", "reversed", "broken"])
def test_batch_layers_of_one_allocation(eng, orc, rng, order, cuda):
    """Decode problems whose tensors sit at fixed strides in one allocation (the layers of one
    cache buffer), in order, reversed, and with two swapped, give the oracle's results; two
    launches of one plan (the merging workgroups reset the arrival counters) agree."""
    cases = [llm_case(orc, rng, nq=1, nkv=1500, kt=Q8_0, vt=Q4_0, max_seq=1536) for _ in range(6)]
    probs, keep = one_allocation(cases)
    idx = list(range(6))
    if order == "reversed":
        idx = idx[::-1]
    elif order == "broken":
        idx[2], idx[3] = idx[3], idx[2]
    launch_batch(eng, [probs[i] for i in idx])
    for i, c in enumerate(cases):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"{order} layer {i}")


def test_batch_masked_prefill_of_one_allocation(eng, orc, rng, cuda):
    """Causal prefill problems (row-tiled kernel) with their masks, each kind of tensor in one
    allocation."""
    mask = orc.causal_mask(40, 300)
    cases = [llm_case(orc, rng, nq=40, nkv=300, kt=F16, vt=Q8_0, mask=mask, max_seq=320) for _ in range(4)]
    probs, keep = one_allocation(cases)
    launch_batch(eng, probs)
    for i, c in enumerate(cases):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"masked layer {i}")


def test_decode_24_layer_step_one_allocation(eng, orc, cuda):
    """The benchmark's decode step with its layers in one K and one V allocation (as the cache
    buffer holds them): 24 layers x 4096 tokens, K q8_0 / V q4_0, one prepared batch."""
    rng = np.random.default_rng(2027)
    cases = [llm_case(orc, rng, nq=1, nkv=4096, kt=Q8_0, vt=Q4_0, max_seq=4096) for _ in range(24)]
    probs, keep = one_allocation(cases)
    launch_batch(eng, probs)
    for i, c in enumerate(cases):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"24-layer step, layer {i}")


def test_short_prefill_over_long_cache_splits(eng, orc, rng, cuda):
    """12 new tokens over a 3000-token q8_0/q4_0 cache: 84 rows per kv head run in the row-tiled
    kernel, and so few row groups over so many keys are split over tokens -- merged by a second
    launch for a single call and by the last-arriving workgroup in a prepared batch."""
    nq, nkv = 12, 3000
    mask = orc.causal_mask(nq, nkv)
    c = llm_case(orc, rng, nq=nq, nkv=nkv, kt=Q8_0, vt=Q4_0, max_seq=nkv + 8, mask=mask, qscale=0.5)
    assert eng.flash_attn_ext_workspace(c.q_d, c.k_d, c.v_d, c.mask_d) > 0   # split over tokens
    _, single, _ = run_case(eng, orc, c, what="short prefill, single call")
    p = cvattn.FaProblem()
    p.q, p.k, p.v, p.mask, p.dst = c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d
    c.dst.fill_(float("nan"))
    ws = workspace(eng.fa_batch_workspace([p]))
    rc, plan = eng.fa_batch_prepare([p], 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    for _ in range(2):   # the arrival counters reset themselves
        assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    check_close(host(c.dst), single, max_abs=1e-5, mean_abs=1e-6, what="short prefill, batch vs single")


# ------------------------------------------------------------------------------------------
# the benchmark configurations at their full sizes
# ------------------------------------------------------------------------------------------
def run_batch(eng, cases, masked=False):
    probs = []
    for c in cases:
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.dst = c.q_d, c.k_d, c.v_d, c.dst_d
        if masked:
            p.mask = c.mask_d
        probs.append(p)
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare(probs, 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    return ws


def test_decode_24_layer_4096_token_step(eng, orc, cuda):
    """The decode step as the benchmark runs it: 24 layers x 4096 cached tokens, K q8_0 / V q4_0, one
    prepared batch (one launch with in-kernel split merges), every layer against the oracle."""
    rng = np.random.default_rng(2026)
    cases = [llm_case(orc, rng, nq=1, nkv=4096, kt=Q8_0, vt=Q4_0, max_seq=4096) for _ in range(24)]
    run_batch(eng, cases)
    for i, c in enumerate(cases):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"24-layer step, layer {i}")


def test_serving_16_ragged_sequences(eng, orc, cuda):
    """Serving decode: 16 sequences with kv_len drawn from U{256..8192} (the benchmark's seed), q8_0 K and
    V, one layer's 16 problems in one launch."""
    lens = np.random.default_rng(20261201).integers(256, 8193, 16)
    rng = np.random.default_rng(33)
    cases = [llm_case(orc, rng, nq=1, nkv=int(n), kt=Q8_0, vt=Q8_0, max_seq=int(n)) for n in lens]
    run_batch(eng, cases)
    for c, n in zip(cases, lens):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"serving kv_len {n}")


def test_prefill_1024_causal(eng, orc, cuda):
    """LLM prefill: 1024 query tokens over 1024 f16 cached tokens with the causal mask, Q/K/V scaled
    by 0.5 (src/cosyvoice-llm.cpp:20-29,101-108)."""
    rng = np.random.default_rng(44)
    mask = orc.causal_mask(1024, 1024)
    c = llm_case(orc, rng, nq=1024, nkv=1024, kt=F16, vt=F16, max_seq=1024, mask=mask, qscale=0.5, kvscale=0.5)
    run_case(eng, orc, c, what="1024-token causal prefill")


# ------------------------------------------------------------------------------------------
# the instances behind the benchmark's numbers, with more row groups than CUs (one key half)
# ------------------------------------------------------------------------------------------
def cu_count():
    return torch.cuda.get_device_properties(0).multi_processor_count


def row_groups(B, Hkv, n_rows, rows_per_group=64):
    """Row-tiled workgroups of a problem before token splits: one per 64 query rows of a kv head."""
    return B * Hkv * ((n_rows + rows_per_group - 1) // rows_per_group)


def batch_of(eng, cases, launches=1):
    probs = []
    for c in cases:
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.dst = c.q_d, c.k_d, c.v_d, c.dst_d
        if c.mask_d is not None:
            p.mask = c.mask_d
        probs.append(p)
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare(probs, 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK, eng.status_string(rc)
    for _ in range(launches):
        for c in cases:
            c.dst.fill_(float("nan"))
        assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    return ws


def test_dit_t1500_f16_prepared_batch(eng, orc, cuda):
    """The benchmark's DiT call: f16 q/k/v views, T=1500, batch 2, 16 heads, no mask, through a
    prepared batch (the timed form).  768 64-row groups > the CU count, and 256 192-row groups
    (the last one 156 rows) give every CU one: the wide form (12 waves per workgroup)."""
    assert row_groups(2, 16, 1500) > cu_count()
    assert row_groups(2, 16, 1500, 192) >= cu_count()
    rng = np.random.default_rng(1500)
    c = dit_case(orc, rng, T=1500, ttype=F16)
    batch_of(eng, [c], launches=2)
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
    check_close(host(c.dst), want, what="dit T=1500 f16 batch")


def test_dit_wide_batch_ragged_lengths(eng, orc, cuda):
    """The wide form over a prepared batch of two problems with different key lengths: 1200 f16
    query rows per (batch, head) over 1200 and 700 keys (448 192-row groups, the last of each
    head 48 rows), launched twice."""
    assert row_groups(2, 16, 1200, 192) * 2 >= cu_count()
    rng = np.random.default_rng(1200)
    cases = [dit_case(orc, rng, T=nkv, Tq=1200, ttype=F16) for nkv in (1200, 700)]
    batch_of(eng, cases, launches=2)
    for c, nkv in zip(cases, (1200, 700)):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"dit wide batch, n_kv {nkv}")


def dit_chunk_bounds(T, chunk=50):
    return list(range(chunk, T, chunk))


def test_dit_t1500_chunk_mask_fp32_views(eng, orc, cuda):
    """The uncached streaming DiT step after the first chunk (src/cosyvoice-token2wav.cpp:285-298):
    fp32 q/k/v views as the flow graph passes them (src/cosyvoice-graph.cpp:370-377), T=1500, a
    chunk boundary every 50 frames, one cvattn_flash_attn_ext call (fp16 copies of K/V, the masked
    one-half kernel)."""
    T = 1500
    assert row_groups(2, 16, T) > cu_count()
    rng = np.random.default_rng(1501)
    mask = orc.chunk_mask(T, dit_chunk_bounds(T))
    c = dit_case(orc, rng, T=T, mask=mask)
    run_case(eng, orc, c, what="dit T=1500 chunk mask, fp32 views")


def test_dit_t1500_chunk_mask_f16_prepared_batch(eng, orc, cuda):
    """The same masked call with f16 q/k/v through a prepared batch, launched twice."""
    T = 1500
    rng = np.random.default_rng(1502)
    mask = orc.chunk_mask(T, dit_chunk_bounds(T))
    c = dit_case(orc, rng, T=T, mask=mask, ttype=F16)
    batch_of(eng, [c], launches=2)
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, 0.125, c.out_shape)
    check_close(host(c.dst), want, what="dit T=1500 chunk mask f16 batch")


def test_dit_stream_chunk_prepared_batch(eng, orc, cuda):
    """The benchmark's DiT streaming call through a prepared batch: a 50-frame chunk over 1000
    cached f16 frames plus itself (n_kv 1050), batch 2, 16 heads."""
    nq, nkv, H, B = 50, 1050, 16, 2
    rng = np.random.default_rng(1050)
    c = Case()
    q = rng.standard_normal((B, nq, H * D)).astype(np.float32)
    c.add("q", q, F32, [D, nq, H, B], [4, 4 * H * D, 4 * D, 4 * H * D * nq])
    for name in ("k", "v"):
        x = orc.f32_to_f16(rng.standard_normal((B, nkv, H * D)).astype(np.float32))
        c.add(name, x, F16, [D, nkv, H, B], [2, 2 * H * D, 2 * D, 2 * H * D * nkv])
    c.mask_h = c.mask_d = None
    c.out_shape = (B, nq, H, D)
    c.dst = empty_f32(*c.out_shape)
    c.dst_d = cvattn.out_view(c.dst.data_ptr(), D, H, nq, B)
    batch_of(eng, [c], launches=2)
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, None, 0.125, c.out_shape)
    check_close(host(c.dst), want, what="dit stream 50x1050 batch")


def test_masked_prefill_batch_one_key_half(eng, orc, cuda):
    """Three 1024-token causal prefill problems in one prepared batch: 3 x 224 row groups > the CU
    count, so the masked batch kernel runs with one key half and no splits; launched twice."""
    assert 3 * row_groups(1, 2, 1024 * 7) > cu_count()
    rng = np.random.default_rng(3072)
    mask = orc.causal_mask(1024, 1024)
    cases = [llm_case(orc, rng, nq=1024, nkv=1024, kt=F16, vt=F16, max_seq=1024, mask=mask, qscale=0.5, kvscale=0.5)
             for _ in range(3)]
    batch_of(eng, cases, launches=2)
    for i, c in enumerate(cases):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"masked prefill batch, problem {i}")


def test_fp32_views_with_no_keys(eng, orc, cuda):
    """n_kv = 0 with fp32 K/V and 300 query rows per head (5 row groups): nothing to copy or read;
    every output row is 0, as ggml gives a row with no visible key."""
    T, B, H = 300, 2, 16
    rng = np.random.default_rng(0)
    q = dev(rng.standard_normal((B, T, H * D)).astype(np.float32))
    kv = dev(np.zeros((B, 1, H * D), dtype=np.float32))
    qd = cvattn.dit_view(q.data_ptr(), T, B)
    kd = cvattn.dit_view(kv.data_ptr(), 0, B)
    out = empty_f32(B, T, H, D)
    ws = run_fa(eng, qd, kd, kd, None, cvattn.out_view(out.data_ptr(), D, H, T, B))
    assert np.all(host(out) == 0.0)
