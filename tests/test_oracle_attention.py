"""Pins the fp64 attention oracle (ggml_flash_attn_ext contract) against torch's
scaled_dot_product_attention in fp64 on the CPU, plus invariants that a wrong index, a dropped
mask term or a transposed operand would break; checks the ggml-CPU-loop restatement against the
fp64 oracle; checks the caller masks by brute force and the KV write."""
import numpy as np
import pytest
import torch

from oracle.oracle import F16, F32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, row_bytes, view

D = 64


def make_problem(orc, rng, *, H=14, Hkv=2, nq=3, nkv=45, B=1, kt=F16, vt=F16, mask=None, qscale=1.0):
    """Seeded problem in the reference's LLM layout: Q [n_q, H, D] f32 permuted, K/V cache rows
    [n_kv, H_kv*D] of type kt/vt (src/cosyvoice-kv-cache.cpp:316-324)."""
    q = (qscale * rng.standard_normal((B, nq, H, D))).astype(np.float32)
    k = rng.standard_normal((B, nkv, Hkv * D)).astype(np.float32)
    v = rng.standard_normal((B, nkv, Hkv * D)).astype(np.float32)
    kb = np.stack([orc.quantize(kt, k[b]) for b in range(B)])
    vb = np.stack([orc.quantize(vt, v[b]) for b in range(B)])
    rk, rv = row_bytes(kt, Hkv * D), row_bytes(vt, Hkv * D)
    es = {F32: 4, F16: 2}
    qt = view(q, F32, [D, nq, H, B], [4, 4 * D * H, 4 * D, 4 * D * H * nq])
    ktd = view(kb, kt, [D, nkv, Hkv, B], [es.get(kt, {Q8_0: 34, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24}.get(kt)),
                                          rk, rk // Hkv, rk * nkv])
    vtd = view(vb, vt, [D, nkv, Hkv, B], [es.get(vt, {Q8_0: 34, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24}.get(vt)),
                                          rv, rv // Hkv, rv * nkv])
    # dequantized K/V exactly as the oracle sees them
    kd = np.stack([np.stack([orc.dequantize(kt, kb[b, j], Hkv * D) for j in range(nkv)]) for b in range(B)])
    vd = np.stack([np.stack([orc.dequantize(vt, vb[b, j], Hkv * D) for j in range(nkv)]) for b in range(B)])
    mt = None
    if mask is not None:
        mt = view(mask, F16, [nkv, nq, 1, 1], [2, 2 * nkv, 2 * nkv * nq, 2 * nkv * nq])
    keep = (q, kb, vb, mask)
    return dict(q=q, kd=kd.reshape(B, nkv, Hkv, D), vd=vd.reshape(B, nkv, Hkv, D), qt=qt, kt=ktd, vt=vtd, mt=mt,
                keep=keep, H=H, Hkv=Hkv, nq=nq, nkv=nkv, B=B)


def torch_ref(p, scale, mask_bits=None):
    q = torch.from_numpy(p["q"]).double().permute(0, 2, 1, 3)  # B H nq D
    k = torch.from_numpy(p["kd"]).double().permute(0, 2, 1, 3)
    v = torch.from_numpy(p["vd"]).double().permute(0, 2, 1, 3)
    rep = p["H"] // p["Hkv"]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    am = None
    if mask_bits is not None:
        am = torch.from_numpy(mask_bits.view(np.float16).astype(np.float64))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=am, scale=scale)
    return o.permute(0, 2, 1, 3).numpy()  # B nq H D


@pytest.mark.parametrize("kt,vt", [(F16, F16), (Q8_0, Q4_0), (Q8_0, Q8_0), (Q5_1, Q4_1), (Q5_0, F32), (F32, Q5_1)])
def test_oracle_matches_torch_sdpa(orc, rng, kt, vt):
    p = make_problem(orc, rng, kt=kt, vt=vt, B=2)
    got = orc.fa_f64(p["qt"], p["kt"], p["vt"], None, 0.125, (p["B"], p["nq"], p["H"], D))
    want = torch_ref(p, 0.125)
    assert np.abs(got - want).max() < 1e-6


def test_oracle_causal_mask_matches_torch(orc, rng):
    nq, nkv = 5, 21
    mask = orc.causal_mask(nq, nkv)
    p = make_problem(orc, rng, nq=nq, nkv=nkv, kt=Q8_0, vt=Q4_0, mask=mask)
    got = orc.fa_f64(p["qt"], p["kt"], p["vt"], p["mt"], 0.125, (1, nq, p["H"], D))
    want = torch_ref(p, 0.125, mask)
    assert np.abs(got - want).max() < 1e-6


def test_oracle_invariants(orc, rng):
    # n_kv = 1: output is the single V row of the kv head
    p = make_problem(orc, rng, nkv=1, kt=F16, vt=F16)
    got = orc.fa_f64(p["qt"], p["kt"], p["vt"], None, 0.125, (1, p["nq"], p["H"], D))
    for h in range(p["H"]):
        assert np.allclose(got[0, :, h], p["vd"][0, 0, h // 7], atol=1e-7)
    # permuting keys together with values changes nothing
    p = make_problem(orc, rng, nkv=33, kt=Q8_0, vt=Q4_0)
    base = orc.fa_f64(p["qt"], p["kt"], p["vt"], None, 0.125, (1, p["nq"], p["H"], D))
    perm = rng.permutation(33)
    _, kb, vb, _ = p["keep"]
    kb2, vb2 = np.ascontiguousarray(kb[:, perm]), np.ascontiguousarray(vb[:, perm])
    rk, rv = row_bytes(Q8_0, 128), row_bytes(Q4_0, 128)
    k2 = view(kb2, Q8_0, [D, 33, 2, 1], [34, rk, rk // 2, rk * 33])
    v2 = view(vb2, Q4_0, [D, 33, 2, 1], [18, rv, rv // 2, rv * 33])
    perm_out = orc.fa_f64(p["qt"], k2, v2, None, 0.125, (1, p["nq"], p["H"], D))
    assert np.abs(perm_out - base).max() < 1e-6
    # identical keys: plain mean of the V rows
    p = make_problem(orc, rng, nkv=9, kt=F32, vt=F32)
    _, kb, vb, _ = p["keep"]
    kb[:] = kb[:, :1]
    got = orc.fa_f64(p["qt"], p["kt"], p["vt"], None, 0.125, (1, p["nq"], p["H"], D))
    vmean = vb.view(np.float32).reshape(1, 9, 2, D).mean(axis=1)
    for h in range(p["H"]):
        assert np.allclose(got[0, :, h], vmean[0, h // 7], atol=1e-6)


def test_oracle_all_masked_row_is_zero(orc, rng):
    nq, nkv = 3, 10
    mask = np.zeros((nq, nkv), dtype=np.uint16)
    mask[1, :] = 0xFC00
    p = make_problem(orc, rng, nq=nq, nkv=nkv, mask=mask)
    got = orc.fa_f64(p["qt"], p["kt"], p["vt"], p["mt"], 0.125, (1, nq, p["H"], D))
    assert np.all(got[0, 1] == 0)
    assert np.all(np.abs(got[0, 0]) > 0)
    cpu = orc.fa_ggml_cpu(p["qt"], p["kt"], p["vt"], p["mt"], 0.125, (1, nq, p["H"], D))
    assert np.all(cpu[0, 1] == 0)


def test_oracle_gqa_equals_repeated_kv(orc, rng):
    p = make_problem(orc, rng, H=14, Hkv=2, kt=F32, vt=F32)
    got = orc.fa_f64(p["qt"], p["kt"], p["vt"], None, 0.125, (1, p["nq"], 14, D))
    _, kb, vb, _ = p["keep"]
    nkv = p["nkv"]
    k14 = np.repeat(kb.view(np.float32).reshape(nkv, 2, D), 7, axis=1).copy()
    v14 = np.repeat(vb.view(np.float32).reshape(nkv, 2, D), 7, axis=1).copy()
    row = 14 * D * 4
    kt = view(k14, F32, [D, nkv, 14, 1], [4, row, 4 * D, row * nkv])
    vt = view(v14, F32, [D, nkv, 14, 1], [4, row, 4 * D, row * nkv])
    rep = orc.fa_f64(p["qt"], kt, vt, None, 0.125, (1, p["nq"], 14, D))
    assert np.abs(got - rep).max() < 1e-7


@pytest.mark.parametrize("kt,vt,tol", [(F16, F16, 5e-3), (Q8_0, Q4_0, 2e-2), (F32, F32, 1e-5), (Q5_1, Q5_1, 2e-2)])
def test_ggml_cpu_restatement_close_to_f64(orc, rng, kt, vt, tol):
    nq, nkv = 4, 300
    mask = orc.causal_mask(nq, nkv)
    p = make_problem(orc, rng, nq=nq, nkv=nkv, kt=kt, vt=vt, mask=mask, B=2)
    ref = orc.fa_f64(p["qt"], p["kt"], p["vt"], p["mt"], 0.125, (2, nq, p["H"], D))
    cpu = orc.fa_ggml_cpu(p["qt"], p["kt"], p["vt"], p["mt"], 0.125, (2, nq, p["H"], D), n_threads=3)
    assert np.abs(cpu - ref).max() < tol
    cpu1 = orc.fa_ggml_cpu(p["qt"], p["kt"], p["vt"], p["mt"], 0.125, (2, nq, p["H"], D), n_threads=1)
    assert np.array_equal(cpu, cpu1)  # threading only splits rows


def test_nonfa_oracle_matches_fa(orc, rng):
    nq, nkv = 3, 17
    mask = orc.causal_mask(nq, nkv)
    p = make_problem(orc, rng, nq=nq, nkv=nkv, kt=F16, vt=F16, mask=mask)
    fa = orc.fa_f64(p["qt"], p["kt"], p["vt"], p["mt"], 0.125, (1, nq, 14, D))
    # transposed V cache [max_seq, H_kv*D] -> view [n_kv, D, H_kv, 1] (src/cosyvoice-kv-cache.cpp:326-348)
    vrows = p["keep"][2][0].view(np.uint16).reshape(nkv, 2 * D)
    vT = np.ascontiguousarray(vrows.T)  # [H_kv*D, n_kv]
    vt = view(vT, F16, [nkv, D, 2, 1], [2, 2 * nkv, 2 * nkv * D, 2 * nkv * D * 2])
    nonfa = orc.attn_nonfa_f64(p["qt"], p["kt"], vt, p["mt"], 0.125, (1, nq, 14, D))
    assert np.abs(fa - nonfa).max() < 1e-6


def test_causal_mask_bruteforce(orc):
    for nb, sl in [(1, 1), (1, 9), (4, 4), (5, 12), (256, 512)]:
        m = orc.causal_mask(nb, sl)
        i = np.arange(nb)[:, None]
        j = np.arange(sl)[None, :]
        want = np.where(j <= sl - nb + i, 0, 0xFC00)
        assert np.array_equal(m, want)


def test_chunk_mask_bruteforce(orc):
    for n, bounds in [(10, []), (10, [4]), (12, [3, 7, 12]), (50, [25, 50]), (7, [2, 2, 5])]:
        m = orc.chunk_mask(n, bounds)
        for i in range(n):
            end = next((b for b in bounds if b > i), n)
            want = [0 if j < end else 0xFC00 for j in range(n)]
            assert list(m[i]) == want


@pytest.mark.parametrize("t", [F32, F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1])
def test_set_rows_oracle(orc, rng, t):
    rows, ne0 = 16, 128
    rb = row_bytes(t, ne0)
    dst = rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)
    before = dst.copy()
    src = rng.standard_normal((3, ne0)).astype(np.float32)
    idx = np.array([5, 0, 13], dtype=np.int32)
    orc.set_rows(dst, t, rb, rows, src, idx)
    for r, i in enumerate(idx):
        assert np.array_equal(dst[i], orc.quantize(t, src[r]))
    untouched = [r for r in range(rows) if r not in idx]
    assert np.array_equal(dst[untouched], before[untouched])


def test_v_idxs_is_the_transposed_write():
    """Scattering V's elements through v_idxs (src/cosyvoice-kv-cache.cpp:338-343,357-377) equals
    writing each token's features down the token column of the [max_seq, n_embd, batch] cache."""
    from oracle.oracle import v_idxs
    rng = np.random.default_rng(3)
    for n_embd, max_seq, T, B in ((128, 40, 7, 1), (1024, 30, 5, 2), (8, 9, 9, 3)):
        pos = rng.permutation(max_seq)[:T]
        v = rng.standard_normal((B * T, n_embd)).astype(np.float32)   # token-major source rows
        flat = np.zeros(B * n_embd * max_seq, np.float32)
        flat[v_idxs(pos, B * T, T, n_embd, max_seq)] = v.reshape(-1)
        cache = flat.reshape(B, n_embd, max_seq)                      # [batch][feature][token]
        want = np.zeros_like(cache)
        for b in range(B):
            want[b][:, pos] = v[b * T:(b + 1) * T].T
        assert np.array_equal(cache, want)
        # every target distinct (no two elements collide)
        assert len(np.unique(v_idxs(pos, B * T, T, n_embd, max_seq))) == B * T * n_embd
