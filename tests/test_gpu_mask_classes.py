"""GPU parity of the mask tile classes (the row-tiled kernel reads, per 64-row group and 64-key
tile, whether a mask shared by every head and sequence is all zero, all -inf, or neither).  The
masks are built tile by tile so that every class and its near misses occur: all +0/-0, all -inf,
zero but for one tiny bias, -inf but for one visible key, random finite biases, and a last tile
that the keys end inside.  Checked against the fp64 oracle through single calls and prepared
batches (launched twice: the classes are recomputed at every launch), for the DiT shape (one query
row per row) and the LLM prefill shape (7 query heads per kv head, so a row group spans about nine
query tokens).  Bar: max-abs <= 2e-3, mean-abs <= 2e-4."""
import numpy as np
import pytest
import torch

import cvattn
from _gpu import check_close, host, workspace
from oracle.oracle import F16, Q8_0
from test_gpu_attention import D, dit_case, llm_case, run_case

pytestmark = pytest.mark.gpu
NEG_INF = np.float16(-np.inf)


def tiled_mask(rng, nq, nkv, row_tile):
    """[nq, nkv] f16 mask: the key tiles of each block of row_tile query rows get one of the
    patterns below; every row keeps at least one visible key."""
    m = np.zeros((nq, nkv), dtype=np.float16)
    kinds = ["zero", "negzero", "off", "spike", "hole", "bias"]
    for q0 in range(0, nq, row_tile):
        for k0 in range(0, nkv, 64):
            blk = m[q0:q0 + row_tile, k0:k0 + 64]
            kind = kinds[rng.integers(len(kinds))]
            if kind == "negzero":
                blk[:] = np.float16(-0.0)
            elif kind == "off":
                blk[:] = NEG_INF
            elif kind == "spike":   # zero but one entry: the tile is not all zero
                blk[rng.integers(blk.shape[0]), rng.integers(blk.shape[1])] = np.float16(1e-3)
            elif kind == "hole":    # -inf but one visible key: the tile is not all -inf
                blk[:] = NEG_INF
                blk[rng.integers(blk.shape[0]), rng.integers(blk.shape[1])] = np.float16(0.5)
            elif kind == "bias":
                blk[:] = rng.standard_normal(blk.shape).astype(np.float16)
    m[:, 0] = np.float16(0.0)       # every row sees key 0
    return m.view(np.uint16)


def batch_run(eng, cases, launches=2):
    probs = []
    for c in cases:
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.mask, p.dst = c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d
        probs.append(p)
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare(probs, 0.125, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK, eng.status_string(rc)
    for _ in range(launches):
        for c in cases:
            c.dst.fill_(float("nan"))
        assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()


@pytest.mark.parametrize("T", [700, 1500])
def test_dit_tile_patterns(eng, orc, rng, T, cuda):
    """16 heads x batch 2: more row groups than CUs, the classified form."""
    mask = tiled_mask(rng, T, T, 64)
    c = dit_case(orc, rng, T=T, B=2, H=16, mask=mask, ttype=F16)
    run_case(eng, orc, c, what=f"DiT T={T}, single call")
    batch_run(eng, [c])
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, 0.125, c.out_shape)
    check_close(host(c.dst), want, what=f"DiT T={T}, prepared batch")


def test_dit_chunk_mask_rows_shared_by_tiles(eng, orc, rng, cuda):
    """The DiT chunk mask (each 50-frame chunk sees itself and every earlier chunk): tiles below
    the staircase are all zero, above it all -inf, on it mixed."""
    T = 1000
    chunk = (np.arange(T) // 50 + 1) * 50
    mask = np.where(np.arange(T)[None, :] < chunk[:, None], np.float16(0), NEG_INF).astype(np.float16).view(np.uint16)
    c = dit_case(orc, rng, T=T, B=2, H=16, mask=mask, ttype=F16)
    run_case(eng, orc, c, what="chunk mask, single call")


@pytest.mark.parametrize("nq,nkv", [(1200, 1200), (1300, 3000)])
def test_llm_prefill_row_groups_across_query_tokens(eng, orc, rng, nq, nkv, cuda):
    """7 query heads per kv head: row r of a row group is query r // 7, so a group's mask rows are
    a run of about nine query tokens (>= 1200 queries: more row groups than CUs, classified)."""
    mask = tiled_mask(rng, nq, nkv, 9)
    c = llm_case(orc, rng, nq=nq, nkv=nkv, kt=Q8_0, vt=Q8_0, max_seq=nkv, mask=mask, qscale=0.5)
    run_case(eng, orc, c, what=f"prefill {nq}x{nkv}, single call")
    batch_run(eng, [c, llm_case(orc, rng, nq=nq, nkv=nkv, kt=Q8_0, vt=Q8_0, max_seq=nkv, mask=mask, qscale=0.5)])
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, 0.125, c.out_shape)
    check_close(host(c.dst), want, what=f"prefill {nq}x{nkv}, prepared batch")


def test_causal_prefill_classes(eng, orc, rng, cuda):
    mask = orc.causal_mask(2048, 2048)
    c = llm_case(orc, rng, nq=2048, nkv=2048, kt=F16, vt=F16, max_seq=2048, mask=mask, qscale=0.5)
    run_case(eng, orc, c, what="causal 2048")


def test_split_token_ranges_with_classes(eng, orc, rng, cuda):
    """Classified row groups whose key range is split over workgroups (few query rows over a
    long cache would split; here a long masked DiT-shaped call whose row groups exceed the CUs)."""
    T = 3000
    mask = tiled_mask(rng, T, T, 64)
    c = dit_case(orc, rng, T=T, Tq=T, B=1, H=8, mask=mask, ttype=F16)
    run_case(eng, orc, c, what="T=3000 tiled mask")


def test_misaligned_workspace_rejected(eng, orc, rng, cuda):
    """The class tables and split partials are written with aligned vector stores: a workspace
    that is not 256-byte aligned is refused (CVATTN_ERR_BAD_ARGS) by single calls and by batch
    preparation, before anything is launched; the aligned one runs."""
    T = 700
    c = dit_case(orc, rng, T=T, B=2, H=16, mask=tiled_mask(rng, T, T, 64), ttype=F16)
    nws = eng.flash_attn_ext_workspace(c.q_d, c.k_d, c.v_d, c.mask_d)
    assert nws > 0  # the class table at least
    ws = workspace(nws + 256)
    base = ws.data_ptr()
    assert base % 256 == 0
    rc = eng.flash_attn_ext(c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d, 0.125, base + 16, nws)
    assert rc == cvattn.ERR_BAD_ARGS, eng.status_string(rc)
    assert eng.flash_attn_ext(c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d, 0.125, base, nws) == cvattn.OK
    p = cvattn.FaProblem()
    p.q, p.k, p.v, p.mask, p.dst = c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d
    nb = eng.fa_batch_workspace([p])
    wb = workspace(nb + 256)
    rc, _ = eng.fa_batch_prepare([p], 0.125, wb.data_ptr() + 64, nb)
    assert rc == cvattn.ERR_BAD_ARGS, eng.status_string(rc)
    torch.cuda.synchronize()


def test_prepared_batch_with_ragged_lengths(eng, orc, rng, cuda):
    """Two prefill problems with different key lengths in one prepared batch (more row groups
    than CUs together, so classified): each has its own class table, located by its first block
    in the launch; checked over two launches."""
    a = llm_case(orc, rng, nq=1200, nkv=1300, kt=Q8_0, vt=Q8_0, max_seq=1300,
                 mask=tiled_mask(rng, 1200, 1300, 9), qscale=0.5)
    b = llm_case(orc, rng, nq=1200, nkv=2100, kt=Q8_0, vt=Q8_0, max_seq=2100,
                 mask=tiled_mask(rng, 1200, 2100, 9), qscale=0.5)
    batch_run(eng, [a, b])
    for i, c in enumerate((a, b)):
        want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"ragged batch, problem {i}")
