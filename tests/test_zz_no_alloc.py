"""cvattn_flash_attn_ext_noalloc (the entry point that allocates nothing: its workspace is the
library's fixed per-GPU scratch array) against cvattn_flash_attn_ext with a caller workspace, on
calls in a row whose workspace needs shrink: the results must be bit-identical (same kernels, same
inputs), and within the parity bar of the fp64 oracle."""
import numpy as np
import pytest
import torch

import cvattn
from _gpu import check_close, empty_f32, host, run_fa
from oracle.oracle import F32, Q4_0, Q8_0
from test_gpu_attention import D, dit_case, llm_case

pytestmark = pytest.mark.gpu


def both(eng, orc, c, scale=0.125):
    """(noalloc output, caller-workspace output), each checked against the oracle."""
    c.dst.fill_(float("nan"))
    rc = eng.flash_attn_ext_noalloc(c.q_d, c.k_d, c.v_d, c.mask_d, c.dst_d, scale)
    assert rc == cvattn.OK, eng.status_string(rc)
    torch.cuda.synchronize()
    got = host(c.dst).copy()
    ref = empty_f32(*c.out_shape)
    B, nq, H, _ = c.out_shape
    run_fa(eng, c.q_d, c.k_d, c.v_d, c.mask_d, cvattn.out_view(ref.data_ptr(), D, H, nq, B), scale)
    want = orc.fa_f64(c.q_h, c.k_h, c.v_h, c.mask_h, scale, c.out_shape)
    check_close(got, want, what="noalloc vs oracle")
    return got, host(ref)


def test_noalloc_matches_the_workspace_call_on_shrinking_calls(eng, orc, cuda):
    rng = np.random.default_rng(77)
    # 1) the DiT call from fp32 views: the scratch holds the fp16 copies of K and V (12.3 MB)
    big = dit_case(orc, rng, T=1500)
    assert eng.flash_attn_ext_workspace(big.q_d, big.k_d, big.v_d, None) > 8 << 20
    got, ref = both(eng, orc, big)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # 2) a smaller call right after: a 4096-token decode split over the chip (split partials in
    #    the scratch, over bytes the first call left behind)
    small = llm_case(orc, rng, nq=1, nkv=4096, kt=Q8_0, vt=Q4_0, max_seq=4096)
    ws = eng.flash_attn_ext_workspace(small.q_d, small.k_d, small.v_d, None)
    assert 0 < ws < 1 << 20
    got, ref = both(eng, orc, small)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # 3) and a smaller fp32-view DiT call again
    mid = dit_case(orc, rng, T=300)
    got, ref = both(eng, orc, mid)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_refuses_shapes_past_its_scratch(eng, cuda):
    T, B = 5000, 2
    q = torch.empty((B, T, 1024), dtype=torch.float32, device="cuda:0")
    qv = cvattn.dit_view(q.data_ptr(), T, B)
    need = eng.flash_attn_ext_workspace(qv, qv, qv, None)
    assert need > cvattn.NOALLOC_SCRATCH_BYTES
    out = empty_f32(B, T, 16, D)
    rc = eng.flash_attn_ext_noalloc(qv, qv, qv, None, cvattn.out_view(out.data_ptr(), D, 16, T, B), 0.125)
    assert rc == cvattn.ERR_WORKSPACE_TOO_SMALL
