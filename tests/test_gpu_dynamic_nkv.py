"""GPU parity of plans whose KV length lives in device memory (cvattn_fa_batch_prepare_dynamic):
the reference decodes each token by reusing one graph and growing the views' ne[1] in place
(src/cosyvoice-llm.cpp:216-222 -> shift_kv_node_pos, src/cosyvoice-kv-cache.cpp:398-408).  Here
one captured HIP graph -- cvattn_shift_n_kv then the prepared launch -- is replayed per token and
each replay is checked against the fp64 oracle at that token's length."""
import ctypes

import numpy as np
import pytest
import torch

import cvattn
from _gpu import check_close, host, workspace
from oracle.oracle import F16, Q4_0, Q8_0
from test_gpu_attention import D, Case, dit_case, llm_case

pytestmark = pytest.mark.gpu


def with_nkv(t, n):
    """The same descriptor over its first n keys (ne[1] = n), as shift_kv_node_pos makes it."""
    u = type(t).from_buffer_copy(t)
    u.ne[1] = n
    return u


def problems_of(cases):
    probs = []
    for c in cases:
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.dst = c.q_d, c.k_d, c.v_d, c.dst_d
        if c.mask_d is not None:
            p.mask = c.mask_d
        probs.append(p)
    return probs


def check_at(orc, cases, n, what):
    for i, c in enumerate(cases):
        mask = None if c.mask_h is None else c.mask_h
        want = orc.fa_f64(c.q_h, with_nkv(c.k_h, n), with_nkv(c.v_h, n), mask, 0.125, c.out_shape)
        check_close(host(c.dst), want, what=f"{what}, problem {i}, n_kv {n}")


def test_graph_replays_follow_a_growing_cache(eng, orc, cuda):
    """Three decode layers (q8_0 K / q4_0 V, 14/2 heads) over a 4100-token capacity sharing one device
    length: one graph of [shift n_kv by 1, launch] replayed five times covers n_kv 4096..4100."""
    cap = 4100
    rng = np.random.default_rng(4096)
    cases = [llm_case(orc, rng, nq=1, nkv=cap, kt=Q8_0, vt=Q4_0, max_seq=cap) for _ in range(3)]
    probs = problems_of(cases)
    n_kv = torch.tensor([4095], dtype=torch.int32, device="cuda:0")
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare_dynamic(probs, 0.125, n_kv.data_ptr(), 0, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK, eng.status_string(rc)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        assert eng.shift_n_kv(n_kv.data_ptr(), 1, 1, stream.cuda_stream) == cvattn.OK
        assert eng.fa_batch_launch(plan, stream.cuda_stream) == cvattn.OK
    torch.cuda.synchronize()
    assert int(n_kv.item()) == 4095   # capture records, it does not run
    for step in range(5):
        for c in cases:
            c.dst.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        n = 4096 + step
        assert int(n_kv.item()) == n
        check_at(orc, cases, n, "graph replay")


@pytest.mark.parametrize("n", [0, 1, 37, 129, 2048, 4100, 5000])
def test_lengths_set_from_the_host(eng, orc, n, cuda):
    """Per-problem lengths (stride 1) written by a copy before the launch: short lengths leave most
    planned splits empty (they merge with weight 0), 0 gives zeros, and a length past the capacity
    is clamped to it."""
    cap = 4100
    rng = np.random.default_rng(n)
    cases = [llm_case(orc, rng, nq=1, nkv=cap, kt=Q8_0, vt=Q8_0, max_seq=cap) for _ in range(2)]
    probs = problems_of(cases)
    lens = [n, max(0, n // 2)]
    n_kv = torch.tensor(lens, dtype=torch.int32, device="cuda:0")
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare_dynamic(probs, 0.125, n_kv.data_ptr(), 1, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    for _ in range(2):   # the arrival counters reset themselves, empty splits included
        for c in cases:
            c.dst.fill_(float("nan"))
        assert eng.fa_batch_launch(plan) == cvattn.OK
    torch.cuda.synchronize()
    for c, m in zip(cases, lens):
        m = min(m, cap)
        if m == 0:
            assert np.all(host(c.dst) == 0.0)
        else:
            check_at(orc, [c], m, "host-set length")


def test_row_tiled_problems_follow_the_device_length(eng, orc, cuda):
    """Problems with more than 64 query rows per kv head (the row-tiled kernel, two key halves and
    token splits over a long capacity): 200 DiT-shaped rows over f16 K/V of capacity 3000."""
    rng = np.random.default_rng(7)
    c = dit_case(orc, rng, T=3000, Tq=200, ttype=F16)
    probs = problems_of([c])
    n_kv = torch.tensor([0], dtype=torch.int32, device="cuda:0")
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare_dynamic(probs, 0.125, n_kv.data_ptr(), 0, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    for n in (3000, 333, 1000, 64, 2999):
        n_kv.fill_(n)
        c.dst.fill_(float("nan"))
        assert eng.fa_batch_launch(plan) == cvattn.OK
        torch.cuda.synchronize()
        check_at(orc, [c], n, "row-tiled")


def test_classified_mask_follows_the_device_length(eng, orc, cuda):
    """A mask shared by every head with more row groups than CUs (the classified form: the
    classification runs at each launch over the keys below the device length, whose last tile
    may be partial), over f16 K/V of capacity 700."""
    from test_gpu_mask_classes import tiled_mask
    rng = np.random.default_rng(11)
    T = 700
    c = dit_case(orc, rng, T=T, B=2, H=16, mask=tiled_mask(rng, T, T, 64), ttype=F16)
    probs = problems_of([c])
    n_kv = torch.tensor([0], dtype=torch.int32, device="cuda:0")
    ws = workspace(eng.fa_batch_workspace(probs))
    rc, plan = eng.fa_batch_prepare_dynamic(probs, 0.125, n_kv.data_ptr(), 0, ws.data_ptr(), ws.numel())
    assert rc == cvattn.OK
    for n in (700, 333, 64, 129, 699):
        n_kv.fill_(n)
        c.dst.fill_(float("nan"))
        assert eng.fa_batch_launch(plan) == cvattn.OK
        torch.cuda.synchronize()
        check_at(orc, [c], n, "classified mask")
