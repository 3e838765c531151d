#!/usr/bin/env python3
"""Benchmark of the attention engine on one MI355X.

Workload (the metric's configuration): full 24-layer Qwen2-0.5B-shape decode attention for one
token, batch 1, 14 query / 2 KV heads, head_dim 64, 4096 cached tokens, K cache q8_0 and V cache
q4_0 produced by ggml's reference quantizers (cvattn_set_rows, bit-exact to quantize_row_*_ref)
from seeded N(0,1) values, N(0,1) queries, scale 1/8.

A step is one token's attention over all 24 layers, run as one prepared batch
(cvattn_fa_batch_launch: one kernel, split partials merged in-kernel).  R independent copies of
the 24-layer cache (R * 20.6 MB >= 512 MB) are cycled so every step streams its KV bytes from HBM,
not from the 256 MB Infinity Cache.  Exactly --steps steps are captured in one HIP graph (step i
reads copy i mod R; graphs starting at different copies alternate so consecutive replays never
re-read a copy); after --warmup untimed steps the graph is replayed 25 times, each replay
bracketed by HIP events on the replay stream, and ms_per_step is the median replay time / steps.

Reported alongside, measured in the same run:
  * the real decode cadence: 24 dependent per-layer launches per token (the headline tok/s),
    through prepared plans and through the drop-in single call cvattn_flash_attn_ext with n_kv
    growing by one per token;
  * flow-DiT attention (T=1500, batch 2 for CFG, 16 heads) TFLOP/s, as f16 views through a
    prepared batch and as the fp32 views the flow graph passes (single calls, also per utterance:
    22 layers x 10 ODE steps);
  * the 1024-token causal prefill, the DiT streaming chunk and the 16-sequence serving step;
  * the CPU baseline: the ggml CPU flash-attention loop restated in oracle/ (a port, built -O3 for
    x86-64-v3 like ggml's CPU backend), timed on a bounded sample of the same decode workload on
    the host cores.

python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "cosyvoice.cpp_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP16_DENSE_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA

L, H, HKV, D, NKV, MAX_SEQ = 24, 14, 2, 64, 4096, 4096
KT_NAME, VT_NAME = "q8_0", "q4_0"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def decode_bytes_per_layer(kt_bytes, vt_bytes, n_kv=NKV):
    # n_kv * H_kv * (D/32) * (bK + bV) + Q + O (f32)
    return n_kv * HKV * (D // 32) * (kt_bytes + vt_bytes) + 2 * H * D * 4


def build_decode(lib, cvattn, torch, dev, n_copies, kt, vt):
    """R copies x 24 layers of K/V caches quantized on the device, plus Q and outputs."""
    rk = cvattn.row_bytes(kt, HKV * D)
    rv = cvattn.row_bytes(vt, HKV * D)
    kbuf = torch.empty((n_copies, L, MAX_SEQ, rk), dtype=torch.uint8, device=dev)
    vbuf = torch.empty((n_copies, L, MAX_SEQ, rv), dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261201)
    idx = torch.arange(MAX_SEQ, dtype=torch.int32, device=dev)
    it = cvattn.contiguous(idx.data_ptr(), cvattn.I32, [MAX_SEQ, 1, 1, 1])
    src = torch.empty((MAX_SEQ, HKV * D), dtype=torch.float32, device=dev)
    st = cvattn.contiguous(src.data_ptr(), cvattn.F32, [HKV * D, MAX_SEQ, 1, 1])
    for r in range(n_copies):
        for layer in range(L):
            for buf, t in ((kbuf, kt), (vbuf, vt)):
                src.normal_(generator=gen)
                dt = cvattn.contiguous(buf[r, layer].data_ptr(), t, [HKV * D, MAX_SEQ, 1, 1])
                rc = lib.set_rows(dt, st, it)
                assert rc == cvattn.OK, lib.status_string(rc)
    q = torch.randn((n_copies, L, H, D), generator=gen, device=dev, dtype=torch.float32)
    out = torch.zeros((n_copies, L, H, D), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def problem(r, layer):
        p = cvattn.FaProblem()
        p.q = cvattn.llm_q_view(q[r, layer].data_ptr(), D, H, 1)
        p.k = cvattn.llm_kv_view(kbuf[r, layer].data_ptr(), kt, D, HKV, NKV, MAX_SEQ)
        p.v = cvattn.llm_kv_view(vbuf[r, layer].data_ptr(), vt, D, HKV, NKV, MAX_SEQ)
        p.dst = cvattn.out_view(out[r, layer].data_ptr(), D, H, 1)
        return p

    return kbuf, vbuf, q, out, problem


def make_plan(lib, cvattn, torch, dev, probs, keep):
    wsb = lib.fa_batch_workspace(probs)
    assert wsb > 0, "batch rejected"
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    keep.append(ws)
    rc, plan = lib.fa_batch_prepare(probs, 1.0 / math.sqrt(D), ws.data_ptr(), ws.numel(),
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == cvattn.OK, lib.status_string(rc)
    keep.append(plan)
    return plan


TIMED_REPEATS = 25
# untimed DiT calls before a DiT leg is timed: on MI355X the T=1500 call settles from ~35 us to
# ~31 us over its first few hundred back-to-back calls (an utterance makes 220 of them)
DIT_WARMUP_CALLS = 1000
# untimed graph replays before the prefill, DiT-stream and serving legs (tens of milliseconds of
# load, for the same clock settling), and before the layer-sequential decode cadence
SETTLE_REPLAYS = 100
CADENCE_SETTLE_REPLAYS = 10


def time_graphs(torch, launch_fns, n_per_graph, warmup_steps, repeats=TIMED_REPEATS):
    """Capture each launch_fn (n_per_graph steps each) in its own HIP graph; replay the graphs in
    turn, first untimed for warmup_steps steps, then `repeats` times with each replay bracketed by
    HIP events on the replay stream.  Returns (median ms per step, per-replay ms list)."""
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    graphs = []
    for fn in launch_fns:
        with torch.cuda.stream(stream):
            fn(stream.cuda_stream)  # eager warm-up of the code path
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn(stream.cuda_stream)
        graphs.append(g)
    torch.cuda.synchronize()
    for i in range(max(1, math.ceil(warmup_steps / n_per_graph))):
        graphs[i % len(graphs)].replay()
    cur = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(repeats)]
    torch.cuda.synchronize()
    for i in range(repeats):
        ev[i][0].record(cur)
        graphs[i % len(graphs)].replay()
        ev[i][1].record(cur)
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) for a, b in ev]
    return statistics.median(per) / n_per_graph, per


def time_graph(torch, launch_fn, n_per_graph, warmup_steps, repeats=TIMED_REPEATS):
    return time_graphs(torch, [launch_fn], n_per_graph, warmup_steps, repeats)[0]


def decode_cadence(lib, cvattn, torch, dev, problem, n_copies, keep):
    """The real decode cadence: 24 dependent per-layer launches per token, from plans prepared on
    the host and from plans reading a device-resident n_kv (one graph replay per token runs
    [cvattn_shift_n_kv +1, 24 layer launches] for each copy, so n_kv grows by one per replay).
    Returns (ms per token, ms per token with device n_kv)."""
    layer_plans = [[make_plan(lib, cvattn, torch, dev, [problem(r, l)], keep) for l in range(L)]
                   for r in range(n_copies)]

    def launch_layers(s):
        for r in range(n_copies):
            for p in layer_plans[r]:
                assert lib.fa_batch_launch(p, s) == cvattn.OK

    ms_seq = time_graph(torch, launch_layers, n_copies, CADENCE_SETTLE_REPLAYS * n_copies)
    log(f"decode 24 sequential layer launches: {ms_seq * 1e3:.2f} us/token")

    n_kv_dev = torch.full((n_copies,), NKV - 64, dtype=torch.int32, device=dev)
    dyn_plans = []
    for r in range(n_copies):
        row = []
        for l_ in range(L):
            probs = [problem(r, l_)]
            wsb = lib.fa_batch_workspace(probs)
            ws_ = torch.empty(wsb, dtype=torch.uint8, device=dev)
            keep.append(ws_)
            rc, pl = lib.fa_batch_prepare_dynamic(probs, 1.0 / math.sqrt(D), n_kv_dev[r:].data_ptr(), 0,
                                                  ws_.data_ptr(), wsb, torch.cuda.current_stream().cuda_stream)
            assert rc == cvattn.OK, lib.status_string(rc)
            keep.append(pl)
            row.append(pl)
        dyn_plans.append(row)

    def launch_dynamic(s):
        for r in range(n_copies):
            assert lib.shift_n_kv(n_kv_dev[r:].data_ptr(), 1, 1, s) == cvattn.OK
            for p in dyn_plans[r]:
                assert lib.fa_batch_launch(p, s) == cvattn.OK

    ms_dyn = time_graph(torch, launch_dynamic, n_copies, 0)
    log(f"decode per-token graph with device n_kv: {ms_dyn * 1e3:.2f} us/token")
    return ms_seq, ms_dyn


def bench_dit(lib, cvattn, torch, dev):
    """Flow-DiT attention layer call: T=1500, B=2, 16 heads, fp16 q/k/v views, no mask, through a
    prepared batch (10 calls per graph replay)."""
    T, B, HD = 1500, 2, 16
    q = torch.randn((B, T, HD * D), device=dev, dtype=torch.float16)
    k = torch.randn((B, T, HD * D), device=dev, dtype=torch.float16)
    v = torch.randn((B, T, HD * D), device=dev, dtype=torch.float16)
    out = torch.empty((B, T, HD, D), device=dev, dtype=torch.float32)
    p = cvattn.FaProblem()
    p.q = cvattn.dit_view(q.data_ptr(), T, B, ttype=cvattn.F16)
    p.k = cvattn.dit_view(k.data_ptr(), T, B, ttype=cvattn.F16)
    p.v = cvattn.dit_view(v.data_ptr(), T, B, ttype=cvattn.F16)
    p.dst = cvattn.out_view(out.data_ptr(), D, HD, T, B)
    keep = []
    plan = make_plan(lib, cvattn, torch, dev, [p], keep)

    def launch(s):
        for _ in range(10):
            assert lib.fa_batch_launch(plan, s) == cvattn.OK

    ms = time_graph(torch, launch, 10, DIT_WARMUP_CALLS)
    flops = 4.0 * D * B * HD * T * T
    return {"workload": "flow-DiT attention layer call, T=1500, batch 2, 16 heads, head_dim 64, fp16, no mask",
            "ms_per_layer_call": ms, "tflops": flops / (ms * 1e-3) / 1e12,
            "mfma_frac": flops / (ms * 1e-3) / 1e12 / FP16_DENSE_PEAK_TFLOPS, "flop_per_call": flops,
            "timed": f"median of {TIMED_REPEATS} graph replays of 10 calls, after {DIT_WARMUP_CALLS} untimed calls"}


def bench_dit_masked(lib, cvattn, torch, dev):
    """The uncached streaming DiT call after the first chunk (src/cosyvoice-token2wav.cpp:285-298):
    T=1500, a chunk boundary every 50 frames, f16 q/k/v through a prepared batch.  FLOPs count the
    visible (row, key) pairs only."""
    T, B, HD = 1500, 2, 16
    q = torch.randn((B, T, HD * D), device=dev, dtype=torch.float16)
    k = torch.randn((B, T, HD * D), device=dev, dtype=torch.float16)
    v = torch.randn((B, T, HD * D), device=dev, dtype=torch.float16)
    out = torch.empty((B, T, HD, D), device=dev, dtype=torch.float32)
    mask = torch.empty((T, T), device=dev, dtype=torch.float16)
    bounds = list(range(50, T, 50))
    assert lib.chunk_mask(cvattn.mask_view(mask.data_ptr(), T, T), bounds) == cvattn.OK
    p = cvattn.FaProblem()
    p.q = cvattn.dit_view(q.data_ptr(), T, B, ttype=cvattn.F16)
    p.k = cvattn.dit_view(k.data_ptr(), T, B, ttype=cvattn.F16)
    p.v = cvattn.dit_view(v.data_ptr(), T, B, ttype=cvattn.F16)
    p.mask = cvattn.mask_view(mask.data_ptr(), T, T)
    p.dst = cvattn.out_view(out.data_ptr(), D, HD, T, B)
    keep = []
    plan = make_plan(lib, cvattn, torch, dev, [p], keep)

    def launch(s):
        for _ in range(10):
            assert lib.fa_batch_launch(plan, s) == cvattn.OK

    ms = time_graph(torch, launch, 10, DIT_WARMUP_CALLS)
    # row i sees keys j < the first boundary above i (all T for the last chunk)
    visible = sum(next((b_ for b_ in bounds if b_ > i), T) for i in range(T))
    flops = 4.0 * D * B * HD * visible
    return {"workload": "flow-DiT attention layer call with the 50-frame chunk mask, T=1500, batch 2, 16 heads, f16",
            "us_per_layer_call": ms * 1e3, "tflops_visible": flops / (ms * 1e-3) / 1e12,
            "visible_fraction": visible / (T * T)}


def bench_dit_f32_views(lib, cvattn, torch, dev):
    """The same DiT call in the form the flow graph passes it (src/cosyvoice-graph.cpp:370-376):
    fp32 q/k/v views of the rope and linear outputs, one cvattn_flash_attn_ext call with its
    workspace (which holds the fp16 copies of K and V made inside the call).  Timed two ways:
    graph-replayed calls, and one utterance's 220 calls (22 layers x 10 ODE steps) issued eagerly
    from the host as a ggml backend would issue them."""
    T, B, HD = 1500, 2, 16
    q = torch.randn((B, T, HD * D), device=dev)
    k = torch.randn((B, T, HD * D), device=dev)
    v = torch.randn((B, T, HD * D), device=dev)
    out = torch.empty((B, T, HD, D), device=dev, dtype=torch.float32)
    qv = cvattn.dit_view(q.data_ptr(), T, B, ttype=cvattn.F32)
    kv = cvattn.dit_view(k.data_ptr(), T, B, ttype=cvattn.F32)
    vv = cvattn.dit_view(v.data_ptr(), T, B, ttype=cvattn.F32)
    dst = cvattn.out_view(out.data_ptr(), D, HD, T, B)
    nws = lib.flash_attn_ext_workspace(qv, kv, vv, None)
    ws = torch.empty(max(1, nws), dtype=torch.uint8, device=dev)

    def launch(s):
        for _ in range(10):
            assert lib.flash_attn_ext(qv, kv, vv, None, dst, 0.125, ws.data_ptr(), nws, s) == cvattn.OK

    ms = time_graph(torch, launch, 10, DIT_WARMUP_CALLS)
    flops = 4.0 * D * B * HD * T * T
    # one utterance, eager: 220 calls on the current stream
    s = torch.cuda.current_stream().cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per_utt = []
    for _ in range(5):
        torch.cuda.synchronize()
        e0.record()
        for _ in range(220):
            assert lib.flash_attn_ext(qv, kv, vv, None, dst, 0.125, ws.data_ptr(), nws, s) == cvattn.OK
        e1.record()
        torch.cuda.synchronize()
        per_utt.append(e0.elapsed_time(e1))
    return {"workload": "flow-DiT attention layer call, T=1500, batch 2, 16 heads, fp32 q/k/v views, single call",
            "us_per_layer_call": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12, "workspace_bytes": nws,
            "ms_per_utterance_eager_220_calls": statistics.median(per_utt)}


def bench_prefill(lib, cvattn, torch, dev):
    """LLM prefill layer call: 1024 query tokens over 1024 f16 cached tokens, causal mask, 14/2 heads
    (Q, K, V ~ 0.5 N(0,1)); 24 layers of the same shape are cycled.  Also the reference's own
    cadence (n_batch 256, src/cosyvoice-model.cpp:53; src/cosyvoice-llm.cpp:101-108): four calls of
    256 query rows over 256/512/768/1024 keys per layer."""
    nq = nkv = 1024
    layers = []
    for _ in range(L):
        kc = (0.5 * torch.randn((nkv, HKV * D), device=dev)).half()
        vc = (0.5 * torch.randn((nkv, HKV * D), device=dev)).half()
        q = 0.5 * torch.randn((nq, H, D), device=dev)
        layers.append((kc, vc, q))
    i = torch.arange(nq, device=dev).view(-1, 1)
    j = torch.arange(nkv, device=dev).view(1, -1)
    mask = torch.where(j <= nkv - nq + i, 0.0, float("-inf")).half().contiguous()
    out = torch.empty((nq, H, D), device=dev, dtype=torch.float32)
    keep = []
    plans, chunk_plans = [], []
    for kc, vc, q in layers:
        p = cvattn.FaProblem()
        p.q = cvattn.llm_q_view(q.data_ptr(), D, H, nq)
        p.k = cvattn.llm_kv_view(kc.data_ptr(), cvattn.F16, D, HKV, nkv, nkv)
        p.v = cvattn.llm_kv_view(vc.data_ptr(), cvattn.F16, D, HKV, nkv, nkv)
        p.mask = cvattn.mask_view(mask.data_ptr(), nkv, nq)
        p.dst = cvattn.out_view(out.data_ptr(), D, H, nq)
        plans.append(make_plan(lib, cvattn, torch, dev, [p], keep))
        for c in range(4):
            n_kv_c = 256 * (c + 1)
            pc = cvattn.FaProblem()
            pc.q = cvattn.llm_q_view(q[256 * c].data_ptr(), D, H, 256)
            pc.k = cvattn.llm_kv_view(kc.data_ptr(), cvattn.F16, D, HKV, n_kv_c, nkv)
            pc.v = cvattn.llm_kv_view(vc.data_ptr(), cvattn.F16, D, HKV, n_kv_c, nkv)
            # rows 256c.. of the causal mask over the first n_kv_c keys: row i sees j <= 256c + i
            pc.mask = cvattn.tensor(mask[256 * c].data_ptr(), cvattn.F16, [n_kv_c, 256, 1, 1],
                                    [2, 2 * nkv, 2 * nkv * 256, 2 * nkv * 256])
            pc.dst = cvattn.out_view(out[256 * c].data_ptr(), D, H, 256)
            chunk_plans.append(make_plan(lib, cvattn, torch, dev, [pc], keep))

    def launch(s):
        for pl in plans:
            assert lib.fa_batch_launch(pl, s) == cvattn.OK

    def launch_chunks(s):
        for pl in chunk_plans:
            assert lib.fa_batch_launch(pl, s) == cvattn.OK

    ms = time_graph(torch, launch, L, SETTLE_REPLAYS * L)
    ms_chunks = time_graph(torch, launch_chunks, L, SETTLE_REPLAYS * L)  # ms per layer (4 launches)
    visible = sum(nkv - nq + ii + 1 for ii in range(nq))
    flops = 4.0 * D * H * visible
    # stored bytes per call: Q f32, K and V f16, O f32, the f16 mask
    nbytes = nq * H * D * 4 + 2 * nkv * HKV * D * 2 + nq * H * D * 4 + nq * nkv * 2
    return {"workload": "LLM prefill layer call, 1024 query tokens, causal mask, 1024 f16 cached tokens, 14/2 heads",
            "us_per_layer_call": ms * 1e3, "tflops": flops / (ms * 1e-3) / 1e12,
            "mfma_frac": flops / (ms * 1e-3) / 1e12 / FP16_DENSE_PEAK_TFLOPS,
            "bytes_per_call": nbytes, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "reference_cadence_4x256": {"us_per_layer": ms_chunks * 1e3,
                                        "tflops": flops / (ms_chunks * 1e-3) / 1e12,
                                        "calls": "256 rows over 256/512/768/1024 keys"}}


def bench_dit_stream(lib, cvattn, torch, dev):
    """Flow-DiT streaming call: a 50-frame query chunk over a cached 1000-frame prefix plus itself
    (n_kv 1050), batch 2, 16 heads, f16 cache views; 66 caches (3 x 22 layers, 568 MB) are cycled
    so each call streams its K/V from HBM, not from the 256 MB Infinity Cache."""
    nq, nkv, B, HD, NL = 50, 1050, 2, 16, 66
    caches = []
    for _ in range(NL):
        k = torch.randn((B, nkv, HD * D), device=dev).half()
        v = torch.randn((B, nkv, HD * D), device=dev).half()
        caches.append((k, v))
    q = torch.randn((B, nq, HD * D), device=dev)
    out = torch.empty((B, nq, HD, D), device=dev, dtype=torch.float32)
    keep, plans = [], []
    for k, v in caches:
        p = cvattn.FaProblem()
        p.q = cvattn.dit_view(q.data_ptr(), nq, B)
        p.k = cvattn.dit_view(k.data_ptr(), nkv, B, ttype=cvattn.F16)
        p.v = cvattn.dit_view(v.data_ptr(), nkv, B, ttype=cvattn.F16)
        p.dst = cvattn.out_view(out.data_ptr(), D, HD, nq, B)
        plans.append(make_plan(lib, cvattn, torch, dev, [p], keep))

    def launch(s):
        for pl in plans:
            assert lib.fa_batch_launch(pl, s) == cvattn.OK

    ms = time_graph(torch, launch, NL, SETTLE_REPLAYS * NL)
    nbytes = 2 * B * nkv * HD * D * 2 + 2 * B * nq * HD * D * 4
    return {"workload": "flow-DiT streaming call, 50-frame chunk over 1000 cached + 50 frames, batch 2, 16 heads, f16 cache",
            "us_per_layer_call": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9,
            "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "caches_cycled": NL,
            "bytes_cycled": NL * 2 * B * nkv * HD * D * 2}


def bench_serving(lib, cvattn, torch, dev):
    """Concurrent-serving decode: 16 sequences x 24 layers, K = V = q8_0, kv_len ~ U{256..8192} (seeded),
    one query token per sequence; a step is 24 launches, one prepared 16-problem batch per layer."""
    import numpy as np

    nseq = 16
    lens = np.random.default_rng(20261201).integers(256, 8193, nseq)
    rk = cvattn.row_bytes(cvattn.Q8_0, HKV * D)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    keep, plans = [], []
    total = 0
    for layer in range(L):
        probs = []
        for s_ in range(nseq):
            n = int(lens[s_])
            # random bytes are valid q8_0 blocks once each block's fp16 scale is made finite and small
            kc = torch.randint(0, 256, (n, rk), dtype=torch.uint8, device=dev, generator=gen)
            vc = torch.randint(0, 256, (n, rk), dtype=torch.uint8, device=dev, generator=gen)
            for t_ in (kc, vc):
                t_.view(n, rk // 34, 34)[:, :, 1] = 0x20
            q = torch.randn((H, D), device=dev)
            out = torch.empty((H, D), device=dev, dtype=torch.float32)
            keep += [kc, vc, q, out]
            p = cvattn.FaProblem()
            p.q = cvattn.llm_q_view(q.data_ptr(), D, H, 1)
            p.k = cvattn.llm_kv_view(kc.data_ptr(), cvattn.Q8_0, D, HKV, n, n)
            p.v = cvattn.llm_kv_view(vc.data_ptr(), cvattn.Q8_0, D, HKV, n, n)
            p.dst = cvattn.out_view(out.data_ptr(), D, H, 1)
            probs.append(p)
            total += n * HKV * 2 * (34 + 34) + 2 * H * D * 4
        plans.append(make_plan(lib, cvattn, torch, dev, probs, keep))

    def launch(s):
        for pl in plans:
            assert lib.fa_batch_launch(pl, s) == cvattn.OK

    ms = time_graph(torch, launch, L, SETTLE_REPLAYS * L)
    step_ms = ms * L
    return {"workload": "serving decode, 16 sequences x 24 layers, q8_0 K and V, ragged kv_len U{256..8192}, "
                        "one launch per layer", "kv_lens": [int(x) for x in lens],
            "us_per_step": step_ms * 1e3, "gbs": total / (step_ms * 1e-3) / 1e9,
            "hbm_frac": total / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "bytes_per_step": total}


def bench_single_call_decode(lib, cvattn, torch, dev, kbuf, vbuf, q, out, n_copies, kt, vt, tokens=64):
    """The drop-in path as a ggml backend drives it: per token, 24 cvattn_flash_attn_ext calls
    (one per layer, src/cosyvoice-llm-job.cpp:135-178 -> src/cosyvoice-llm.cpp:302) with n_kv read
    from the views at call time, growing by one per token from 4000; eager host issue, each
    token on its own cache copy.  GPU time per token from HIP events around the whole run."""
    s = torch.cuda.current_stream().cuda_stream
    n0 = NKV - tokens
    views = []
    wsb = 0
    for t in range(tokens):
        r = t % n_copies
        row = []
        for layer in range(L):
            qv = cvattn.llm_q_view(q[r, layer].data_ptr(), D, H, 1)
            kv = cvattn.llm_kv_view(kbuf[r, layer].data_ptr(), kt, D, HKV, n0 + t, MAX_SEQ)
            vv = cvattn.llm_kv_view(vbuf[r, layer].data_ptr(), vt, D, HKV, n0 + t, MAX_SEQ)
            dv = cvattn.out_view(out[r, layer].data_ptr(), D, H, 1)
            wsb = max(wsb, lib.flash_attn_ext_workspace(qv, kv, vv, None))
            row.append((qv, kv, vv, dv))
        views.append(row)
    ws = torch.empty(max(256, wsb), dtype=torch.uint8, device=dev)

    def run():
        for row in views:
            for qv, kv, vv, dv in row:
                assert lib.flash_attn_ext(qv, kv, vv, None, dv, 0.125, ws.data_ptr(), ws.numel(), s) == cvattn.OK

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per = []
    for _ in range(5):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record()
        run()
        e1.record()
        torch.cuda.synchronize()
        per.append((e0.elapsed_time(e1), time.perf_counter() - t0))
    gpu_ms = statistics.median(p[0] for p in per)
    host_s = statistics.median(p[1] for p in per)
    return {"workload": f"{tokens} tokens x 24 single cvattn_flash_attn_ext calls, n_kv {n0}..{NKV - 1}, "
                        "q8_0 K / q4_0 V, eager host issue", "us_per_token": gpu_ms * 1e3 / tokens,
            "tok_per_s": tokens / (gpu_ms * 1e-3), "host_wall_us_per_token": host_s * 1e6 / tokens}


def cpu_baseline(kbuf, vbuf, q, budget_s=12.0):
    """ggml CPU flash-attention loop (restated in oracle/, the -O3 x86-64-v3 build) on copy 0 of
    the decode workload."""
    import numpy as np

    from oracle.oracle import Q4_0, Q8_0, Oracle, row_bytes, view

    orc = Oracle(os.path.join(ROOT, "oracle", "liboracle_fast.so"))
    threads = min(H, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count())
    rk, rv = row_bytes(Q8_0, HKV * D), row_bytes(Q4_0, HKV * D)
    kh = kbuf[0].cpu().numpy()
    vh = vbuf[0].cpu().numpy()
    qh = q[0].cpu().numpy()
    layers_done, t0 = 0, time.perf_counter()
    while True:
        layer = layers_done % L
        qt = view(qh[layer], 0, [D, 1, H, 1], [4, 4 * D * H, 4 * D, 4 * D * H])
        kt = view(kh[layer], Q8_0, [D, NKV, HKV, 1], [34, rk, rk // HKV, rk * MAX_SEQ])
        vt = view(vh[layer], Q4_0, [D, NKV, HKV, 1], [18, rv, rv // HKV, rv * MAX_SEQ])
        orc.fa_ggml_cpu(qt, kt, vt, None, 0.125, (H, D), n_threads=threads)
        layers_done += 1
        el = time.perf_counter() - t0
        if layers_done % L == 0 and el >= budget_s:
            break
        if layers_done >= 200 * L:
            break
    sec_per_token = el / (layers_done / L)
    gbs = decode_bytes_per_layer(34, 18) * L / sec_per_token / 1e9
    return {"value": gbs, "unit": "GB/s", "cores": threads, "kind": "port",
            "host_cores": os.cpu_count(), "cpu_model": cpu_model(),
            "tok_per_s": 1.0 / sec_per_token,
            "sample": f"{layers_done // L} tokens x 24 layers of the same q8_0/q4_0 4096-token decode, "
                      f"ggml CPU flash-attention loop restated in C (oracle/oracle.c, -O3 x86-64-v3 build), "
                      f"{threads} threads; a lower bound on ggml's hand-vectorised CPU kernels"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def device_info(torch):
    p = torch.cuda.get_device_properties(0)
    return {"name": p.name, "gcn_arch": getattr(p, "gcnArchName", None), "compute_units": p.multi_processor_count,
            "hbm_bytes": p.total_memory}


TRAFFIC_PROFILE = os.path.join("profiles", "decode_q8_0_q4_0_24x4096_counters.md")


def read_traffic():
    """HBM bytes per launch of the decode kernel, from the rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    committed under profiles/ (counters cannot be read from inside this process)."""
    path = os.path.join(ROOT, TRAFFIC_PROFILE)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1])
            except ValueError:
                return None
    return None


def stream_floor(torch, dev):
    """What plain streaming kernels reach over a working set the size of one decode step
    (20,619,264 B), cycled over 27 buffers so the 256 MB last-level cache cannot hold it, and over
    4x and 16x that size: torch's device copy (read + write) and a sum (read)."""
    step = 20619264
    out = []
    for mult, n_buf in ((1, 27), (4, 4), (16, 4)):
        nbytes = step * mult
        bufs = [torch.randn(nbytes // 4, device=dev) for _ in range(n_buf)]
        dst = [torch.empty_like(bufs[0]) for _ in range(2)]
        red = torch.empty((), device=dev)

        def launch_copy(s):
            for i, b in enumerate(bufs):
                dst[i & 1].copy_(b)

        def launch_sum(s):
            for b in bufs:
                torch.sum(b, dim=0, out=red)

        for name, fn, moved in (("copy", launch_copy, 2 * nbytes), ("sum", launch_sum, nbytes)):
            ms = time_graph(torch, fn, n_buf, n_buf)
            out.append({"kernel": name, "working_set_bytes": nbytes, "us": ms * 1e3,
                        "gbs_moved": moved / (ms * 1e-3) / 1e9})
        del bufs, dst
    return {"stream_floor": out}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=27, help="decode steps per timed graph replay")
    # ~35 ms of untimed steps: the step settles ~2% faster once the clock has risen under load
    # (13.22-13.32 us after 27 steps, 13.05-13.06 us after 2700)
    ap.add_argument("--warmup", type=int, default=2700, help="untimed decode steps before timing")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-dit", action="store_true", help="skip the DiT legs")
    ap.add_argument("--no-extra", action="store_true", help="skip the prefill, DiT-stream, serving and single-call legs")
    ap.add_argument("--no-cadence", action="store_true",
                    help="skip the per-layer decode cadence legs (counter passes over the 24-layer step alone)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 256 MiB device copies (reference kernels for the HBM counters)")
    ap.add_argument("--stream-floor", action="store_true",
                    help="only time plain device copies and sums over the decode step's 20.6 MB working set "
                         "(27 copies cycled, as the decode leg), and over 4x and 16x that size")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (the attention path runs "
              "on one GPU: sequences, layers and DiT heads are independent work, so a multi-GPU form would "
              "shard them with no exchange inside attention)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        sys.exit(2)

    import torch

    import cvattn

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = 256 * 2**20 // 4
        a = torch.randn(n, device=dev)
        b = torch.empty_like(a)
        for _ in range(10):
            b.copy_(a)  # the runtime's blit kernel
        for _ in range(10):
            torch.neg(a, out=b)  # an elementwise kernel: plain vector loads and stores
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n * 4, "bytes_written": n * 4,
                          "launches": {"copyBuffer": 10, "neg": 10}}))
        return
    if args.stream_floor:
        print(json.dumps(stream_floor(torch, dev)))
        return
    lib = cvattn.lib()
    kt, vt = cvattn.Q8_0, cvattn.Q4_0
    per_layer = decode_bytes_per_layer(34, 18)
    per_copy = L * (MAX_SEQ * (cvattn.row_bytes(kt, HKV * D) + cvattn.row_bytes(vt, HKV * D)))
    n_copies = max(2, math.ceil(512 * 2**20 / per_copy))
    log(f"building {n_copies} copies of the 24-layer q8_0/q4_0 cache ({n_copies * per_copy / 2**20:.0f} MiB)")
    kbuf, vbuf, q, out, problem = build_decode(lib, cvattn, torch, dev, n_copies, kt, vt)

    keep = []
    plans = [make_plan(lib, cvattn, torch, dev, [problem(r, l) for l in range(L)], keep) for r in range(n_copies)]

    # exactly K steps per graph; graphs start at different copies so replays never re-read a copy
    K = args.steps
    n_graphs = 1 if K >= n_copies else math.ceil(n_copies / K)

    def graph_fn(j):
        def launch(s):
            for i in range(K):
                assert lib.fa_batch_launch(plans[(j * K + i) % n_copies], s) == cvattn.OK
        return launch

    ms, per_replay = time_graphs(torch, [graph_fn(j) for j in range(n_graphs)], K, args.warmup)
    bytes_step = per_layer * L
    gbs = bytes_step / (ms * 1e-3) / 1e9
    log(f"decode 24x4096 batched: {ms * 1e3:.2f} us/step (median of {TIMED_REPEATS} replays of {K}), {gbs:.0f} GB/s")

    ms_seq = ms_dyn = None
    if not args.no_cadence:
        ms_seq, ms_dyn = decode_cadence(lib, cvattn, torch, dev, problem, n_copies, keep)

    extra = {}

    if not args.no_dit:
        extra["dit_attn"] = bench_dit(lib, cvattn, torch, dev)
        log(f"dit T=1500: {extra['dit_attn']['ms_per_layer_call'] * 1e3:.1f} us/call, "
            f"{extra['dit_attn']['tflops']:.1f} TFLOP/s")
    if not args.no_extra and not args.no_dit:
        extra["dit_attn_f32_views"] = bench_dit_f32_views(lib, cvattn, torch, dev)
        log(f"dit T=1500 fp32 views: {extra['dit_attn_f32_views']['us_per_layer_call']:.1f} us/call, "
            f"{extra['dit_attn_f32_views']['tflops']:.1f} TFLOP/s, "
            f"{extra['dit_attn_f32_views']['ms_per_utterance_eager_220_calls']:.2f} ms/utterance eager")
        extra["dit_attn_chunk_mask"] = bench_dit_masked(lib, cvattn, torch, dev)
        log(f"dit T=1500 chunk mask: {extra['dit_attn_chunk_mask']['us_per_layer_call']:.1f} us/call")
    if not args.no_extra:
        extra["decode_single_calls"] = bench_single_call_decode(lib, cvattn, torch, dev, kbuf, vbuf, q, out,
                                                                n_copies, kt, vt)
        log(f"decode single calls: {extra['decode_single_calls']['us_per_token']:.1f} us/token")
        extra["prefill_attn"] = bench_prefill(lib, cvattn, torch, dev)
        log(f"prefill 1024 causal: {extra['prefill_attn']['us_per_layer_call']:.1f} us/layer, "
            f"{extra['prefill_attn']['tflops']:.1f} TFLOP/s; 4x256 chunks "
            f"{extra['prefill_attn']['reference_cadence_4x256']['us_per_layer']:.1f} us/layer")
        extra["dit_stream_attn"] = bench_dit_stream(lib, cvattn, torch, dev)
        log(f"dit stream 50x1050: {extra['dit_stream_attn']['us_per_layer_call']:.1f} us/call, "
            f"{extra['dit_stream_attn']['gbs']:.0f} GB/s")
        extra["serving_decode_attn"] = bench_serving(lib, cvattn, torch, dev)
        log(f"serving 16x24 ragged q8_0: {extra['serving_decode_attn']['us_per_step']:.1f} us/step, "
            f"{extra['serving_decode_attn']['gbs']:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(kbuf, vbuf, q)
        log(f"cpu baseline: {cpu['value']:.3f} GB/s ({cpu['cores']} threads)")

    traffic = read_traffic()
    res = {
        "metric": "LLM decode-attn GB/s + tok/s (q8_0 KV, 4k ctx); DiT attn TFLOP/s",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "repeats": TIMED_REPEATS,
        "ms_per_step": ms,
        "ms_per_replay": per_replay,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA + f32",
        "data": "synthetic: seeded N(0,1) K/V quantized on device with ggml's reference quantizers, N(0,1) Q",
        "device": device_info(torch),
        "config": {
            "workload": "decode attention, 24 layers x 1 token, batch 1, 14/2 heads, head_dim 64, "
                        "kv_len 4096, K q8_0 / V q4_0 (the 24 layers run as one prepared batch)",
            "kv_copies_cycled": n_copies,
            "bytes_per_step": bytes_step,
        },
        # the decode rate a token loop reaches: layer l+1 needs layer l's output, so one launch per layer
        "tok_per_s": 1000.0 / ms_seq if ms_seq else None,
        "us_per_token": ms_seq * 1e3 if ms_seq else None,
        "tok_per_s_basis": "24 dependent one-layer launches per token (prepared plans, graph-replayed)",
        "decode_graph_device_n_kv": {"us_per_token": ms_dyn * 1e3 if ms_dyn else None,
                                     "tok_per_s": 1000.0 / ms_dyn if ms_dyn else None,
                                     "workload": "per token one graph replay: cvattn_shift_n_kv + 24 layer launches "
                                                 "of plans prepared with a device n_kv (4033.. tokens, capacity 4096)"},
        "layer_batched_synthetic": {"tok_per_s": 1000.0 / ms,
                                    "note": "the 24 layers of one token in one launch (the value's step); "
                                            "not reachable by a decoder, whose layers depend on each other"},
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": gbs / HBM_PEAK_GBS,
            "traffic": traffic,
            "traffic_source": f"{TRAFFIC_PROFILE} (rocprofv3 FETCH_SIZE/WRITE_SIZE passes, copy-calibrated)",
        },
        "cpu_baseline": cpu,
    }
    res.update(extra)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
