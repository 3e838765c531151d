"""Host logic of the DiT streaming cache (cvattn_dit_cache_*, cvattn_dit_schedule), CPU only:
the slot layout and views against the tensors cosyvoice_kv_cache builds
(src/cosyvoice-kv-cache.cpp:45-146,309-355, src/cosyvoice-loader.cpp:1011-1029), and the per-step
plan of token2wav (src/cosyvoice-token2wav.cpp:101-167,352-412) through the properties a
streaming run depends on.  No device memory is touched: the cache records layout only."""
import ctypes
import itertools

import pytest

import cvattn
from cvattn import F16, F32, Q4_0, Q8_0

FAKE_DEV = 0x7f0000000000  # 256-byte aligned, never dereferenced here


def params(**kw):
    p = cvattn.DitCacheParams()
    d = dict(layers=22, heads=16, head_dim=64, max_seq=1100, batch=2, k_type=Q8_0, v_type=Q4_0, n_slots=5,
             n_host_slots=2, flash_attn=1)
    d.update(kw)
    for k, v in d.items():
        setattr(p, k, v)
    return p


def test_sizes_follow_the_reference_tensors(eng):
    p = params()
    dev, host = eng.dit_cache_bytes(p)
    k = 1024 // 32 * 34 * 1100 * 2     # q8_0 [1024, max_seq, 2]
    v = 1024 // 32 * 18 * 1100 * 2     # q4_0
    al = lambda x: (x + 255) // 256 * 256
    assert dev == 5 * 22 * (al(k) + al(v))
    assert host == 2 * 22 * (k + v)
    pt = params(flash_attn=0, v_type=F16)                       # transposed V [max_seq, 1024, 2] f16
    dev_t, _ = eng.dit_cache_bytes(pt)
    assert dev_t == 5 * 22 * (al(k) + al(2 * 1100 * 1024 * 2))
    assert eng.dit_cache_bytes(params(flash_attn=0, v_type=Q8_0)) == (0, 0)   # transposed V must be f32/f16


def make(eng, p):
    dev, host = eng.dit_cache_bytes(p)
    rc, c = eng.dit_cache_create(p, FAKE_DEV, dev, FAKE_DEV if host else 0, host)
    assert rc == cvattn.OK
    return c


def test_views_and_slots(eng):
    p = params()
    c = make(eng, p)
    L = eng.L
    try:
        rc, (kc, vc, kv, vv) = eng.dit_cache_layer(c, 3, 1050)
        assert rc == cvattn.OK
        k_al = (1024 // 32 * 34 * 1100 * 2 + 255) // 256 * 256
        v_al = (1024 // 32 * 18 * 1100 * 2 + 255) // 256 * 256
        assert kc.data == FAKE_DEV + 3 * (k_al + v_al) and vc.data == kc.data + k_al
        # set_rows target [1024, max_seq, 2] and the permuted view [64, n_kv, 16, 2] (kv-cache.cpp:316-318)
        assert list(kc.ne) == [1024, 1100, 2, 1] and list(kc.nb)[:3] == [34, 1088, 1088 * 1100]
        assert list(kv.ne) == [64, 1050, 16, 2] and list(kv.nb) == [34, 1088, 68, 1088 * 1100]
        assert list(vv.ne) == [64, 1050, 16, 2] and list(vv.nb) == [18, 576, 36, 576 * 1100]
        # slots: slide walks forward (flash attention), bind picks any, both bounded
        assert L.cvattn_dit_cache_slot(c) == 0
        assert L.cvattn_dit_cache_slide(c) == cvattn.OK and L.cvattn_dit_cache_slot(c) == 1
        rc, (kc1, _, _, _) = eng.dit_cache_layer(c, 3, 10)
        assert kc1.data == kc.data + 22 * (k_al + v_al)
        assert L.cvattn_dit_cache_bind_slot(c, 4) == cvattn.OK
        assert L.cvattn_dit_cache_slide(c) == cvattn.ERR_BAD_ARGS       # no slot after the last
        assert L.cvattn_dit_cache_bind_slot(c, 5) == cvattn.ERR_BAD_ARGS
        assert L.cvattn_dit_cache_set_len(c, 1100) == cvattn.OK and L.cvattn_dit_cache_len(c) == 1100
        assert L.cvattn_dit_cache_set_len(c, 1101) == cvattn.ERR_BAD_ARGS
        assert eng.dit_cache_layer(c, 22, 5)[0] == cvattn.ERR_BAD_ARGS
        assert eng.dit_cache_layer(c, 0, 1101)[0] == cvattn.ERR_BAD_ARGS
        assert L.cvattn_dit_cache_offload(c, 2, 10, None) == cvattn.ERR_BAD_ARGS  # host slots 0..1
    finally:
        L.cvattn_dit_cache_destroy(c)


def test_transposed_v_views(eng):
    p = params(flash_attn=0, v_type=F16)
    c = make(eng, p)
    try:
        rc, (kc, vc, kv, vv) = eng.dit_cache_layer(c, 0, 300)
        # V cache [max_seq, 1024, 2] and the view [n_kv, 64, 16, 2] (kv-cache.cpp:104-108,345)
        assert list(vc.ne) == [1100, 1024, 2, 1] and list(vc.nb)[:2] == [2, 2200]
        assert list(vv.ne) == [300, 64, 16, 2] and list(vv.nb) == [2, 2200, 2200 * 64, 2200 * 1024]
        assert eng.L.cvattn_dit_cache_slide(c) == cvattn.ERR_UNSUPPORTED  # the reference aborts here
    finally:
        eng.L.cvattn_dit_cache_destroy(c)


def test_create_rejects_small_buffers(eng):
    p = params()
    dev, host = eng.dit_cache_bytes(p)
    assert eng.dit_cache_create(p, FAKE_DEV, dev - 1, FAKE_DEV, host)[0] == cvattn.ERR_WORKSPACE_TOO_SMALL
    assert eng.dit_cache_create(p, FAKE_DEV, dev, 0, 0)[0] == cvattn.ERR_WORKSPACE_TOO_SMALL
    assert eng.dit_cache_create(p, FAKE_DEV + 16, dev, FAKE_DEV, host)[0] == cvattn.ERR_BAD_ARGS


# ------------------------------------------------------------------------------------------
# the step plan
# ------------------------------------------------------------------------------------------
def sched(eng, n, fix, off, cut, offset, streaming=True, slidable=True):
    rc, steps = eng.dit_schedule(n, fix, off, cut, offset, streaming, slidable)
    assert rc == cvattn.OK
    return steps


def test_one_shot_plan(eng):
    steps = sched(eng, 10, 0, 0, 37, 0, streaming=False)
    assert [s.rebuild for s in steps] == [1, 1] + [0] * 7 + [1]
    assert [s.cut_len for s in steps] == [0] * 9 + [37]
    assert all(s.cache_kv == 0 and s.slot == -1 and s.host_slot == -1 for s in steps)


CASES = [(10, f, o) for f in range(0, 11) for o in range(0, 11 - f)]


@pytest.mark.parametrize("n,fix,off", CASES)
def test_streaming_plan_properties(eng, n, fix, off):
    n_slots = fix + (1 if off else 0)
    first = n - fix - off
    per_chunk = []
    for offset, cut, slidable in itertools.product((0, 250), (0, 37), (1, 0)):
        steps = sched(eng, n, fix, off, cut, offset, slidable=slidable)
        cached = [i for i, s in enumerate(steps) if s.cache_kv]
        assert cached == list(range(first, n))
        offl = [i for i, s in enumerate(steps) if s.offload]
        assert offl == list(range(first, first + off))
        for i, s in enumerate(steps):
            assert s.load == (s.offload and offset != 0)
            assert s.mask == (i < first and offset != 0)
            assert s.slice == (offset != 0 and i == first)
            if s.cache_kv:
                assert 0 <= s.slot < max(n_slots, 1)
            else:
                assert s.slot == -1
            if s.offload:
                assert s.slot == 0 and s.host_slot == i - first   # staging slot, host slot per step
            else:
                assert s.host_slot == -1
            if i > 0 and s.cache_kv and not slidable:
                assert s.rebuild
        # every fixed step has a device slot of its own, apart from the staging slot
        fixed_slots = [steps[i].slot for i in range(first + off, n)]
        assert len(set(fixed_slots)) == len(fixed_slots)
        assert not off or 0 not in fixed_slots
        # the last step takes the cut on a first chunk; on later chunks only when it is also the
        # step before the (absent) cached steps, which takes the offset
        want_last = cut if offset == 0 else (offset if first == n else 0)
        assert steps[n - 1].cut_len == want_last
        if offset != 0 and first >= 1:
            assert steps[first - 1].cut_len == offset
        per_chunk.append([(s.slot, s.host_slot if s.load or s.offload else -1) for s in steps])
    # the slots a step uses do not depend on the chunk (first or later, cut or not) nor on whether
    # the schedule slides or rebinds: what chunk k wrote at step i, chunk k+1 reads at step i
    assert all(pc == per_chunk[0] for pc in per_chunk)


def test_schedule_rejects(eng):
    assert eng.dit_schedule(10, 8, 3, 0, 0, True, True)[0] == cvattn.ERR_BAD_ARGS
    assert eng.dit_schedule(1, 0, 0, 0, 0, True, True)[0] == cvattn.ERR_BAD_ARGS


def test_step_inputs_argument_checks(eng):
    m = cvattn.contiguous(0x1000, F16, [100, 100, 1, 1])
    assert eng.chunk_mask(m, [50, 20]) == cvattn.ERR_BAD_ARGS          # unsorted bounds
    assert eng.chunk_mask(m, list(range(300))) == cvattn.ERR_BAD_ARGS  # more than the kernel takes
    m32 = cvattn.contiguous(0x1000, F32, [100, 100, 1, 1])
    assert eng.chunk_mask(m32, [50]) == cvattn.ERR_BAD_ARGS
    p = cvattn.contiguous(0x1000, F16, [100, 2, 1, 1])
    assert eng.fill_positions(p, 0) == cvattn.ERR_BAD_ARGS
    assert eng.v_idxs(0x1000, 0x2000, 10, 0, 1024, 100) == cvattn.ERR_BAD_ARGS
    assert eng.v_idxs(0x1000, 0x2000, 4, 2, 1024, 2 ** 21) == cvattn.ERR_UNSUPPORTED   # past int32
