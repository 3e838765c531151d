"""CPU-side checks of the C ABI: the library loads, exports every entry point include/cvattn.h
declares, and its host-side validation (the supports_op probe, workspace sizing, error codes)
behaves like ggml's shape rules.  No kernel is launched here."""
import ctypes
import os
import re

import pytest

import cvattn
from cvattn import F16, F32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cvattn.h")
FAKE = 0x1000  # never dereferenced: validation-only calls


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"CVATTN_API\s+[\w\s\*]+?\b(cvattn_\w+)\s*\(", text)))


def test_header_symbols_exported(eng):
    syms = header_symbols()
    assert len(syms) >= 12
    for s in syms:
        assert hasattr(eng.L, s), s
    assert set(syms) == set(cvattn.EXPORTED)


def test_type_table(eng):
    for t, (blk, size) in {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_0: (32, 18), Q4_1: (32, 20),
                           Q5_0: (32, 22), Q5_1: (32, 24)}.items():
        assert eng.block_size(t) == blk and eng.type_size(t) == size
    assert eng.block_size(99) == 0 and eng.type_size(99) == 0


def llm(n_q=1, n_kv=512, kt=Q8_0, vt=Q4_0, H=14, Hkv=2, max_seq=4096):
    q = cvattn.llm_q_view(FAKE, 64, H, n_q)
    k = cvattn.llm_kv_view(FAKE, kt, 64, Hkv, n_kv, max_seq)
    v = cvattn.llm_kv_view(FAKE, vt, 64, Hkv, n_kv, max_seq)
    dst = cvattn.out_view(FAKE, 64, H, n_q)
    return q, k, v, dst


@pytest.mark.parametrize("kt", [F32, F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1])
@pytest.mark.parametrize("vt", [F32, F16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1])
def test_supports_every_kv_type_pair(eng, kt, vt):
    """Every type the loader's fallback chain can pick (src/cosyvoice-loader.cpp:498-510)."""
    q, k, v, _ = llm(kt=kt, vt=vt)
    assert eng.supports_flash_attn_ext(q, k, v, None)


def test_supports_rejects(eng):
    q, k, v, _ = llm()
    bad = cvattn.llm_kv_view(FAKE, Q8_0, 128, 1, 512, 4096)  # head size 128
    assert not eng.supports_flash_attn_ext(q, bad, v, None)
    k26 = cvattn.tensor(FAKE, 26, list(k.ne), list(k.nb))  # i32 keys
    assert not eng.supports_flash_attn_ext(q, k26, v, None)
    q3 = cvattn.llm_q_view(FAKE, 64, 15, 1)  # 15 heads over 2 kv heads
    assert not eng.supports_flash_attn_ext(q3, k, v, None)
    m = cvattn.mask_view(FAKE, 100, 1)  # mask shorter than n_kv
    assert not eng.supports_flash_attn_ext(q, k, v, m)
    m = cvattn.mask_view(FAKE, 512, 1)
    assert eng.supports_flash_attn_ext(q, k, v, m)
    mf32 = cvattn.tensor(FAKE, F32, [512, 1, 1, 1], [4, 2048, 2048, 2048])
    assert not eng.supports_flash_attn_ext(q, k, v, mf32)


def test_probe_shapes_of_loader(eng):
    """cosyvoice_check_kv_cache_types probes q [64,1,14,1] against a 1-row cache (loader.cpp:543-567)."""
    for kt in (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, F16, F32):
        q = cvattn.contiguous(FAKE, F32, [64, 1, 14, 1])
        k = cvattn.llm_kv_view(FAKE, kt, 64, 2, 1, 1)
        v = cvattn.llm_kv_view(FAKE, kt, 64, 2, 1, 1)
        assert eng.supports_flash_attn_ext(q, k, v, None)


def test_workspace_and_errors(eng):
    q, k, v, dst = llm(n_kv=4096)
    ws = eng.flash_attn_ext_workspace(q, k, v, None)
    assert ws > 0  # long decode is split over the chip
    assert eng.flash_attn_ext(q, k, v, None, dst, 0.125, 0, 0) == cvattn.ERR_WORKSPACE_TOO_SMALL
    assert eng.flash_attn_ext(q, k, v, None, dst, 0.125, FAKE, ws, max_bias=1.0) == cvattn.ERR_UNSUPPORTED
    assert eng.flash_attn_ext(q, k, v, None, dst, 0.125, FAKE, ws, softcap=30.0) == cvattn.ERR_UNSUPPORTED
    assert eng.flash_attn_ext(q, k, v, None, dst, float("nan"), FAKE, ws) == cvattn.ERR_BAD_ARGS
    bad_dst = cvattn.out_view(FAKE, 64, 14, 2)
    assert eng.flash_attn_ext(q, k, v, None, bad_dst, 0.125, FAKE, ws) == cvattn.ERR_BAD_ARGS
    assert eng.status_string(cvattn.ERR_WORKSPACE_TOO_SMALL) == "workspace too small"
    # tiny problems need no workspace
    q, k, v, dst = llm(n_kv=64)
    assert eng.flash_attn_ext_workspace(q, k, v, None) == 0


def test_workspace_holds_fp16_copies_of_fp32_kv(eng):
    """fp32 K/V read by many row groups (the DiT call without cache) are copied to fp16 in the
    workspace: 64 halfs per K/V row, token rows of the transposed V padded to 8 halfs."""
    T, H, B = 1500, 16, 2

    def dit(t, n=T):
        es = 4 if t == F32 else 2
        return cvattn.tensor(FAKE, t, [64, n, H, B], [es, es * 64 * H, es * 64, es * 64 * H * n])

    rows = T * H * B
    assert eng.flash_attn_ext_workspace(dit(F16), dit(F16), dit(F16), None) == 0
    assert eng.flash_attn_ext_workspace(dit(F32), dit(F32), dit(F16), None) == rows * 64 * 2
    both = eng.flash_attn_ext_workspace(dit(F32), dit(F32), dit(F32), None)
    assert both == 2 * rows * 64 * 2  # K copy (256-byte aligned size) then V copy
    assert eng.flash_attn_ext_workspace(dit(F32), dit(F16), dit(F32), None) == rows * 64 * 2
    # a short query run (a single row group) stages fp32 directly
    assert eng.flash_attn_ext_workspace(dit(F32, 50), dit(F32, 50), dit(F32, 50), None) == 0
    # transposed V of the non-flash form: [T, 64, H, B] with T = 301 -> rows of 304 halfs
    n = 301
    vt = cvattn.tensor(FAKE, F32, [n, 64, H, B], [4, 4 * n, 4 * n * 64, 4 * n * 64 * H])
    k = dit(F32, n)
    assert eng.attn_nonfa_workspace(dit(F32, n), k, vt, None) == n * H * B * 64 * 2 + 64 * H * B * 304 * 2


def test_batch_validation(eng):
    probs = []
    for n_kv in (256, 1000, 8192):
        q, k, v, dst = llm(n_kv=n_kv, kt=Q8_0, vt=Q8_0, max_seq=8192)
        p = cvattn.FaProblem()
        p.q, p.k, p.v, p.dst = q, k, v, dst
        probs.append(p)
    ws = eng.fa_batch_workspace(probs)
    assert ws > 0
    rc, _ = eng.fa_batch_prepare(probs, 0.125, 0, 0)
    assert rc == cvattn.ERR_WORKSPACE_TOO_SMALL
    q, k, v, dst = llm(n_kv=10, kt=Q8_0, vt=Q4_0)  # a different V type cannot join the batch
    p = cvattn.FaProblem()
    p.q, p.k, p.v, p.dst = q, k, v, dst
    assert eng.fa_batch_workspace(probs + [p]) == 0


def test_set_rows_validation(eng):
    dst = cvattn.contiguous(FAKE, Q8_0, [128, 4096, 1, 1])
    src = cvattn.contiguous(FAKE, F32, [128, 3, 1, 1])
    idx = cvattn.contiguous(FAKE, 26, [3, 1, 1, 1])
    assert eng.supports_set_rows(dst, src, idx)
    src_bad = cvattn.contiguous(FAKE, F32, [96, 3, 1, 1])
    assert not eng.supports_set_rows(dst, src_bad, idx)
    dst40 = cvattn.contiguous(FAKE, F16, [40, 16, 1, 1])
    src40 = cvattn.contiguous(FAKE, F32, [40, 3, 1, 1])
    assert eng.supports_set_rows(dst40, src40, idx)  # f16 rows need no block alignment
    dstq40 = cvattn.contiguous(FAKE, F16, [40, 16, 1, 1])
    dstq40.type = Q4_0
    assert not eng.supports_set_rows(dstq40, src40, idx)


def test_library_is_loaded_from_tree(eng):
    assert os.path.dirname(eng.path) == os.path.join(ROOT, "cosyvoice.cpp_amd")
    assert isinstance(eng.L, ctypes.CDLL)


def test_rope_argument_checks(eng):
    """cvattn_rope / cvattn_rope_set_rows reject what ggml_rope_ext would not compute the same way;
    every case returns before any kernel launch."""
    x = cvattn.contiguous(FAKE, F32, [64, 14, 5, 1])
    pos = cvattn.contiguous(FAKE, cvattn.I32, [5, 1, 1, 1])
    assert eng.rope(x, x, pos, 64, 1, 1e6) == cvattn.ERR_UNSUPPORTED        # GLM/vision modes
    assert eng.rope(x, x, pos, 63, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_BAD_ARGS  # odd dims
    assert eng.rope(x, x, pos, 66, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_BAD_ARGS  # dims > ne0
    assert eng.rope(x, x, pos, 64, cvattn.ROPE_NEOX, 0.0) == cvattn.ERR_BAD_ARGS  # base
    pos4 = cvattn.contiguous(FAKE, cvattn.I32, [4, 1, 1, 1])
    assert eng.rope(x, x, pos4, 64, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_BAD_ARGS  # one per i2
    h16 = cvattn.contiguous(FAKE, F16, [64, 14, 5, 1])
    assert eng.rope(h16, x, pos, 64, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_UNSUPPORTED

    cache = cvattn.contiguous(FAKE, Q8_0, [128, 4096, 1, 1])
    src = cvattn.contiguous(FAKE, F32, [128, 3, 1, 1])
    idx = cvattn.contiguous(FAKE, cvattn.I32, [3, 1, 1, 1])
    rs = eng.rope_set_rows
    assert rs(cache, src, idx, idx, 96, 64, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_BAD_ARGS   # 128 % 96
    assert rs(cache, src, idx, idx, 64, 80, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_BAD_ARGS   # dims > head
    assert rs(cache, src, idx, idx, 64, 64, 8, 1e6) == cvattn.ERR_UNSUPPORTED
    assert rs(cache, src, idx, pos4, 64, 64, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_BAD_ARGS  # 4 != 3 rows
    posf = cvattn.contiguous(FAKE, F32, [3, 1, 1, 1])
    assert rs(cache, src, idx, posf, 64, 64, cvattn.ROPE_NEOX, 1e6) == cvattn.ERR_UNSUPPORTED


def test_nonfa_argument_checks(eng):
    """The transposed-V entry: the V cache must be f32/f16 with tokens contiguous and Dv = 64."""
    n = 2000    # long enough that the decode rows are split over tokens
    q, k, _, dst = llm(n_kv=n, kt=Q8_0)
    max_seq = 4096
    vt = cvattn.tensor(FAKE, F16, [n, 64, 2, 1], [2, 2 * max_seq, 2 * max_seq * 64, 2 * max_seq * 128])
    assert eng.supports_attn_nonfa(q, k, vt, None)
    assert eng.attn_nonfa_workspace(q, k, vt, None) > 0
    vq = cvattn.tensor(FAKE, Q8_0, [n, 64, 2, 1], [34, 34 * max_seq, 34 * max_seq * 64, 34 * max_seq * 128])
    assert not eng.supports_attn_nonfa(q, k, vq, None)
    assert eng.attn_nonfa(q, k, vq, None, dst, 0.125) == cvattn.ERR_UNSUPPORTED
    vbad = cvattn.tensor(FAKE, F16, [n - 1, 64, 2, 1], list(vt.nb))            # n_kv mismatch
    assert eng.attn_nonfa(q, k, vbad, None, dst, 0.125) == cvattn.ERR_BAD_ARGS
    v32 = cvattn.tensor(FAKE, F16, [n, 32, 2, 1], list(vt.nb))                 # Dv 32
    assert eng.attn_nonfa(q, k, v32, None, dst, 0.125) == cvattn.ERR_UNSUPPORTED
    vstr = cvattn.tensor(FAKE, F16, [n, 64, 2, 1], [4] + list(vt.nb)[1:])      # tokens not contiguous
    assert eng.attn_nonfa(q, k, vstr, None, dst, 0.125) == cvattn.ERR_BAD_ARGS
    assert eng.attn_nonfa(q, k, vt, None, dst, 0.125, 0, 0) == cvattn.ERR_WORKSPACE_TOO_SMALL


def test_views_past_32_bit_offsets_are_refused(eng):
    """Both attention kernels address one head's K/V rows with 32-bit byte offsets (token * nb1):
    a view whose head spans 2^31 bytes or more is reported unsupported (so the host keeps its own
    path) instead of being read through a clamped buffer range."""
    n_kv = 600000
    q = cvattn.dit_view(FAKE, 2000, 1)
    big = cvattn.dit_view(FAKE, n_kv, 1)                        # fp32 rows: 600000 * 4096 B > 2^31
    small = cvattn.dit_view(FAKE, n_kv, 1, ttype=cvattn.F16)    # fp16 rows: 600000 * 2048 B < 2^31
    for k, v in ((big, small), (small, big), (big, big)):
        assert not eng.supports_flash_attn_ext(q, k, v, None)
        dst = cvattn.out_view(FAKE, 64, 16, 2000, 1)
        assert eng.flash_attn_ext(q, k, v, None, dst, 0.125, FAKE, 1 << 40) == cvattn.ERR_UNSUPPORTED
    assert eng.supports_flash_attn_ext(q, small, small, None)
    # one decode row over the same long view (the decode kernel has the same bound)
    q1 = cvattn.dit_view(FAKE, 1, 1)
    assert not eng.supports_flash_attn_ext(q1, big, small, None)
    # a prepared batch holding such a problem is refused as well
    p = cvattn.FaProblem()
    p.q, p.k, p.v, p.dst = q1, big, small, cvattn.out_view(FAKE, 64, 16, 1, 1)
    assert eng.fa_batch_workspace([p]) == 0


def test_fp32_views_with_no_keys_need_no_copy(eng):
    """n_kv = 0 with fp32 K/V and many query row groups: nothing to copy to fp16, so no
    workspace (the call itself writes zeros; see the GPU test of the same shape)."""
    q = cvattn.dit_view(FAKE, 300, 2)
    k = cvattn.dit_view(FAKE, 0, 2)
    assert eng.supports_flash_attn_ext(q, k, k, None)
    assert eng.flash_attn_ext_workspace(q, k, k, None) == 0


def test_dynamic_plan_validation(eng):
    q, k, v, dst = llm(n_kv=4096)
    p = cvattn.FaProblem()
    p.q, p.k, p.v, p.dst = q, k, v, dst
    ws = eng.fa_batch_workspace([p])
    assert ws > 0
    rc, _ = eng.fa_batch_prepare_dynamic([p], 0.125, 0, 0, FAKE, ws)            # no device length
    assert rc == cvattn.ERR_BAD_ARGS
    rc, _ = eng.fa_batch_prepare_dynamic([p], 0.125, FAKE, 2, FAKE, ws)         # stride 0 or 1 only
    assert rc == cvattn.ERR_BAD_ARGS
    rc, _ = eng.fa_batch_prepare_dynamic([p], 0.125, FAKE + 2, 0, FAKE, ws)     # int32 alignment
    assert rc == cvattn.ERR_BAD_ARGS
    rc, _ = eng.fa_batch_prepare_dynamic([p], 0.125, FAKE, 0, FAKE, ws - 1)
    assert rc == cvattn.ERR_WORKSPACE_TOO_SMALL
    assert eng.shift_n_kv(0, 1, 1) == cvattn.ERR_BAD_ARGS
    assert eng.shift_n_kv(FAKE, -1, 1) == cvattn.ERR_BAD_ARGS
    assert eng.shift_n_kv(0, 0, 1) == cvattn.OK       # nothing to do, no launch


def test_noalloc_size_limit_checked_before_any_launch(eng):
    """fp32 DiT views of 5000 frames need more than the fixed scratch array for their fp16 K/V
    copies: refused with WORKSPACE_TOO_SMALL before anything touches the device."""
    T, B = 5000, 2
    qv = cvattn.dit_view(FAKE, T, B)
    assert eng.flash_attn_ext_workspace(qv, qv, qv, None) > cvattn.NOALLOC_SCRATCH_BYTES
    dst = cvattn.out_view(FAKE, 64, 16, T, B)
    assert eng.flash_attn_ext_noalloc(qv, qv, qv, None, dst, 0.125) == cvattn.ERR_WORKSPACE_TOO_SMALL
    assert eng.flash_attn_ext_noalloc(qv, qv, qv, None, dst, 0.125, max_bias=1.0) == cvattn.ERR_UNSUPPORTED
