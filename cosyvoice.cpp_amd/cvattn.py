"""ctypes binding of libcvattn.so (include/cvattn.h) plus the tensor views cosyvoice.cpp builds
around its attention nodes, so callers can feed the engine exactly the stride patterns of the
reference's graphs.

The views restate:
  * LLM KV cache  src/cosyvoice-kv-cache.cpp:104-119 (cache [H_kv*D, max_seq, batch] per layer)
                  and :316-324 (view_4d + permute(0,2,1,3) -> [D, n_kv, H_kv, B]);
  * LLM query     src/cosyvoice-llm.cpp:40-60 (rope output [D, H, n_q] permuted -> [D, n_q, H, 1]);
  * DiT q/k/v     src/cosyvoice-graph.cpp:357-371 ([1024, T, B] rows split into 16 heads of 64,
                  permuted -> [64, T, 16, B]);
  * output        ggml_flash_attn_ext's dst, f32 contiguous [Dv, H, n_q, B].

The library is required: importing this module raises if libcvattn.so is missing, and nothing
here falls back to another implementation.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcvattn.so")

# ggml_type codes
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, I32 = 0, 1, 2, 3, 6, 7, 8, 26
TYPE_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1", Q8_0: "q8_0"}
TYPE_BY_NAME = {v: k for k, v in TYPE_NAMES.items()}
BLOCK = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32}
TYPE_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34}

OK, ERR_UNSUPPORTED, ERR_BAD_ARGS, ERR_WORKSPACE_TOO_SMALL, ERR_HIP = 0, 1, 2, 3, 4
NOALLOC_SCRATCH_BYTES = 32 << 20  # CVATTN_NOALLOC_SCRATCH_BYTES
ROPE_NORMAL, ROPE_NEOX = 0, 2  # CVATTN_ROPE_* (ggml rope modes)
PREC_DEFAULT, PREC_F32 = 0, 10


def row_bytes(t: int, n: int) -> int:
    """Bytes of n elements of type t (n a multiple of the block size)."""
    assert n % BLOCK[t] == 0
    return n // BLOCK[t] * TYPE_BYTES[t]


class Tensor(ctypes.Structure):
    """cvattn_tensor: ggml_tensor's data/type/ne/nb."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]

    def __repr__(self) -> str:  # pragma: no cover - debugging aid
        return f"Tensor(type={self.type}, ne={list(self.ne)}, nb={list(self.nb)})"


class FaProblem(ctypes.Structure):
    _fields_ = [("q", Tensor), ("k", Tensor), ("v", Tensor), ("mask", Tensor), ("dst", Tensor)]


class DitCacheParams(ctypes.Structure):
    """cvattn_dit_cache_params"""
    _fields_ = [(n, ctypes.c_int32) for n in ("layers", "heads", "head_dim", "max_seq", "batch", "k_type", "v_type",
                                              "n_slots", "n_host_slots", "flash_attn")]


class DitStep(ctypes.Structure):
    """cvattn_dit_step"""
    _fields_ = [(n, ctypes.c_int32) for n in ("rebuild", "cache_kv", "load", "offload", "slide", "slice", "mask",
                                              "slot", "host_slot")] + [("cut_len", ctypes.c_int64)]


class FaPlan(ctypes.Structure):
    _fields_ = [("opaque", ctypes.c_uint64 * 64)]


def tensor(data: int, ttype: int, ne, nb) -> Tensor:
    t = Tensor()
    t.data = ctypes.c_void_p(int(data)) if data else None
    t.type = ttype
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


def contiguous(data: int, ttype: int, ne) -> Tensor:
    """ggml_new_tensor layout: nb0 = type size, nb1 = row bytes, then products."""
    ne = list(ne) + [1] * (4 - len(ne))
    nb = [TYPE_BYTES[ttype] if ttype in TYPE_BYTES else 4]
    nb.append(row_bytes(ttype, ne[0]) if ttype in TYPE_BYTES else 4 * ne[0])
    nb.append(nb[1] * ne[1])
    nb.append(nb[2] * ne[2])
    return tensor(data, ttype, ne, nb)


# ---------------------------------------------------------------------------------------------
# Views of the reference graphs
# ---------------------------------------------------------------------------------------------
def llm_cache_row_bytes(ttype: int, head_dim: int, n_kv_heads: int) -> int:
    return row_bytes(ttype, head_dim * n_kv_heads)


def llm_kv_view(data: int, ttype: int, head_dim: int, n_kv_heads: int, n_kv: int, max_seq: int,
                batch: int = 1) -> Tensor:
    """K or V cache view read by attention (src/cosyvoice-kv-cache.cpp:316-318, 322-324)."""
    row = llm_cache_row_bytes(ttype, head_dim, n_kv_heads)
    return tensor(data, ttype, [head_dim, n_kv, n_kv_heads, batch],
                  [TYPE_BYTES[ttype], row, row // n_kv_heads, row * max_seq])


def llm_q_view(data: int, head_dim: int, n_heads: int, n_q: int, ttype: int = F32) -> Tensor:
    """Query after RoPE [D, H, n_q] permuted (0,2,1,3) (src/cosyvoice-llm.cpp:56-60)."""
    es = TYPE_BYTES[ttype]
    return tensor(data, ttype, [head_dim, n_q, n_heads, 1],
                  [es, es * head_dim * n_heads, es * head_dim, es * head_dim * n_heads * n_q])


def dit_view(data: int, seq: int, batch: int, heads: int = 16, head_dim: int = 64, ttype: int = F32,
             row_elems: int | None = None) -> Tensor:
    """DiT q/k/v: [heads*head_dim, seq, batch] split into heads and permuted (0,2,1,3)
    (src/cosyvoice-graph.cpp:357-371) -> [head_dim, seq, heads, batch]."""
    es = TYPE_BYTES[ttype]
    row = (row_elems or heads * head_dim) * es
    return tensor(data, ttype, [head_dim, seq, heads, batch], [es, row, head_dim * es, row * seq])


def out_view(data: int, head_dim: int, n_heads: int, n_q: int, batch: int = 1) -> Tensor:
    return contiguous(data, F32, [head_dim, n_heads, n_q, batch])


def mask_view(data: int, n_kv: int, n_q: int, row_elems: int | None = None) -> Tensor:
    """f16 mask [n_kv, n_q] (src/cosyvoice-llm.cpp:101-108: nb1 = n_kv*2)."""
    row = (row_elems or n_kv) * 2
    return tensor(data, F16, [n_kv, n_q, 1, 1], [2, row, row * n_q, row * n_q])


# ---------------------------------------------------------------------------------------------
# Library
# ---------------------------------------------------------------------------------------------
class Lib:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise ImportError(f"libcvattn.so not built at {path}; run __graft_entry__.build()")
        self.path = path
        L = ctypes.CDLL(path)
        P = ctypes.POINTER(Tensor)
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        L.cvattn_supports_flash_attn_ext.argtypes = [P, P, P, P]
        L.cvattn_supports_flash_attn_ext.restype = ctypes.c_int
        L.cvattn_flash_attn_ext_workspace.argtypes = [P, P, P, P]
        L.cvattn_flash_attn_ext_workspace.restype = sz
        L.cvattn_flash_attn_ext.argtypes = [P, P, P, P, P, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                            ctypes.c_int, vp, sz, vp]
        L.cvattn_flash_attn_ext.restype = ctypes.c_int
        L.cvattn_flash_attn_ext_noalloc.argtypes = [P, P, P, P, P, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                                    ctypes.c_int, vp]
        L.cvattn_flash_attn_ext_noalloc.restype = ctypes.c_int
        PP = ctypes.POINTER(FaProblem)
        L.cvattn_fa_batch_workspace.argtypes = [PP, ctypes.c_int]
        L.cvattn_fa_batch_workspace.restype = sz
        L.cvattn_fa_batch_prepare.argtypes = [PP, ctypes.c_int, ctypes.c_float, vp, sz, vp, ctypes.POINTER(FaPlan)]
        L.cvattn_fa_batch_prepare.restype = ctypes.c_int
        L.cvattn_fa_batch_launch.argtypes = [ctypes.POINTER(FaPlan), vp]
        L.cvattn_fa_batch_launch.restype = ctypes.c_int
        L.cvattn_fa_batch_prepare_dynamic.argtypes = [PP, ctypes.c_int, ctypes.c_float, vp, ctypes.c_int, vp, sz, vp,
                                                      ctypes.POINTER(FaPlan)]
        L.cvattn_fa_batch_prepare_dynamic.restype = ctypes.c_int
        L.cvattn_shift_n_kv.argtypes = [vp, ctypes.c_int, ctypes.c_int32, vp]
        L.cvattn_shift_n_kv.restype = ctypes.c_int
        L.cvattn_block_size.argtypes = [ctypes.c_int]
        L.cvattn_block_size.restype = ctypes.c_int64
        L.cvattn_type_size.argtypes = [ctypes.c_int]
        L.cvattn_type_size.restype = ctypes.c_int64
        L.cvattn_dequantize.argtypes = [ctypes.c_int, vp, vp, ctypes.c_int64, vp]
        L.cvattn_dequantize.restype = ctypes.c_int
        L.cvattn_supports_set_rows.argtypes = [P, P, P]
        L.cvattn_supports_set_rows.restype = ctypes.c_int
        L.cvattn_set_rows.argtypes = [P, P, P, vp]
        L.cvattn_set_rows.restype = ctypes.c_int
        L.cvattn_supports_attn_nonfa.argtypes = [P, P, P, P]
        L.cvattn_supports_attn_nonfa.restype = ctypes.c_int
        L.cvattn_attn_nonfa_workspace.argtypes = [P, P, P, P]
        L.cvattn_attn_nonfa_workspace.restype = sz
        L.cvattn_attn_nonfa.argtypes = [P, P, P, P, P, ctypes.c_float, vp, sz, vp]
        L.cvattn_attn_nonfa.restype = ctypes.c_int
        DP = ctypes.POINTER(DitCacheParams)
        L.cvattn_dit_cache_device_bytes.argtypes = [DP]
        L.cvattn_dit_cache_device_bytes.restype = sz
        L.cvattn_dit_cache_host_bytes.argtypes = [DP]
        L.cvattn_dit_cache_host_bytes.restype = sz
        L.cvattn_dit_cache_create.argtypes = [DP, vp, sz, vp, sz, ctypes.POINTER(vp)]
        L.cvattn_dit_cache_create.restype = ctypes.c_int
        L.cvattn_dit_cache_destroy.argtypes = [vp]
        L.cvattn_dit_cache_destroy.restype = None
        L.cvattn_dit_cache_bind_slot.argtypes = [vp, ctypes.c_int]
        L.cvattn_dit_cache_bind_slot.restype = ctypes.c_int
        L.cvattn_dit_cache_slide.argtypes = [vp]
        L.cvattn_dit_cache_slide.restype = ctypes.c_int
        L.cvattn_dit_cache_slot.argtypes = [vp]
        L.cvattn_dit_cache_slot.restype = ctypes.c_int
        L.cvattn_dit_cache_set_len.argtypes = [vp, ctypes.c_uint32]
        L.cvattn_dit_cache_set_len.restype = ctypes.c_int
        L.cvattn_dit_cache_len.argtypes = [vp]
        L.cvattn_dit_cache_len.restype = ctypes.c_uint32
        L.cvattn_dit_cache_layer.argtypes = [vp, ctypes.c_int, ctypes.c_int64, P, P, P, P]
        L.cvattn_dit_cache_layer.restype = ctypes.c_int
        L.cvattn_dit_cache_offload.argtypes = [vp, ctypes.c_int, ctypes.c_uint32, vp]
        L.cvattn_dit_cache_offload.restype = ctypes.c_int
        L.cvattn_dit_cache_load.argtypes = [vp, ctypes.c_int, vp]
        L.cvattn_dit_cache_load.restype = ctypes.c_int
        L.cvattn_fill_positions.argtypes = [P, ctypes.c_int32, vp]
        L.cvattn_fill_positions.restype = ctypes.c_int
        L.cvattn_chunk_mask.argtypes = [P, ctypes.POINTER(ctypes.c_uint32), ctypes.c_int, vp]
        L.cvattn_chunk_mask.restype = ctypes.c_int
        L.cvattn_v_idxs.argtypes = [vp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp]
        L.cvattn_v_idxs.restype = ctypes.c_int
        L.cvattn_dit_schedule.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32,
                                          ctypes.c_int, ctypes.c_int, ctypes.POINTER(DitStep)]
        L.cvattn_dit_schedule.restype = ctypes.c_int
        L.cvattn_rope.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, vp]
        L.cvattn_rope.restype = ctypes.c_int
        L.cvattn_rope_set_rows.argtypes = [P, P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                           ctypes.c_float, vp]
        L.cvattn_rope_set_rows.restype = ctypes.c_int
        L.cvattn_status_string.argtypes = [ctypes.c_int]
        L.cvattn_status_string.restype = ctypes.c_char_p
        self.L = L

    # -- flash attention --
    @staticmethod
    def _p(t):
        return ctypes.byref(t) if t is not None else None

    def supports_flash_attn_ext(self, q, k, v, mask=None) -> bool:
        return bool(self.L.cvattn_supports_flash_attn_ext(self._p(q), self._p(k), self._p(v), self._p(mask)))

    def flash_attn_ext_workspace(self, q, k, v, mask=None) -> int:
        return int(self.L.cvattn_flash_attn_ext_workspace(self._p(q), self._p(k), self._p(v), self._p(mask)))

    def flash_attn_ext(self, q, k, v, mask, dst, scale, ws=0, ws_bytes=0, stream=0, max_bias=0.0,
                       softcap=0.0, prec=PREC_F32) -> int:
        return int(self.L.cvattn_flash_attn_ext(self._p(q), self._p(k), self._p(v), self._p(mask), self._p(dst),
                                                scale, max_bias, softcap, prec, ws or None, ws_bytes,
                                                stream or None))

    def flash_attn_ext_noalloc(self, q, k, v, mask, dst, scale, stream=0, max_bias=0.0, softcap=0.0,
                               prec=PREC_F32) -> int:
        return int(self.L.cvattn_flash_attn_ext_noalloc(self._p(q), self._p(k), self._p(v), self._p(mask),
                                                        self._p(dst), scale, max_bias, softcap, prec, stream or None))

    def fa_batch_workspace(self, problems) -> int:
        arr = (FaProblem * len(problems))(*problems)
        return int(self.L.cvattn_fa_batch_workspace(arr, len(problems)))

    def fa_batch_prepare(self, problems, scale, ws, ws_bytes, stream=0):
        arr = (FaProblem * len(problems))(*problems)
        plan = FaPlan()
        rc = int(self.L.cvattn_fa_batch_prepare(arr, len(problems), scale, ws or None, ws_bytes, stream or None,
                                                ctypes.byref(plan)))
        return rc, plan

    def fa_batch_launch(self, plan, stream=0) -> int:
        return int(self.L.cvattn_fa_batch_launch(ctypes.byref(plan), stream or None))

    def fa_batch_prepare_dynamic(self, problems, scale, n_kv_dev, n_kv_stride, ws, ws_bytes, stream=0):
        arr = (FaProblem * len(problems))(*problems)
        plan = FaPlan()
        rc = int(self.L.cvattn_fa_batch_prepare_dynamic(arr, len(problems), scale, n_kv_dev or None, n_kv_stride,
                                                        ws or None, ws_bytes, stream or None, ctypes.byref(plan)))
        return rc, plan

    def shift_n_kv(self, n_kv_dev, n, delta, stream=0) -> int:
        return int(self.L.cvattn_shift_n_kv(n_kv_dev or None, n, delta, stream or None))

    # -- formats / KV write --
    def block_size(self, t) -> int:
        return int(self.L.cvattn_block_size(t))

    def type_size(self, t) -> int:
        return int(self.L.cvattn_type_size(t))

    def dequantize(self, t, src, dst, n, stream=0) -> int:
        return int(self.L.cvattn_dequantize(t, src or None, dst or None, n, stream or None))

    def supports_set_rows(self, dst, src, idx) -> bool:
        return bool(self.L.cvattn_supports_set_rows(self._p(dst), self._p(src), self._p(idx)))

    def set_rows(self, dst, src, idx, stream=0) -> int:
        return int(self.L.cvattn_set_rows(self._p(dst), self._p(src), self._p(idx), stream or None))

    def supports_attn_nonfa(self, q, k, vt, mask=None) -> bool:
        return bool(self.L.cvattn_supports_attn_nonfa(self._p(q), self._p(k), self._p(vt), self._p(mask)))

    def attn_nonfa_workspace(self, q, k, vt, mask=None) -> int:
        return int(self.L.cvattn_attn_nonfa_workspace(self._p(q), self._p(k), self._p(vt), self._p(mask)))

    def attn_nonfa(self, q, k, vt, mask, dst, scale, ws=0, ws_bytes=0, stream=0) -> int:
        return int(self.L.cvattn_attn_nonfa(self._p(q), self._p(k), self._p(vt), self._p(mask), self._p(dst), scale,
                                            ws or None, ws_bytes, stream or None))

    def rope(self, dst, src, pos, n_dims, mode, freq_base, freq_scale=1.0, stream=0) -> int:
        return int(self.L.cvattn_rope(self._p(dst), self._p(src), self._p(pos), n_dims, mode, freq_base, freq_scale,
                                      stream or None))

    def rope_set_rows(self, dst, src, idx, pos, head, n_dims, mode, freq_base, freq_scale=1.0, stream=0) -> int:
        return int(self.L.cvattn_rope_set_rows(self._p(dst), self._p(src), self._p(idx), self._p(pos), head, n_dims,
                                               mode, freq_base, freq_scale, stream or None))

    # -- DiT streaming cache --
    def dit_cache_bytes(self, params: DitCacheParams):
        return (int(self.L.cvattn_dit_cache_device_bytes(ctypes.byref(params))),
                int(self.L.cvattn_dit_cache_host_bytes(ctypes.byref(params))))

    def dit_cache_create(self, params: DitCacheParams, dev_ptr, dev_bytes, host_ptr=0, host_bytes=0):
        h = ctypes.c_void_p()
        rc = self.L.cvattn_dit_cache_create(ctypes.byref(params), dev_ptr or None, dev_bytes, host_ptr or None,
                                            host_bytes, ctypes.byref(h))
        return rc, h

    def dit_cache_layer(self, cache, layer, n_kv):
        ts = [Tensor() for _ in range(4)]
        rc = self.L.cvattn_dit_cache_layer(cache, layer, n_kv, *[ctypes.byref(t) for t in ts])
        return rc, ts

    def chunk_mask(self, mask, bounds, stream=0) -> int:
        arr = (ctypes.c_uint32 * max(1, len(bounds)))(*[int(b) for b in bounds])
        return int(self.L.cvattn_chunk_mask(self._p(mask), arr, len(bounds), stream or None))

    def fill_positions(self, pos, base, stream=0) -> int:
        return int(self.L.cvattn_fill_positions(self._p(pos), base, stream or None))

    def v_idxs(self, idx_ptr, pos_ptr, n_tokens, n_per_batch, n_embd, max_seq, stream=0) -> int:
        return int(self.L.cvattn_v_idxs(idx_ptr or None, pos_ptr or None, n_tokens, n_per_batch, n_embd, max_seq,
                                        stream or None))

    def dit_schedule(self, n_steps, n_fixed, n_offloadable, cut_len, offset, streaming, kv_slidable):
        out = (DitStep * n_steps)()
        rc = self.L.cvattn_dit_schedule(n_steps, n_fixed, n_offloadable, cut_len, offset, int(streaming),
                                        int(kv_slidable), out)
        return rc, list(out)

    def status_string(self, rc) -> str:
        return self.L.cvattn_status_string(rc).decode()


EXPORTED = [
    "cvattn_supports_flash_attn_ext", "cvattn_flash_attn_ext_workspace", "cvattn_flash_attn_ext",
    "cvattn_flash_attn_ext_noalloc",
    "cvattn_fa_batch_workspace", "cvattn_fa_batch_prepare", "cvattn_fa_batch_launch",
    "cvattn_fa_batch_prepare_dynamic", "cvattn_shift_n_kv",
    "cvattn_block_size", "cvattn_type_size", "cvattn_dequantize",
    "cvattn_supports_set_rows", "cvattn_set_rows", "cvattn_rope", "cvattn_rope_set_rows",
    "cvattn_supports_attn_nonfa", "cvattn_attn_nonfa_workspace", "cvattn_attn_nonfa",
    "cvattn_dit_cache_device_bytes", "cvattn_dit_cache_host_bytes", "cvattn_dit_cache_create",
    "cvattn_dit_cache_destroy", "cvattn_dit_cache_bind_slot", "cvattn_dit_cache_slide", "cvattn_dit_cache_slot",
    "cvattn_dit_cache_set_len", "cvattn_dit_cache_len", "cvattn_dit_cache_layer", "cvattn_dit_cache_offload",
    "cvattn_dit_cache_load", "cvattn_fill_positions", "cvattn_chunk_mask", "cvattn_v_idxs", "cvattn_dit_schedule", "cvattn_status_string",
]

_lib = None


def lib() -> Lib:
    global _lib
    if _lib is None:
        _lib = Lib()
    return _lib
