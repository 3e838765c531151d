"""ctypes binding of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the
checker (or the timed CPU baseline).  Functions take numpy arrays in host memory.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
ROPE_NORMAL, ROPE_NEOX = 0, 2
BLOCK = {F32: 1, F16: 1, Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32}
TYPE_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34}
QUANT_TYPES = [Q8_0, Q4_0, Q4_1, Q5_0, Q5_1]
KV_TYPES = [F32, F16] + QUANT_TYPES


class OrTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


def row_bytes(t: int, n: int) -> int:
    assert n % BLOCK[t] == 0
    return n // BLOCK[t] * TYPE_BYTES[t]


def view(buf: np.ndarray, ttype: int, ne, nb, offset: int = 0) -> OrTensor:
    """Descriptor over a host numpy buffer (kept alive by the caller)."""
    t = OrTensor()
    t.data = ctypes.c_void_p(buf.ctypes.data + offset)
    t.type = ttype
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


class Oracle:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise ImportError(f"liboracle.so not built at {path}; run `make -C oracle`")
        L = ctypes.CDLL(path)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        P = ctypes.POINTER(OrTensor)
        L.or_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.or_fp32_to_fp16.restype = ctypes.c_uint16
        L.or_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.or_fp16_to_fp32.restype = ctypes.c_float
        L.or_fp32_to_fp16_row.argtypes = [vp, vp, i64]
        L.or_fp16_to_fp32_row.argtypes = [vp, vp, i64]
        L.or_quantize_row.argtypes = [ctypes.c_int, vp, vp, i64]
        L.or_quantize_row.restype = ctypes.c_int
        L.or_dequantize_row.argtypes = [ctypes.c_int, vp, vp, i64]
        L.or_dequantize_row.restype = ctypes.c_int
        L.or_quantize_row_q8_0_cpu.argtypes = [vp, vp, i64]
        L.or_flash_attn_ext_f64.argtypes = [P, P, P, P, vp, ctypes.c_float]
        L.or_flash_attn_ext_f64.restype = ctypes.c_int
        L.or_flash_attn_ext_ggml_cpu.argtypes = [P, P, P, P, vp, ctypes.c_float, ctypes.c_int]
        L.or_flash_attn_ext_ggml_cpu.restype = ctypes.c_int
        L.or_attn_nonfa_f64.argtypes = [P, P, P, P, vp, ctypes.c_float]
        L.or_attn_nonfa_f64.restype = ctypes.c_int
        L.or_causal_mask.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32]
        L.or_chunk_mask.argtypes = [vp, i64, vp, i64]
        L.or_set_rows.argtypes = [vp, ctypes.c_int, ctypes.c_size_t, i64, vp, ctypes.c_size_t, i64, vp, i64]
        L.or_set_rows.restype = ctypes.c_int
        L.or_rope_f32.argtypes = [vp, vp, i64, i64, vp, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        L.or_rope_f32.restype = ctypes.c_int
        self.L = L

    # -- fp16 --
    def f32_to_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(x.shape, dtype=np.uint16)
        self.L.or_fp32_to_fp16_row(x.ctypes.data, y.ctypes.data, x.size)
        return y

    def f16_to_f32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        y = np.empty(h.shape, dtype=np.float32)
        self.L.or_fp16_to_fp32_row(h.ctypes.data, y.ctypes.data, h.size)
        return y

    # -- blocks --
    def quantize(self, ttype: int, x: np.ndarray) -> np.ndarray:
        """Rows of x (last dim) -> ggml bytes, uint8 [..., row_bytes]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[-1]
        rb = row_bytes(ttype, n)
        y = np.zeros(x.shape[:-1] + (rb,), dtype=np.uint8)
        rows = x.reshape(-1, n)
        yr = y.reshape(-1, rb)
        for r in range(rows.shape[0]):
            rc = self.L.or_quantize_row(ttype, rows[r].ctypes.data, yr[r].ctypes.data, n)
            assert rc == 0
        return y

    def quantize_flat(self, ttype: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.zeros(row_bytes(ttype, x.size), dtype=np.uint8)
        assert self.L.or_quantize_row(ttype, x.ctypes.data, y.ctypes.data, x.size) == 0
        return y

    def dequantize(self, ttype: int, b: np.ndarray, n: int) -> np.ndarray:
        b = np.ascontiguousarray(b, dtype=np.uint8)
        y = np.empty(n, dtype=np.float32)
        assert self.L.or_dequantize_row(ttype, b.ctypes.data, y.ctypes.data, n) == 0
        return y

    def quantize_q8_0_cpu(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        y = np.zeros(row_bytes(Q8_0, x.size), dtype=np.uint8)
        self.L.or_quantize_row_q8_0_cpu(x.ctypes.data, y.ctypes.data, x.size)
        return y

    # -- attention --
    def fa_f64(self, q: OrTensor, k: OrTensor, v: OrTensor, mask, scale: float, out_shape) -> np.ndarray:
        dst = np.zeros(out_shape, dtype=np.float32)
        rc = self.L.or_flash_attn_ext_f64(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v),
                                          ctypes.byref(mask) if mask is not None else None, dst.ctypes.data, scale)
        assert rc == 0
        return dst

    def fa_ggml_cpu(self, q, k, v, mask, scale: float, out_shape, n_threads: int = 1) -> np.ndarray:
        dst = np.zeros(out_shape, dtype=np.float32)
        rc = self.L.or_flash_attn_ext_ggml_cpu(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v),
                                               ctypes.byref(mask) if mask is not None else None, dst.ctypes.data,
                                               scale, n_threads)
        assert rc == 0
        return dst

    def attn_nonfa_f64(self, q, k, vt, mask, scale: float, out_shape) -> np.ndarray:
        dst = np.zeros(out_shape, dtype=np.float32)
        rc = self.L.or_attn_nonfa_f64(ctypes.byref(q), ctypes.byref(k), ctypes.byref(vt),
                                      ctypes.byref(mask) if mask is not None else None, dst.ctypes.data, scale)
        assert rc == 0
        return dst

    # -- masks / KV write --
    def causal_mask(self, n_batch: int, seq_len: int) -> np.ndarray:
        m = np.zeros((n_batch, seq_len), dtype=np.uint16)
        self.L.or_causal_mask(m.ctypes.data, n_batch, seq_len)
        return m

    def chunk_mask(self, n: int, bounds) -> np.ndarray:
        b = np.ascontiguousarray(bounds, dtype=np.uint32)
        m = np.zeros((n, n), dtype=np.uint16)
        self.L.or_chunk_mask(m.ctypes.data, n, b.ctypes.data if b.size else None, b.size)
        return m

    def set_rows(self, dst: np.ndarray, dst_type: int, dst_nb1: int, dst_rows: int, src: np.ndarray,
                 idx: np.ndarray) -> None:
        src = np.ascontiguousarray(src, dtype=np.float32)
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        rc = self.L.or_set_rows(dst.ctypes.data, dst_type, dst_nb1, dst_rows, src.ctypes.data, src.shape[-1] * 4,
                                src.shape[-1], idx.ctypes.data, idx.size)
        assert rc == 0

    def rope(self, x: np.ndarray, pos, n_dims: int, mode: int, freq_base: float, freq_scale: float = 1.0) -> np.ndarray:
        """ggml_rope_ext on rows of x[..., ne0]; pos gives one position per row (x.shape[:-1])."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        ne0 = x.shape[-1]
        n_rows = x.size // ne0
        p = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, dtype=np.int32), x.shape[:-1])).reshape(-1)
        y = np.empty_like(x)
        rc = self.L.or_rope_f32(x.ctypes.data, y.ctypes.data, ne0, n_rows, p.ctypes.data, n_dims, mode,
                                freq_base, freq_scale)
        if rc:
            raise ValueError("or_rope_f32 rejected its arguments")
        return y


def v_idxs(positions, n_tokens: int, n_tokens_per_batch: int, n_embd: int, max_seq: int) -> np.ndarray:
    """The element-scatter index of the transposed V cache, as cosyvoice_kv_cache::set_input_v_idxs
    fills it (src/cosyvoice-kv-cache.cpp:357-377): source element (token i, feature j) of the
    flattened [n_embd, n_tokens] V goes to element base(i) + j*max_seq of the flattened
    [max_seq, n_embd, batch] cache, base(i) = (i / n_tokens_per_batch)*max_seq*n_embd +
    positions[i % n_tokens_per_batch]."""
    pos = np.asarray(positions, dtype=np.int64)
    i = np.arange(n_tokens, dtype=np.int64)
    base = (i // n_tokens_per_batch) * max_seq * n_embd + pos[i % n_tokens_per_batch]
    j = np.arange(n_embd, dtype=np.int64)
    return (base[:, None] + j[None, :] * max_seq).reshape(-1).astype(np.int32)


_oracle = None


def oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle
