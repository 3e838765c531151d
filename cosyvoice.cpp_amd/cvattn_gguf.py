"""ctypes binding of the model-file side of the engine (include/cvattn_gguf.h, in
libcvattn_host.so): the GGUF v3 reader, the attention geometry of a CosyVoice3 model file, and the
prompt-speech asset.  Host code only; nothing here touches the GPU."""
from __future__ import annotations

import ctypes
import os

import cvattn

HERE = os.path.dirname(os.path.abspath(__file__))
HOST_LIB_PATH = os.path.join(HERE, "libcvattn_host.so")

(T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, T_UINT64, T_INT64,
 T_FLOAT64, T_COUNT) = range(14)


class LlmAttnConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("n_layers", "n_heads", "n_kv_heads", "k_head_dim", "v_head_dim")] + \
               [("rope_theta", ctypes.c_float)]


class DitAttnConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("depth", "heads", "k_head_dim", "v_head_dim")]


class PromptSpeechView(ctypes.Structure):
    _fields_ = [("text", ctypes.c_void_p), ("text_len", ctypes.c_uint32),
                ("feat", ctypes.c_void_p), ("feat_rows", ctypes.c_uint32), ("feat_cols", ctypes.c_uint32),
                ("embedding", ctypes.c_void_p), ("emb_rows", ctypes.c_uint32), ("emb_cols", ctypes.c_uint32),
                ("tokens", ctypes.c_void_p), ("n_tokens", ctypes.c_uint32)]


EXPORTED = [
    "cvattn_gguf_open", "cvattn_gguf_close", "cvattn_gguf_alignment", "cvattn_gguf_n_kv", "cvattn_gguf_find_key",
    "cvattn_gguf_key", "cvattn_gguf_kv_type", "cvattn_gguf_arr_type", "cvattn_gguf_val_u32", "cvattn_gguf_val_i32",
    "cvattn_gguf_val_f32", "cvattn_gguf_val_data", "cvattn_gguf_val_str", "cvattn_gguf_arr_n", "cvattn_gguf_arr_data",
    "cvattn_gguf_arr_str", "cvattn_gguf_n_tensors", "cvattn_gguf_find_tensor", "cvattn_gguf_tensor",
    "cvattn_gguf_llm_attn_config", "cvattn_gguf_dit_attn_config", "cvattn_prompt_speech_load",
    "cvattn_prompt_speech_load_from_file", "cvattn_prompt_speech_save_to_file", "cvattn_prompt_speech_get_crc32",
    "cvattn_prompt_speech_free", "cvattn_prompt_speech_create", "cvattn_prompt_speech_get",
]


class HostLib:
    def __init__(self, path: str = HOST_LIB_PATH):
        if not os.path.exists(path):
            raise ImportError(f"libcvattn_host.so not built at {path}; run __graft_entry__.build()")
        self.path = path
        L = ctypes.CDLL(path, use_errno=True)
        vp, sz, i64, u32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_uint32
        cp = ctypes.c_char_p
        L.cvattn_gguf_open.argtypes = [vp, sz, ctypes.POINTER(vp), ctypes.c_char_p, sz]
        L.cvattn_gguf_open.restype = ctypes.c_int
        L.cvattn_gguf_close.argtypes = [vp]
        L.cvattn_gguf_close.restype = None
        L.cvattn_gguf_alignment.argtypes = [vp]
        L.cvattn_gguf_alignment.restype = sz
        L.cvattn_gguf_n_kv.argtypes = [vp]
        L.cvattn_gguf_n_kv.restype = i64
        L.cvattn_gguf_find_key.argtypes = [vp, cp]
        L.cvattn_gguf_find_key.restype = i64
        L.cvattn_gguf_key.argtypes = [vp, i64]
        L.cvattn_gguf_key.restype = cp
        for f in ("cvattn_gguf_kv_type", "cvattn_gguf_arr_type"):
            getattr(L, f).argtypes = [vp, i64]
            getattr(L, f).restype = ctypes.c_int
        L.cvattn_gguf_val_u32.argtypes = [vp, i64]
        L.cvattn_gguf_val_u32.restype = u32
        L.cvattn_gguf_val_i32.argtypes = [vp, i64]
        L.cvattn_gguf_val_i32.restype = ctypes.c_int32
        L.cvattn_gguf_val_f32.argtypes = [vp, i64]
        L.cvattn_gguf_val_f32.restype = ctypes.c_float
        L.cvattn_gguf_val_data.argtypes = [vp, i64, ctypes.POINTER(sz)]
        L.cvattn_gguf_val_data.restype = vp
        L.cvattn_gguf_val_str.argtypes = [vp, i64]
        L.cvattn_gguf_val_str.restype = cp
        L.cvattn_gguf_arr_n.argtypes = [vp, i64]
        L.cvattn_gguf_arr_n.restype = sz
        L.cvattn_gguf_arr_data.argtypes = [vp, i64]
        L.cvattn_gguf_arr_data.restype = vp
        L.cvattn_gguf_arr_str.argtypes = [vp, i64, sz, ctypes.POINTER(sz)]
        L.cvattn_gguf_arr_str.restype = vp
        L.cvattn_gguf_n_tensors.argtypes = [vp]
        L.cvattn_gguf_n_tensors.restype = i64
        L.cvattn_gguf_find_tensor.argtypes = [vp, cp]
        L.cvattn_gguf_find_tensor.restype = i64
        L.cvattn_gguf_tensor.argtypes = [vp, i64, ctypes.POINTER(cvattn.Tensor), ctypes.POINTER(cp),
                                         ctypes.POINTER(ctypes.c_uint64)]
        L.cvattn_gguf_tensor.restype = ctypes.c_int
        L.cvattn_gguf_llm_attn_config.argtypes = [vp, cp, ctypes.POINTER(LlmAttnConfig)]
        L.cvattn_gguf_llm_attn_config.restype = ctypes.c_int
        L.cvattn_gguf_dit_attn_config.argtypes = [vp, cp, ctypes.POINTER(DitAttnConfig)]
        L.cvattn_gguf_dit_attn_config.restype = ctypes.c_int
        L.cvattn_prompt_speech_load.argtypes = [vp, sz]
        L.cvattn_prompt_speech_load.restype = vp
        L.cvattn_prompt_speech_load_from_file.argtypes = [cp]
        L.cvattn_prompt_speech_load_from_file.restype = vp
        L.cvattn_prompt_speech_save_to_file.argtypes = [vp, cp]
        L.cvattn_prompt_speech_save_to_file.restype = ctypes.c_int
        L.cvattn_prompt_speech_get_crc32.argtypes = [vp]
        L.cvattn_prompt_speech_get_crc32.restype = u32
        L.cvattn_prompt_speech_free.argtypes = [vp]
        L.cvattn_prompt_speech_free.restype = None
        L.cvattn_prompt_speech_create.argtypes = [vp, u32, vp, u32, u32, vp, u32, u32, vp, u32]
        L.cvattn_prompt_speech_create.restype = vp
        L.cvattn_prompt_speech_get.argtypes = [vp, ctypes.POINTER(PromptSpeechView)]
        L.cvattn_prompt_speech_get.restype = ctypes.c_int
        self.L = L


class Gguf:
    """A parsed GGUF image (keeps the bytes alive: tensors and string arrays point into them)."""

    def __init__(self, lib: HostLib, data: bytes):
        self.lib, self.L = lib, lib.L
        self.buf = ctypes.create_string_buffer(bytes(data), len(data)) if data else None
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        self.rc = self.L.cvattn_gguf_open(ctypes.cast(self.buf, ctypes.c_void_p) if self.buf else None, len(data),
                                          ctypes.byref(h), err, 256)
        self.error = err.value.decode(errors="replace")
        self.h = h.value

    def __bool__(self):
        return self.rc == cvattn.OK

    def close(self):
        if self.h:
            self.L.cvattn_gguf_close(self.h)
            self.h = None

    def __del__(self):  # pragma: no cover - finaliser
        try:
            self.close()
        except Exception:
            pass

    def find_key(self, key: str) -> int:
        return int(self.L.cvattn_gguf_find_key(self.h, key.encode()))

    def tensor(self, i: int):
        t = cvattn.Tensor()
        name = ctypes.c_char_p()
        off = ctypes.c_uint64()
        rc = self.L.cvattn_gguf_tensor(self.h, i, ctypes.byref(t), ctypes.byref(name), ctypes.byref(off))
        return rc, t, (name.value.decode() if name.value is not None else None), off.value

    def data_offset(self, ptr: int) -> int:
        """Byte offset of a pointer the library returned, from the start of the parsed image."""
        return ptr - ctypes.addressof(self.buf)
