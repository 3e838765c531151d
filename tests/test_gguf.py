"""The model-file side (include/cvattn_gguf.h): the GGUF v3 reader that cosyvoice.cpp's loader and
prompt assets go through (common/gguf_parser.cpp:142-407), the attention geometry the loader reads
from a CosyVoice3 file (src/cosyvoice-loader.cpp:247-251,447-454,996-1025), and the prompt-speech
asset (src/cosyvoice-prompt.cpp:8-108,213-241).

No model or prompt file ships with the reference, so the files here are synthetic, written by an
independent implementation of the published GGUF layout (tests/_gguf.py); the engine's own writer
is read back by that implementation and compared byte for byte with it.  The prompt checksum is
pinned to zlib's CRC-32 through the closed form of the reference's chaining (it starts from 0 and
feeds each result back un-inverted): crc(bytes, v) = zlib.crc32(bytes, v ^ 0xFFFFFFFF)."""
import ctypes
import errno
import os
import struct
import zlib

import numpy as np
import pytest

import _gguf as G
import cvattn
import cvattn_gguf as CG


@pytest.fixture(scope="module")
def host():
    return CG.HostLib()


def parse(host, img):
    return CG.Gguf(host, img)


def f16(x):
    return np.asarray(x, dtype=np.float16).tobytes()


# ------------------------------------------------------------------------------------------
# the reader
# ------------------------------------------------------------------------------------------
KVS = [("general.architecture", G.STR, "cosyvoice3"),
       ("u8", G.U8, 200), ("i8", G.I8, -5), ("u16", G.U16, 60000), ("i16", G.I16, -30000),
       ("u32", G.U32, 4000000000), ("i32", G.I32, -123456), ("f32", G.F32, 1.5), ("bool", G.BOOL, True),
       ("u64", G.U64, 1 << 40), ("i64", G.I64, -(1 << 40)), ("f64", G.F64, 2.25),
       ("arr.i32", G.ARR, (G.I32, [1, -2, 3, 7])), ("arr.f32", G.ARR, (G.F32, [0.5, 1.25])),
       ("arr.str", G.ARR, (G.STR, ["a", "", "héllo"])), ("arr.empty", G.ARR, (G.U8, [])),
       ("empty.str", G.STR, "")]


def tensors(rng):
    out = []
    for name, gt, ne in (("w.f32", 0, [7, 3]), ("w.f16", 1, [64, 2, 3]), ("k.q8_0", 8, [128, 5]),
                         ("v.q4_0", 2, [64, 4, 1, 2]), ("ids", 26, [9]), ("text", 24, [11]), ("bf", 30, [5]),
                         ("k.q4_K", 12, [256, 2]), ("empty", 0, [0, 4])):
        n = G.tensor_bytes(gt, ne)
        out.append((name, gt, ne, rng.integers(0, 256, n, dtype=np.uint8).tobytes()))
    return out


@pytest.mark.parametrize("alignment", [32, 64, 1])
def test_reader_round_trips_every_value_and_tensor(host, alignment):
    rng = np.random.default_rng(alignment)
    kvs = list(KVS)
    if alignment != 32:
        kvs.append(("general.alignment", G.U32, alignment))
    ts = tensors(rng)
    img = G.write(kvs, ts, alignment=alignment)
    g = parse(host, img)
    assert g, g.error
    L, h = host.L, g.h
    assert L.cvattn_gguf_alignment(h) == alignment
    assert L.cvattn_gguf_n_kv(h) == len(kvs)
    for i, (k, t, v) in enumerate(kvs):
        assert g.find_key(k) == i
        assert L.cvattn_gguf_key(h, i).decode() == k
        assert L.cvattn_gguf_kv_type(h, i) == t
        if t == G.ARR:
            et, vals = v
            assert L.cvattn_gguf_arr_type(h, i) == et
            assert L.cvattn_gguf_arr_n(h, i) == len(vals)
            if et == G.STR:
                assert L.cvattn_gguf_arr_data(h, i) is None
                for j, sv in enumerate(vals):
                    n = ctypes.c_size_t()
                    p = L.cvattn_gguf_arr_str(h, i, j, ctypes.byref(n))
                    assert ctypes.string_at(p, n.value).decode() == sv
                    assert g.data_offset(p) > 0   # points into the image: no copy
            elif vals:
                p = L.cvattn_gguf_arr_data(h, i)
                got = np.frombuffer(ctypes.string_at(p, len(vals) * np.dtype(G.NP[et]).itemsize), dtype=G.NP[et])
                assert np.array_equal(got, np.array(vals, dtype=G.NP[et]))
        elif t == G.STR:
            assert L.cvattn_gguf_val_str(h, i).decode() == v
            assert L.cvattn_gguf_arr_type(h, i) == CG.T_COUNT
        else:
            n = ctypes.c_size_t()
            p = L.cvattn_gguf_val_data(h, i, ctypes.byref(n))
            assert ctypes.string_at(p, n.value) == struct.pack(G.FMT[t], v)
    # scalar accessors read the first four bytes as the reference does, 0 for narrower values
    assert L.cvattn_gguf_val_u32(h, g.find_key("u32")) == 4000000000
    assert L.cvattn_gguf_val_i32(h, g.find_key("i32")) == -123456
    assert L.cvattn_gguf_val_f32(h, g.find_key("f32")) == 1.5
    assert L.cvattn_gguf_val_u32(h, g.find_key("u16")) == 0
    assert L.cvattn_gguf_val_u32(h, g.find_key("u64")) == 0     # low word of 2^40
    assert g.find_key("missing") == -1
    # tensors: descriptors with contiguous strides and data in the image's data section
    assert L.cvattn_gguf_n_tensors(h) == len(ts)
    _, want_t, _ = G.read(img)
    for i, (name, gt, ne, data) in enumerate(ts):
        assert L.cvattn_gguf_find_tensor(h, name.encode()) == i
        rc, t, nm, off = g.tensor(i)
        assert rc == cvattn.OK and nm == name and t.type == gt
        full = list(ne) + [1] * (4 - len(ne))
        assert list(t.ne) == full
        size, blck = G.GGML[gt]
        nb = [size, full[0] // blck * size]
        nb += [nb[1] * full[1], nb[1] * full[1] * full[2]]
        assert list(t.nb) == nb
        assert off == want_t[i][4]
        if data:
            assert g.data_offset(t.data) % alignment == 0
            assert ctypes.string_at(t.data, len(data)) == data
    assert L.cvattn_gguf_find_tensor(h, b"nope") == -1
    assert g.tensor(len(ts))[0] == cvattn.ERR_BAD_ARGS


def corrupt_cases():
    good_t = [("w", 0, [4, 2], bytes(32))]
    img = G.write([("k", G.U32, 1)], good_t)
    hdr_end = 24
    yield "too small", img[:20], "too small"
    yield "magic", b"GGUX" + img[4:], "magic"
    yield "version 2", G.write([("k", G.U32, 1)], good_t, version=2), "version"
    yield "truncated kv", img[:hdr_end + 5], "truncated|exceed"
    yield "truncated tensor info", img[:img.index(b"\x01\x00\x00\x00\x00\x00\x00\x00w") + 12], "truncated|exceed"
    yield "negative counts", img[:8] + struct.pack("<qq", -1, 1) + img[24:], "counts"
    yield "huge counts", img[:8] + struct.pack("<qq", 1, 1 << 40) + img[24:], "exceed"
    yield "bad value type", G.write([("k", 99, b"")], []), "value type"
    yield "array of arrays", G.write([("k", G.ARR, (G.ARR, []))], []), "element type"
    yield "5 dims", G.write([], [("w", 0, [1, 1, 1, 1, 2], bytes(8))]), "dimensions"
    yield "negative dim", G.write([], [("w", 0, [-1], b"")]), "negative"
    yield "retired type", G.write([], [("w", 4, [32], bytes(20))]), "type"
    yield "unknown type", G.write([], [("w", 99, [32], bytes(20))]), "type"
    yield "ragged row", G.write([], [("w", 8, [48], bytes(34))]), "block"
    yield "long name", G.write([], [("x" * 64, 0, [1], bytes(4))]), "too long"
    yield "alignment 3", G.write([("general.alignment", G.U32, 3)], good_t), "power of 2"
    yield "alignment 0", G.write([("general.alignment", G.U32, 0)], good_t), "power of 2"
    # offsets not end to end
    two = G.write([], [("a", 0, [4], bytes(16)), ("b", 0, [4], bytes(16))])
    i = two.index(b"b") + 1 + 4 + 8 + 4     # name, n_dims, ne[0], type -> offset of the 2nd tensor
    yield "gap", two[:i] + struct.pack("<Q", 64) + two[i + 8:], "offset"
    yield "data beyond", img[:len(img) - 16], "beyond"
    yield "string too long", b"GGUF" + struct.pack("<Iqq", 3, 0, 1) + struct.pack("<Q", 1 << 31) + b"k" * 16, "truncated"


@pytest.mark.parametrize("what,img,msg", list(corrupt_cases()), ids=[c[0] for c in corrupt_cases()])
def test_reader_refuses_malformed_images(host, what, img, msg):
    g = parse(host, img)
    assert not g and g.rc == cvattn.ERR_BAD_ARGS and g.h is None
    assert any(m in g.error for m in msg.split("|")), (what, g.error)


def test_reader_takes_the_first_alignment_key_and_reads_it_as_the_reference(host):
    # a u8 alignment value has fewer than 4 bytes: the reference keeps the default
    img = G.write([("general.alignment", G.U8, 64)], [("w", 0, [4], bytes(16))], alignment=32)
    g = parse(host, img)
    assert g and host.L.cvattn_gguf_alignment(g.h) == 32


# ------------------------------------------------------------------------------------------
# the attention geometry of a CosyVoice3 file
# ------------------------------------------------------------------------------------------
def cosyvoice3_like(prefix_llm="", prefix_dit="decoder.estimator"):
    def k(prefix, name):
        return f"{prefix}.{name}" if prefix else name
    kvs = [(k(prefix_llm, "num_hidden_layers"), G.I32, 24), (k(prefix_llm, "num_attention_heads"), G.I32, 14),
           (k(prefix_llm, "num_key_value_heads"), G.I32, 2), (k(prefix_llm, "rope_theta"), G.F32, 1e6),
           (k(prefix_dit, "heads"), G.I32, 16), (k(prefix_dit, "depth"), G.I32, 22)]
    ts = [(k(k(prefix_llm, "layers"), "0.self_attn.q_proj.weight"), 1, [896, 896], None),
          (k(k(prefix_llm, "layers"), "0.self_attn.k_proj.weight"), 1, [896, 128], None),
          (k(k(prefix_llm, "layers"), "0.self_attn.v_proj.weight"), 1, [896, 128], None),
          (f"{prefix_dit}.transformer_blocks.0.attn.to_k.weight", 1, [1024, 1024], None),
          (f"{prefix_dit}.transformer_blocks.0.attn.to_v.weight", 1, [1024, 1024], None)]
    return G.write(kvs, [(n, gt, ne, bytes(G.tensor_bytes(gt, ne))) for n, gt, ne, _ in ts])


def test_attention_geometry_of_a_cosyvoice3_file(host):
    g = parse(host, cosyvoice3_like())
    assert g, g.error
    llm = CG.LlmAttnConfig()
    assert host.L.cvattn_gguf_llm_attn_config(g.h, b"", ctypes.byref(llm)) == cvattn.OK
    assert (llm.n_layers, llm.n_heads, llm.n_kv_heads, llm.k_head_dim, llm.v_head_dim) == (24, 14, 2, 64, 64)
    assert llm.rope_theta == 1e6
    dit = CG.DitAttnConfig()
    assert host.L.cvattn_gguf_dit_attn_config(g.h, b"decoder.estimator", ctypes.byref(dit)) == cvattn.OK
    assert (dit.depth, dit.heads, dit.k_head_dim, dit.v_head_dim) == (22, 16, 64, 64)
    # the same under an "llm" prefix, and a missing key refused
    g2 = parse(host, cosyvoice3_like(prefix_llm="llm"))
    assert host.L.cvattn_gguf_llm_attn_config(g2.h, b"llm", ctypes.byref(llm)) == cvattn.OK
    assert llm.n_kv_heads == 2 and llm.k_head_dim == 64
    assert host.L.cvattn_gguf_llm_attn_config(g2.h, b"", ctypes.byref(llm)) == cvattn.ERR_BAD_ARGS
    assert host.L.cvattn_gguf_dit_attn_config(g.h, b"flow", ctypes.byref(dit)) == cvattn.ERR_BAD_ARGS


def test_geometry_describes_the_engines_kv_views(host):
    """The geometry read from the file gives the LLM cache row the engine's views expect: H_kv heads
    of head_dim elements per token (q8_0: 2 x 68 B = 136 B)."""
    g = parse(host, cosyvoice3_like())
    llm = CG.LlmAttnConfig()
    assert host.L.cvattn_gguf_llm_attn_config(g.h, b"", ctypes.byref(llm)) == cvattn.OK
    v = cvattn.llm_kv_view(0x1000, cvattn.Q8_0, llm.k_head_dim, llm.n_kv_heads, 512, 4096)
    assert list(v.ne) == [64, 512, 2, 1] and v.nb[1] == 136 and v.nb[2] == 68
    lib = cvattn.lib()
    q = cvattn.llm_q_view(0x1000, llm.k_head_dim, llm.n_heads, 1)
    assert lib.supports_flash_attn_ext(q, v, v, None)


# ------------------------------------------------------------------------------------------
# prompt speech
# ------------------------------------------------------------------------------------------
def ref_crc(data: bytes, v: int) -> int:
    """The reference's crc32_context::calculate(data, len, v) in terms of zlib."""
    return zlib.crc32(data, v ^ 0xFFFFFFFF)


def expected_crc(text: bytes, feat, emb, tokens) -> int:
    c = ref_crc(text, 0)
    c = ref_crc(struct.pack("<I", len(text)), c)
    c = ref_crc(feat.astype("<f4").tobytes(), c)
    c = ref_crc(struct.pack("<II", *feat.shape), c)
    c = ref_crc(emb.astype("<f4").tobytes(), c)
    c = ref_crc(struct.pack("<II", *emb.shape), c)
    c = ref_crc(tokens.astype("<i4").tobytes(), c)
    c = ref_crc(struct.pack("<I", len(tokens)), c)
    return c


def sample(rng, rows=37, cols=80, n_tokens=25, text="希望你以后能够做的比我还好呦。"):
    t = text.encode()
    feat = rng.standard_normal((rows, cols)).astype(np.float32)
    emb = rng.standard_normal((1, 192)).astype(np.float32)
    tok = rng.integers(0, 6561, n_tokens).astype(np.int32)
    return t, feat, emb, tok


def create(host, t, feat, emb, tok):
    L = host.L
    ptr = lambda a: a.ctypes.data if a.size else None  # noqa: E731
    return L.cvattn_prompt_speech_create(t, len(t), ptr(feat), feat.shape[0], feat.shape[1], ptr(emb), emb.shape[0],
                                         emb.shape[1], ptr(tok), len(tok))


def view(host, p):
    v = CG.PromptSpeechView()
    assert host.L.cvattn_prompt_speech_get(p, ctypes.byref(v)) == cvattn.OK
    text = ctypes.string_at(v.text, v.text_len) if v.text_len else b""
    feat = np.frombuffer(ctypes.string_at(v.feat, 4 * v.feat_rows * v.feat_cols), np.float32).reshape(
        v.feat_rows, v.feat_cols) if v.feat_rows * v.feat_cols else np.zeros((v.feat_rows, v.feat_cols), np.float32)
    emb = np.frombuffer(ctypes.string_at(v.embedding, 4 * v.emb_rows * v.emb_cols), np.float32).reshape(
        v.emb_rows, v.emb_cols)
    tok = np.frombuffer(ctypes.string_at(v.tokens, 4 * v.n_tokens), np.int32) if v.n_tokens else np.zeros(0, np.int32)
    return text, feat, emb, tok


def n_dims(ne):
    """ggml writes a tensor's dimensions up to the last one above 1 (at least one)."""
    ne = list(ne)
    while len(ne) > 1 and ne[-1] == 1:
        ne.pop()
    return ne


def prompt_file(t, feat, emb, tok, crc=None, types=(0, 0, 26, 24)):
    kvs = [] if crc is None else [("crc32", G.U32, crc)]
    return G.write(kvs, [("feat", types[0], n_dims([feat.shape[1], feat.shape[0]]), feat.tobytes()),
                         ("embedding", types[1], n_dims([emb.shape[1], emb.shape[0]]), emb.tobytes()),
                         ("tokens", types[2], [len(tok)], tok.tobytes()),
                         ("text", types[3], [len(t)], t)])


def test_prompt_crc32_is_the_references_chained_checksum(host):
    rng = np.random.default_rng(1)
    t, feat, emb, tok = sample(rng)
    p = create(host, t, feat, emb, tok)
    assert p
    assert host.L.cvattn_prompt_speech_get_crc32(p) == expected_crc(t, feat, emb, tok)
    host.L.cvattn_prompt_speech_free(p)
    # a one-byte change of any part changes it
    feat2 = feat.copy()
    feat2[3, 7] = np.nextafter(feat2[3, 7], np.float32(10))
    p2 = create(host, t, feat2, emb, tok)
    assert host.L.cvattn_prompt_speech_get_crc32(p2) != expected_crc(t, feat, emb, tok)
    host.L.cvattn_prompt_speech_free(p2)


def test_prompt_speech_save_matches_the_format_and_loads_back(host, tmp_path):
    rng = np.random.default_rng(2)
    t, feat, emb, tok = sample(rng)
    p = create(host, t, feat, emb, tok)
    path = str(tmp_path / "prompt.gguf")
    assert host.L.cvattn_prompt_speech_save_to_file(p, path.encode()) == 1
    img = open(path, "rb").read()
    # byte-identical to the independent writer's file of the same content
    assert img == prompt_file(t, feat, emb, tok, crc=expected_crc(t, feat, emb, tok))
    kv, ts, _ = G.read(img)
    assert kv["crc32"] == (G.U32, expected_crc(t, feat, emb, tok))
    assert [x[0] for x in ts] == ["feat", "embedding", "tokens", "text"]
    assert ts[0][2] == [80, 37] and ts[1][2] == [192] and ts[3][3] == t
    q = host.L.cvattn_prompt_speech_load_from_file(path.encode())
    assert q
    t2, f2, e2, k2 = view(host, q)
    assert t2 == t and np.array_equal(f2, feat) and np.array_equal(e2, emb) and np.array_equal(k2, tok)
    assert host.L.cvattn_prompt_speech_get_crc32(q) == host.L.cvattn_prompt_speech_get_crc32(p)
    host.L.cvattn_prompt_speech_free(p)
    host.L.cvattn_prompt_speech_free(q)


def test_prompt_speech_load_from_memory_without_crc_key(host):
    rng = np.random.default_rng(3)
    t, feat, emb, tok = sample(rng, rows=1, n_tokens=0, text="")
    img = prompt_file(t, feat, emb, tok)
    buf = ctypes.create_string_buffer(img, len(img))
    p = host.L.cvattn_prompt_speech_load(buf, len(img))
    assert p
    t2, f2, e2, k2 = view(host, p)
    assert t2 == b"" and f2.shape == (1, 80) and np.array_equal(f2, feat) and k2.size == 0
    assert host.L.cvattn_prompt_speech_get_crc32(p) == expected_crc(t, feat, emb, tok)
    host.L.cvattn_prompt_speech_free(p)


@pytest.mark.parametrize("case", ["bad crc", "feat f16", "tokens f32", "text u8 as i32", "no text", "3-d feat",
                                  "not gguf"])
def test_prompt_speech_load_refuses_bad_files_with_eilseq(host, case):
    rng = np.random.default_rng(4)
    t, feat, emb, tok = sample(rng)
    crc = expected_crc(t, feat, emb, tok)
    if case == "bad crc":
        img = prompt_file(t, feat, emb, tok, crc=crc ^ 1)
    elif case == "feat f16":
        img = G.write([], [("feat", 1, [80, 37], f16(feat)), ("embedding", 0, [192, 1], emb.tobytes()),
                           ("tokens", 26, [len(tok)], tok.tobytes()), ("text", 24, [len(t)], t)])
    elif case == "tokens f32":
        img = prompt_file(t, feat, emb, tok, types=(0, 0, 0, 24))
    elif case == "text u8 as i32":
        img = prompt_file(t, feat, emb, tok.astype(np.int32), types=(0, 0, 26, 26)) if len(t) % 4 == 0 else \
            G.write([], [("feat", 0, [80, 37], feat.tobytes()), ("embedding", 0, [192, 1], emb.tobytes()),
                         ("tokens", 26, [len(tok)], tok.tobytes()), ("text", 26, [1], bytes(4))])
    elif case == "no text":
        img = G.write([], [("feat", 0, [80, 37], feat.tobytes()), ("embedding", 0, [192, 1], emb.tobytes()),
                           ("tokens", 26, [len(tok)], tok.tobytes())])
    elif case == "3-d feat":
        img = G.write([], [("feat", 0, [80, 37, 1, 1], feat.tobytes()), ("embedding", 0, [192, 1, 2], bytes(1536)),
                           ("tokens", 26, [len(tok)], tok.tobytes()), ("text", 24, [len(t)], t)])
    else:
        img = b"not a gguf file at all, definitely not" * 2
    buf = ctypes.create_string_buffer(img, len(img))
    ctypes.set_errno(0)
    p = host.L.cvattn_prompt_speech_load(buf, len(img))
    assert not p
    assert ctypes.get_errno() == errno.EILSEQ


def test_prompt_speech_missing_file(host, tmp_path):
    assert not host.L.cvattn_prompt_speech_load_from_file(str(tmp_path / "absent.gguf").encode())
    assert host.L.cvattn_prompt_speech_save_to_file(None, b"/tmp/x") == 0


def test_host_library_exports_every_declared_symbol(host):
    import re
    hdr = open(os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "cvattn_gguf.h")).read()
    syms = sorted(set(re.findall(r"CVATTN_API\s+[\w\s\*]+?\b(cvattn_\w+)\s*\(", hdr)))
    assert set(syms) == set(CG.EXPORTED)
    for s in syms:
        assert hasattr(host.L, s), s
