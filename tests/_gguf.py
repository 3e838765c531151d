"""An independent GGUF v3 writer and reader written from the published format (ggml's gguf.md):
used by the tests to make synthetic model and prompt-speech files and to read what the engine's
C++ writer produces.  Layout: "GGUF", u32 version 3, i64 n_tensors, i64 n_kv; key/values (string
key, i32 type, value; arrays as i32 element type, u64 count, elements; strings as u64 length +
bytes); tensor infos (string name, u32 n_dims, i64 ne[n_dims], i32 ggml type, u64 offset); zero
padding to the alignment (32, or the u32 general.alignment); each tensor's bytes padded to it."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
       I64: "<q", F64: "<d"}
NP = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32, F32: np.float32,
      BOOL: np.uint8, U64: np.uint64, I64: np.int64, F64: np.float64}

# ggml type -> (block bytes, block elements) for the types the tests write
GGML = {0: (4, 1), 1: (2, 1), 2: (18, 32), 3: (20, 32), 6: (22, 32), 7: (24, 32), 8: (34, 32), 12: (144, 256),
        24: (1, 1), 26: (4, 1), 30: (2, 1)}


def gstr(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def pad(n, a):
    return (n + a - 1) // a * a


def value_bytes(t, v):
    if t == STR:
        return gstr(v)
    if t not in FMT:  # a type code outside the format: raw bytes, for malformed-file tests
        return bytes(v)
    return struct.pack(FMT[t], v)


def write(kvs, tensors, alignment=32, version=3):
    """kvs: [(key, type, value)] with type ARR values given as (elem_type, [values]);
    tensors: [(name, ggml_type, ne list, raw bytes)].  Returns the image bytes."""
    out = bytearray(b"GGUF" + struct.pack("<I", version) + struct.pack("<qq", len(tensors), len(kvs)))
    for key, t, v in kvs:
        out += gstr(key) + struct.pack("<i", t)
        if t == ARR:
            et, vals = v
            out += struct.pack("<iQ", et, len(vals))
            for x in vals:
                out += value_bytes(et, x)
        else:
            out += value_bytes(t, v)
    off = 0
    for name, gt, ne, data in tensors:
        out += gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<q", n) for n in ne)
        out += struct.pack("<iQ", gt, off)
        off += pad(len(data), alignment)
    out += bytes(pad(len(out), alignment) - len(out))
    for name, gt, ne, data in tensors:
        out += data
        out += bytes(pad(len(out), alignment) - len(out))
    return bytes(out)


def tensor_bytes(gt, ne):
    size, blck = GGML[gt]
    n = 1
    for x in ne[1:]:
        n *= x
    return ne[0] // blck * size * n


def read(img):
    """Returns (kv dict key -> (type, value), [(name, ggml_type, ne, bytes, offset)], alignment)."""
    p = 0

    def take(fmt):
        nonlocal p
        v = struct.unpack_from(fmt, img, p)
        p += struct.calcsize(fmt)
        return v[0] if len(v) == 1 else v

    def s():
        nonlocal p
        n = take("<Q")
        b = img[p:p + n]
        p += n
        return b.decode()

    assert img[:4] == b"GGUF"
    p = 4
    assert take("<I") == 3
    nt, nkv = take("<q"), take("<q")
    kv = {}
    for _ in range(nkv):
        k = s()
        t = take("<i")
        if t == ARR:
            et, n = take("<i"), take("<Q")
            kv[k] = (ARR, (et, [s() if et == STR else take(FMT[et]) for _ in range(n)]))
        else:
            kv[k] = (t, s() if t == STR else take(FMT[t]))
    infos = []
    for _ in range(nt):
        name = s()
        nd = take("<I")
        ne = [take("<q") for _ in range(nd)]
        gt, off = take("<i"), take("<Q")
        infos.append((name, gt, ne, off))
    align = kv.get("general.alignment", (U32, 32))[1]
    base = pad(p, align)
    return kv, [(n, gt, ne, img[base + off:base + off + tensor_bytes(gt, ne)], off) for n, gt, ne, off in infos], align
