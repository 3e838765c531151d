"""Blocks whose quantizer inputs land exactly on rounding ties, with their expected codes written
out by hand from the tie rule of each ggml *_ref quantizer (restated in oracle/oracle.c):

  q8_0          q = roundf(x * id)                 ties away from zero
  q4_0 / q5_0   q = (int8)(x * id + 8.5 | 16.5)    truncation of a positive sum: ties round up
  q4_1 / q5_1   q = (int8)((x - min) * id + 0.5)   ties round up
  q8_0 x86 CPU  q = nearbyint(x * 127 / amax)      ties to even

Each block's scale is chosen so that |id| = 1 exactly (d = amax/127 with amax 127, d = max/-8 with
max -8, d = (max - min)/15 with max - min 15, ...), so x * id is the input itself and the ties are
exact in fp32.  A quantizer using rint instead of roundf, roundf instead of the +0.5 truncation,
or the truncation without its offset gives different codes on these blocks.
"""
import numpy as np

from oracle.oracle import Q4_0, Q4_1, Q5_0, Q5_1, Q8_0


def _half(x):
    v = int(np.float16(x).view(np.uint16))
    return [v & 0xFF, v >> 8]


def _pack_nibbles(codes):
    c = np.asarray(codes, dtype=np.int64)
    return [int((c[j] & 15) | ((c[j + 16] & 15) << 4)) for j in range(16)]


def _qh(codes):
    c = np.asarray(codes, dtype=np.int64)
    bits = 0
    for j in range(32):
        bits |= int((c[j] >> 4) & 1) << j
    return list(bits.to_bytes(4, "little"))


def _block(head, rest):
    x = np.zeros(32, dtype=np.float32)
    vals = list(head) + list(rest)
    x[: len(vals)] = vals
    return x


def tie_cases():
    """{type: [(x float32[32], expected bytes uint8[type size])]}"""
    ties = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5]
    out = {}
    # q8_0: amax 127 -> d = 1, id = 1.  roundf: +-0.5 -> +-1, +-1.5 -> +-2, +-2.5 -> +-3,
    # 126.5 -> 127 (rint would give 0, +-2, +-2, 126).
    x = _block([127.0], ties + [126.5, -126.5, 3.25])
    codes = [127, 1, -1, 2, -2, 3, -3, 127, -127, 3] + [0] * 22
    out[Q8_0] = [(x, np.array(_half(1.0) + list(np.array(codes, dtype=np.int8).view(np.uint8)), dtype=np.uint8))]
    # q4_0: the first max-|x| element is -8 -> d = -8/-8 = 1, id = 1; q = (int8)(x + 8.5), at most 15.
    # +0.5 -> 9, -0.5 -> 8, +1.5 -> 10, -1.5 -> 7, +2.5 -> 11, -2.5 -> 6, 7.5 -> 16 -> 15, -7.5 -> 1
    x = _block([-8.0], ties + [7.5, -7.5, 6.5])
    codes = [0, 9, 8, 10, 7, 11, 6, 15, 1, 15] + [8] * 22
    out[Q4_0] = [(x, np.array(_half(1.0) + _pack_nibbles(codes), dtype=np.uint8))]
    # the same with max +8: d = -1, id = -1, so x * id flips: +0.5 -> -0.5 + 8.5 = 8 ...
    x = _block([8.0], ties)
    codes = [0, 8, 9, 7, 10, 6, 11] + [8] * 25
    out[Q4_0].append((x, np.array(_half(-1.0) + _pack_nibbles(codes), dtype=np.uint8)))
    # q5_0: max -16 -> d = 1; q = (int8)(x + 16.5), at most 31
    x = _block([-16.0], ties + [14.5, 15.5, -15.5])
    codes = [0, 17, 16, 18, 15, 19, 14, 31, 31, 1] + [16] * 22
    out[Q5_0] = [(x, np.array(_half(1.0) + _qh(codes) + _pack_nibbles(codes), dtype=np.uint8))]
    # q4_1: min 0, max 15 -> d = 1, m = 0; q = (int8)(x + 0.5): 0.5 -> 1, 1.5 -> 2, 2.5 -> 3, 14.5 -> 15
    x = _block([0.0, 15.0], [0.5, 1.5, 2.5, 13.5, 14.5, 7.25])
    codes = [0, 15, 1, 2, 3, 14, 15, 7] + [0] * 24
    out[Q4_1] = [(x, np.array(_half(1.0) + _half(0.0) + _pack_nibbles(codes), dtype=np.uint8))]
    # min -4, max 11 -> d = 1, m = -4: x - min = -3.5 + 4 = 0.5 -> 1, -2.5 -> 2, 10.5 -> 15
    x = _block([-4.0, 11.0], [-3.5, -2.5, 10.5, 0.5])
    codes = [0, 15, 1, 2, 15, 5] + [4] * 26
    out[Q4_1].append((x, np.array(_half(1.0) + _half(-4.0) + _pack_nibbles(codes), dtype=np.uint8)))
    # q5_1: min 0, max 31 -> d = 1; 0.5 -> 1, 1.5 -> 2, 2.5 -> 3, 29.5 -> 30, 30.5 -> 31
    x = _block([0.0, 31.0], [0.5, 1.5, 2.5, 29.5, 30.5, 16.5])
    codes = [0, 31, 1, 2, 3, 30, 31, 17] + [0] * 24
    out[Q5_1] = [(x, np.array(_half(1.0) + _half(0.0) + _qh(codes) + _pack_nibbles(codes), dtype=np.uint8))]
    return out


def tie_q8_0_cpu_case():
    """The x86 CPU q8_0 variant (id = 127/amax, round half to even) on the q8_0 tie block:
    +-0.5 -> 0, +-1.5 -> +-2, +-2.5 -> +-2, 126.5 -> 126."""
    x = tie_cases()[Q8_0][0][0]
    codes = [127, 0, 0, 2, -2, 2, -2, 126, -126, 3] + [0] * 22
    return x, np.array(_half(1.0) + list(np.array(codes, dtype=np.int8).view(np.uint8)), dtype=np.uint8)
