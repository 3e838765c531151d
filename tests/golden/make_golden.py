"""Writes the committed golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no tests, golden vectors or fixtures for its attention path, and ggml (where
the block formats and flash-attention arithmetic live) is not vendored, so these fixtures are
produced by this repository's oracle after it has been pinned by the closed-form/known-answer/
library checks in tests/test_oracle_*.py.  They freeze seeded inputs and the oracle's outputs so
the GPU tests (and later changes to the oracle) are checked against fixed data.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.oracle import F16, F32, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, QUANT_TYPES, oracle, row_bytes, view  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def block_fixture(orc):
    rng = np.random.default_rng(20261201)
    data = {}
    # 64 blocks: N(0,1), wide dynamic range, all-equal, zeros, single spikes, ties
    x = rng.standard_normal((64, 32)).astype(np.float32)
    x[8:16] *= np.float32(1e-3)
    x[16:24] *= np.float32(1e3)
    x[24] = 0.0
    x[25] = 1.5
    x[26] = 0.0
    x[26, 7] = -2.0
    x[27] = np.linspace(-1, 1, 32, dtype=np.float32)
    x[28] = np.round(x[28] * 4) / 4  # many ties
    x[29, :] = x[29, 0]
    x[29, 17] = -x[29, 0]  # equal magnitudes of both signs
    data["x"] = x
    for t in QUANT_TYPES:
        b = orc.quantize(t, x)
        data[f"bytes_{t}"] = b
        data[f"deq_{t}"] = np.stack([orc.dequantize(t, b[i], 32) for i in range(64)])
    np.savez_compressed(os.path.join(OUT, "blocks.npz"), **data)


def attn_decode_512_f16(orc):
    """Single-layer Qwen2-0.5B decode: 14/2 heads, D=64, f16 KV, n_kv=512, scale 1/8, no mask."""
    rng = np.random.default_rng(1)
    H, Hkv, D, nkv = 14, 2, 64, 512
    q = rng.standard_normal((H, D)).astype(np.float32)
    k = rng.standard_normal((nkv, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((nkv, Hkv, D)).astype(np.float32)
    kh = orc.f32_to_f16(k)
    vh = orc.f32_to_f16(v)
    row = Hkv * D * 2
    qt = view(q, F32, [D, 1, H, 1], [4, 4 * D * H, 4 * D, 4 * D * H])
    kt = view(kh, F16, [D, nkv, Hkv, 1], [2, row, row // Hkv, row * nkv])
    vt = view(vh, F16, [D, nkv, Hkv, 1], [2, row, row // Hkv, row * nkv])
    out = orc.fa_f64(qt, kt, vt, None, 0.125, (1, 1, H, D))
    np.savez_compressed(os.path.join(OUT, "attn_decode_512_f16.npz"), q=q, k_f16=kh, v_f16=vh, out=out.reshape(H, D))


def attn_prefill_small(orc):
    """Causal prefill chunk: 8 new tokens over 40 cached, K q8_0, V q4_0, 14/2 heads."""
    rng = np.random.default_rng(2)
    H, Hkv, D, nq, nkv = 14, 2, 64, 8, 40
    q = (0.5 * rng.standard_normal((nq, H, D))).astype(np.float32)
    k = (0.5 * rng.standard_normal((nkv, Hkv * D))).astype(np.float32)
    v = (0.5 * rng.standard_normal((nkv, Hkv * D))).astype(np.float32)
    kq = orc.quantize(Q8_0, k)
    vq = orc.quantize(Q4_0, v)
    mask = orc.causal_mask(nq, nkv)
    rk, rv = row_bytes(Q8_0, Hkv * D), row_bytes(Q4_0, Hkv * D)
    qt = view(q, F32, [D, nq, H, 1], [4, 4 * D * H, 4 * D, 4 * D * H * nq])
    kt = view(kq, Q8_0, [D, nkv, Hkv, 1], [34, rk, rk // Hkv, rk * nkv])
    vt = view(vq, Q4_0, [D, nkv, Hkv, 1], [18, rv, rv // Hkv, rv * nkv])
    mt = view(mask, F16, [nkv, nq, 1, 1], [2, 2 * nkv, 2 * nkv * nq, 2 * nkv * nq])
    out = orc.fa_f64(qt, kt, vt, mt, 0.125, (1, nq, H, D))
    np.savez_compressed(os.path.join(OUT, "attn_prefill_small.npz"), q=q, k_q8_0=kq, v_q4_0=vq, mask=mask, out=out)


def attn_dit_small(orc):
    """DiT bidirectional with the chunk-block mask: T=40, B=2, 16 heads, f32 q/k/v views.
    Inputs are fp16-representable (stored as float16 to keep the fixture small)."""
    rng = np.random.default_rng(3)
    T, B, H, D = 40, 2, 16, 64
    q = rng.standard_normal((B, T, H * D)).astype(np.float16).astype(np.float32)
    k = rng.standard_normal((B, T, H * D)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((B, T, H * D)).astype(np.float16).astype(np.float32)
    mask = orc.chunk_mask(T, [16, 32])
    row = 4 * H * D
    qt = view(q, F32, [D, T, H, B], [4, row, 4 * D, row * T])
    kt = view(k, F32, [D, T, H, B], [4, row, 4 * D, row * T])
    vt = view(v, F32, [D, T, H, B], [4, row, 4 * D, row * T])
    mt = view(mask, F16, [T, T, 1, 1], [2, 2 * T, 2 * T * T, 2 * T * T])
    out = orc.fa_f64(qt, kt, vt, mt, 0.125, (B, T, H, D))
    np.savez_compressed(os.path.join(OUT, "attn_dit_small.npz"), q=q.astype(np.float16), k=k.astype(np.float16),
                        v=v.astype(np.float16), mask=mask, out=out)


def main():
    orc = oracle()
    block_fixture(orc)
    attn_decode_512_f16(orc)
    attn_prefill_small(orc)
    attn_dit_small(orc)
    print("wrote fixtures to", OUT)


if __name__ == "__main__":
    main()
