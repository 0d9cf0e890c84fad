"""Seeded synthetic inputs shared by the tests (bf16 words drawn from N(0, 1) * amplitude)."""
from __future__ import annotations

import numpy as np

from oracle.gqa_oracle import fp32_to_bf16_u16


def bf16_normal(rng, shape, amplitude=1.0):
    return fp32_to_bf16_u16(rng.standard_normal(shape, dtype=np.float32) * np.float32(amplitude))


def kv_with_outliers(rng, shape, amplitude=1.0, fraction=0.0, factor=1.0):
    """K rows [..., L, D]; a seeded `fraction` of rows is scaled by `factor` before rounding."""
    x = rng.standard_normal(shape, dtype=np.float32) * np.float32(amplitude)
    if fraction > 0:
        rows = x.reshape(-1, shape[-1])
        n = max(1, int(round(fraction * rows.shape[0])))
        idx = rng.choice(rows.shape[0], size=n, replace=False)
        rows[idx] *= np.float32(factor)
    return fp32_to_bf16_u16(x)


def cancelling_kv(rng, hkv, n, d):
    """K/V words [hkv, n, d] in row pairs: row 2j+1 repeats row 2j's K but for dim 0 and negates its
    V, so the pair's softmax weights are close and their V contributions almost cancel (n even)."""
    k = fp32_to_bf16_u16(rng.standard_normal((hkv, n, d), dtype=np.float32))
    v = fp32_to_bf16_u16(rng.standard_normal((hkv, n, d), dtype=np.float32))
    k[:, 1::2] = k[:, 0::2]
    k[:, 1::2, 0] = fp32_to_bf16_u16(rng.standard_normal((hkv, n // 2), dtype=np.float32) * np.float32(0.05))
    v[:, 1::2] = v[:, 0::2] ^ np.uint16(0x8000)
    return k, v
