"""Writes the golden fixtures of the GQA attention path (tests/golden/*.npz).

The expected outputs come from torch's float64 scaled_dot_product_attention on the CPU --
an implementation independent of oracle/gqa_oracle.py -- applied to bf16 inputs drawn from
N(0, 1) with fixed seeds.  Cases follow the reference's transaction contract
(sw/attn_driver.py:469-550: Q [32, L, 128], K/V [8, L, 128], head h reads kv head h // 4,
scale 1/sqrt(128), mask kv_pos <= q_pos with absolute position bases) and the board-shape
decode config (8 q / 2 kv heads, D 64, 256 keys, scale 1/8, no mask).

Each file holds: q, k, v (uint16 bf16 words), expected (float32 rounding of the float64 result), lse (float64, natural log),
scale, causal, q_pos_base, kv_pos_base.  Run from the repository root:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bf16_words(rng, shape):
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(torch.bfloat16)
    return x.view(torch.int16).numpy().view(np.uint16)


def words_to_f64(w):
    return torch.from_numpy((w.astype(np.uint32) << 16).view(np.float32)).to(torch.float64)


def sdpa(q, k, v, scale, causal, qb, kb):
    qf, kf, vf = words_to_f64(q), words_to_f64(k), words_to_f64(v)
    lq, lk = qf.shape[1], kf.shape[1]
    mask = None
    if causal:
        mask = (kb + torch.arange(lk))[None, :] <= (qb + torch.arange(lq))[:, None]
        assert bool(mask.any(dim=1).all()), "every query row needs a valid key"
    out = torch.nn.functional.scaled_dot_product_attention(qf[None], kf[None], vf[None], attn_mask=mask,
                                                           scale=scale, enable_gqa=True)[0]
    s = torch.matmul(qf.view(kf.shape[0], -1, lq, qf.shape[2]), kf[:, None].transpose(-1, -2)) * scale
    s = s.reshape(qf.shape[0], lq, lk)
    if mask is not None:
        s = torch.where(mask[None], s, torch.tensor(-math.inf, dtype=torch.float64))
    lse = torch.logsumexp(s, dim=-1)
    return out.numpy(), lse.numpy()


CASES = {
    # name: (seed, H_q, H_kv, D, Lq, Lk, causal, q_pos_base, kv_pos_base, scale)
    "board_l8_causal": (11, 32, 8, 128, 8, 8, True, 0, 0, None),
    "board_l5_q3kv3_causal": (12, 32, 8, 128, 5, 5, True, 3, 3, None),
    "board_l6_q31kv7_noncausal": (13, 32, 8, 128, 6, 6, False, 31, 7, None),
    "decode_c1_board_shape": (14, 8, 2, 64, 1, 256, False, 0, 0, 0.125),
}


def main():
    for name, (seed, hq, hkv, d, lq, lk, causal, qb, kb, scale) in CASES.items():
        rng = np.random.default_rng(seed)
        q = bf16_words(rng, (hq, lq, d))
        k = bf16_words(rng, (hkv, lk, d))
        v = bf16_words(rng, (hkv, lk, d))
        sc = float(np.float32(scale if scale is not None else 1.0 / math.sqrt(d)))
        out, lse = sdpa(q, k, v, sc, causal, qb, kb)
        np.savez_compressed(HERE / f"{name}.npz", q=q, k=k, v=v, expected=out.astype(np.float32), lse=lse, scale=sc, causal=causal,
                            q_pos_base=qb, kv_pos_base=kb)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
