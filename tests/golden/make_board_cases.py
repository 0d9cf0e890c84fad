"""Writes board-format functional cases (tests/golden/board_cases/case_*.npz).

The files use the reference's case format (sw/board_matrix.py:117-126: q_heads, k_heads,
v_heads as bf16 words, expected_o as bf16 words, seq_len, causal, q_pos_base, kv_pos_base).
The reference's case generator and its board-verified expected outputs are not in the
snapshot, so expected_o here is the output of oracle/rtl_exact.c -- the C restatement of the
deployed KV260 arithmetic -- on seeded N(0, 1) inputs; the engine's kv260 numerics must
reproduce it word for word.  Build the oracle first (make -C oracle), then run from the
repository root:  python tests/golden/make_board_cases.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import gqa_oracle as orc  # noqa: E402
from oracle import rtl_exact as rtl  # noqa: E402

OUT = Path(__file__).resolve().parent / "board_cases"
CASES = [  # (seq_len, causal, q_pos_base, kv_pos_base, seed)
    (4, True, 0, 0, 31),
    (6, False, 3, 3, 32),
    (5, True, 31, 7, 33),
]


def main() -> None:
    OUT.mkdir(exist_ok=True)
    for L, causal, qb, kb, seed in CASES:
        rng = np.random.default_rng(seed)
        q = orc.fp32_to_bf16_u16(rng.standard_normal((32, L, 128)).astype(np.float32))
        k = orc.fp32_to_bf16_u16(rng.standard_normal((8, L, 128)).astype(np.float32))
        v = orc.fp32_to_bf16_u16(rng.standard_normal((8, L, 128)).astype(np.float32))
        expected, _, _ = rtl.attention(q, k, v, causal=causal, q_pos_base=qb, kv_pos_base=kb)
        name = f"case_L{L}_q{qb}_kv{kb}_{'causal' if causal else 'noncausal'}.npz"
        np.savez_compressed(OUT / name, q_heads=q, k_heads=k, v_heads=v, expected_o=expected, seq_len=L,
                            causal=int(causal), q_pos_base=qb, kv_pos_base=kb)
        print(f"wrote {name}")


if __name__ == "__main__":
    main()
