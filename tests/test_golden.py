"""Golden fixtures (tests/golden, written by tests/golden/make_golden.py from torch's float64
scaled_dot_product_attention): the oracle on the CPU and the engine on the GPU.

The reference ships no golden vectors for this path (its golden model and board NPZ cases are
absent from the snapshot), so these fixtures come from an implementation independent of
the oracle.  Tolerance for the engine: every output row within 2 bf16 ulp of the row's
largest |expected|.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import gqa_oracle as orc

GOLDEN = sorted((Path(__file__).resolve().parent / "golden").glob("*.npz"))


def load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_fixtures_present():
    assert len(GOLDEN) >= 4


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_oracle_matches_golden(path):
    g = load(path)
    out, lse = orc.attention(orc.bf16_u16_to_fp32(g["q"]), orc.bf16_u16_to_fp32(g["k"]),
                             orc.bf16_u16_to_fp32(g["v"]), scale=float(g["scale"]), causal=bool(g["causal"]),
                             q_pos_base=int(g["q_pos_base"]), kv_pos_base=int(g["kv_pos_base"]))
    np.testing.assert_allclose(out, g["expected"], rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(lse, g["lse"], rtol=1e-12, atol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_engine_matches_golden(path):
    from lara_amd.attn_driver import AttentionAccelerator

    g = load(path)
    q, k, v = g["q"], g["k"], g["v"]
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    print(f"[golden] {path.stem}", flush=True)
    with AttentionAccelerator(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=lk, max_q_len=lq,
                              scale=float(g["scale"])) as acc:
        if lq == lk and hq == 32 and hkv == 8 and d == 128:
            out = acc.run_attention(q, k, v, q_pos_base=int(g["q_pos_base"]), kv_pos_base=int(g["kv_pos_base"]),
                                    causal=bool(g["causal"]))
        else:
            acc.load_kv(k, v)
            out = acc.decode_step(q[:, 0][None], np.array([lk], np.int32))[0][:, None]
    err = orc.row_ulp_error(out, g["expected"])
    assert float(err.max()) <= 2.0
