"""GPU KV260 RTL-exact mode against the C restatement of the board's arithmetic, word for word.

The engine's kv260 numerics (lara_amd/csrc/rtl_exact.hip) and the oracle (oracle/rtl_exact.c) are
independent implementations of the same bit-level contract; every output word must be equal.
"""
import numpy as np
import pytest

from lara_amd.attn_driver import AttentionAccelerator
from oracle import gqa_oracle as orc
from oracle import rtl_exact as rtl
from tests import _kv260_cases as kc
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu


def run_both(q, k, v, *, causal, qb, kb):
    hq, L, d = q.shape
    hkv = k.shape[0]
    print(f"[kv260] hq={hq} hkv={hkv} d={d} L={L} causal={causal} q_pos_base={qb} kv_pos_base={kb}", flush=True)
    with AttentionAccelerator(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=L, max_q_len=L,
                              numerics="kv260") as acc:
        out = acc.run_attention(q, k, v, q_pos_base=qb, kv_pos_base=kb, causal=causal)
    want, _, _ = rtl.attention(q, k, v, causal=causal, q_pos_base=qb, kv_pos_base=kb)
    return out, want


@pytest.mark.parametrize("L,causal,qb,kb", [(1, True, 0, 0), (16, True, 0, 0), (16, False, 0, 0), (33, True, 3, 3),
                                            (64, True, 31, 7), (100, False, 5, 9), (128, True, 0, 0),
                                            (130, True, 0, 64)])
def test_kv260_mode_bit_exact_board_shape(L, causal, qb, kb):
    rng = np.random.default_rng(2000 + L + qb + kb + causal)
    q = bf16_normal(rng, (32, L, 128))
    k = bf16_normal(rng, (8, L, 128))
    v = bf16_normal(rng, (8, L, 128))
    out, want = run_both(q, k, v, causal=causal, qb=qb, kb=kb)
    mism = np.argwhere(out != want)
    assert mism.size == 0, f"{len(mism)} mismatching words, first at {tuple(mism[0])}"


def test_kv260_mode_bit_exact_long_and_d64():
    rng = np.random.default_rng(2100)
    L = 512
    q = bf16_normal(rng, (8, L, 128))
    k = bf16_normal(rng, (2, L, 128), 2.0)
    v = bf16_normal(rng, (2, L, 128))
    out, want = run_both(q, k, v, causal=True, qb=0, kb=0)
    assert np.array_equal(out, want)
    q = bf16_normal(rng, (8, 96, 64))
    k = bf16_normal(rng, (2, 96, 64), 3.0)  # larger scores: many p fall below the table's -8
    v = bf16_normal(rng, (2, 96, 64))
    out, want = run_both(q, k, v, causal=False, qb=0, kb=0)
    assert np.array_equal(out, want)


@pytest.mark.parametrize("name", [c.name for c in kc.all_cases()])
def test_kv260_mode_constructed_composition_cases(name):
    """The engine's output words on the transactions built so that each composition step of the
    board's arithmetic decides a word, against the words derived by hand."""
    case = {c.name: c for c in kc.all_cases()}[name]
    q, k, v = case.tensors()
    out, _ = run_both(q, k, v, causal=False, qb=0, kb=0)
    bad = np.argwhere(out != case.expected_out())
    assert bad.size == 0, f"{name}: {len(bad)} words differ, first at {tuple(bad[0])}"


def test_kv260_mode_edges():
    rng = np.random.default_rng(2200)
    L = 40
    z = np.zeros((32, L, 128), np.uint16)
    out, want = run_both(z, z[:8], z[:8], causal=True, qb=0, kb=0)
    assert np.array_equal(out, want) and not out.any()
    # words with zero exponent (bf16 subnormals read as 0), signed zeros, huge and tiny values
    q = bf16_normal(rng, (32, L, 128))
    k = bf16_normal(rng, (8, L, 128))
    v = bf16_normal(rng, (8, L, 128))
    q[:, :, :8] = rng.choice(np.uint16([0x0001, 0x8001, 0x0000, 0x8000, 0x7F00, 0x0080]), size=(32, L, 8))
    v[:, :, 8:16] = rng.choice(np.uint16([0x0000, 0x8000, 0x0080, 0x8080, 0x7E00]), size=(8, L, 8))
    out, want = run_both(q, k, v, causal=True, qb=0, kb=0)
    assert np.array_equal(out, want)


def test_kv260_mode_close_to_exact_and_decode_refuses():
    rng = np.random.default_rng(2300)
    L = 64
    q = bf16_normal(rng, (32, L, 128))
    k = bf16_normal(rng, (8, L, 128))
    v = bf16_normal(rng, (8, L, 128))
    out, _ = run_both(q, k, v, causal=True, qb=0, kb=0)
    exact, _ = orc.attention(orc.bf16_u16_to_fp32(q), orc.bf16_u16_to_fp32(k), orc.bf16_u16_to_fp32(v), causal=True)
    assert float(orc.row_ulp_error(out, exact).max()) <= 3.0
    with AttentionAccelerator(max_seq_len=L, numerics="kv260") as acc:
        with pytest.raises(RuntimeError):
            acc.decode_step(q[:, 0][None], np.array([L], np.int32))


def test_board_functional_matrix_on_board_format_cases(tmp_path):
    """lara_amd.board_matrix over board-format case files: every word matches, and a planted
    one-word error in expected_o is reported as a failure."""
    from pathlib import Path

    from lara_amd import board_matrix

    cases = Path(__file__).resolve().parent / "golden" / "board_cases"
    assert board_matrix.main(["--cases", str(cases), "--output-dir", str(tmp_path / "ok")]) == 0
    bad = tmp_path / "bad_cases"
    bad.mkdir()
    src = sorted(cases.glob("case_*.npz"))[0]
    with np.load(src, allow_pickle=False) as d:
        files = {k: d[k] for k in d.files}
    files["expected_o"] = files["expected_o"].copy()
    files["expected_o"][3, 1, 7] ^= 1
    np.savez(bad / src.name, **files)
    assert board_matrix.main(["--cases", str(bad), "--output-dir", str(tmp_path / "bad")]) == 1
