"""Word-level pins of how the KV260 restatement (oracle/rtl_exact.c) composes its primitives.

The constructed transactions of tests/_kv260_cases.py decide one output, m or l word each through
one composition step -- P truncation, the order of the sequential sums, the per-sub-block O update
and rescale, the reciprocal-table normalise, the Q.K order -- with the expected word derived from
IEEE float32 operations and the ROM lookups.  The restatement must give exactly those words, and
each mistake the C library can plant on purpose (PLANT_* flags) must be rejected by the case built
against it.
"""
import numpy as np
import pytest

from oracle import rtl_exact as rtl
from tests import _kv260_cases as kc

CASES = {c.name: c for c in kc.all_cases()}


def run(case, plant=0):
    q, k, v = case.tensors()
    return rtl.attention(q, k, v, causal=False, plant=plant)


@pytest.mark.parametrize("name", list(CASES))
def test_constructed_case_words(name):
    case = CASES[name]
    out, m, l = run(case)
    want = case.expected_out()
    bad = np.argwhere(out != want)
    assert bad.size == 0, (f"{name}: {len(bad)} words differ, first at {tuple(bad[0])}: "
                           f"0x{int(out[tuple(bad[0])]):04x} != 0x{int(want[tuple(bad[0])]):04x}")
    assert np.all(m == case.m_bits), f"{name}: m 0x{int(m.flat[0]):08x} != 0x{case.m_bits:08x}"
    assert np.all(l == case.l_bits), f"{name}: l 0x{int(l.flat[0]):08x} != 0x{case.l_bits:08x}"


@pytest.mark.parametrize("plant", list(rtl.PLANTS))
def test_planted_mistake_is_rejected(plant):
    """Every planted mistake changes at least one word of the case built against it."""
    catchers = [c for c in CASES.values() if plant in c.catches]
    assert catchers, f"no constructed case is built against {plant}"
    for case in catchers:
        out, m, l = run(case, rtl.PLANTS[plant])
        same = (np.array_equal(out, case.expected_out()) and np.all(m == case.m_bits)
                and np.all(l == case.l_bits))
        assert not same, f"{case.name} does not reject the planted {plant}"


def test_planted_p_rounding_moves_words_of_random_transactions():
    """P rounded to nearest even instead of truncated changes many words of an ordinary
    transaction while staying close to exact attention: only a word-level check catches it."""
    from oracle import gqa_oracle as orc

    rng = np.random.default_rng(6)
    L = 64
    q = orc.fp32_to_bf16_u16(rng.standard_normal((8, L, 128)).astype(np.float32) * 3)
    k = orc.fp32_to_bf16_u16(rng.standard_normal((2, L, 128)).astype(np.float32))
    v = orc.fp32_to_bf16_u16(rng.standard_normal((2, L, 128)).astype(np.float32))
    out, _, _ = rtl.attention(q, k, v, causal=False)
    planted, _, _ = rtl.attention(q, k, v, causal=False, plant=rtl.PLANT_P_RNE)
    exact, _ = orc.attention(orc.bf16_u16_to_fp32(q), orc.bf16_u16_to_fp32(k), orc.bf16_u16_to_fp32(v))
    assert (planted != out).mean() > 0.05
    assert float(orc.row_ulp_error(planted, exact).max()) <= 3.0


def test_rne_helper_from_its_definition():
    assert kc.rne_word(1.0 + 2.0 ** -8) == 0x3F80          # tie to the even word
    assert kc.rne_word(1.0 + 3 * 2.0 ** -8) == 0x3F82      # tie up to the even word
    assert kc.rne_word(1.0 + 2.0 ** -8 + 2.0 ** -20) == 0x3F81
    assert kc.rne_word(-3.0) == 0xC040 and kc.rne_word(0.0) == 0
