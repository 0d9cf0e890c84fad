"""Constructed KV260 transactions whose output words follow from a few float32 operations.

Each case feeds the datapath inputs built so that one composition step of the board's arithmetic
decides an output word, an ``l`` word or an ``m`` word, and so that the plausible alternative of
that step gives a different word:

* ``p_truncation`` -- the PV operand is the upper half of the fp32 P word
  (hw/rtl/attn_top.sv:653-658), not P rounded to nearest even;
* ``sum_order`` -- a sub-block's PV products are summed key 0 first (sequential fp32 adds,
  hw/rtl/attn_top.sv:462-625), not key 15 first or pairwise;
* ``subblock_delta`` -- O is updated once per 16-key sub-block with the sub-block's own sum
  (hw/rtl/mem/output_buffer.sv:873-885), not key by key in one running sum;
* ``subblock_rescale`` -- the running max and the correction are taken per 16-key sub-block
  (hw/rtl/core/softmax_engine.sv:858-1073), not per 64-key tile; the row sum adds key 0 first;
* ``reciprocal_normalise`` -- O is multiplied by the reciprocal table's R(l)
  (hw/rtl/mem/output_buffer.sv:271-286), not divided by l;
* ``qk_order`` -- Q.K is summed dimension 0 first (hw/rtl/core/attn_tile.sv:176-248);
* ``exp_fraction`` -- the exp table's interpolation fraction r / 2^26 becomes fp32 with its
  significand truncated to 24 bits (``q26_to_fp32``, hw/rtl/core/softmax_engine.sv:547-566, used at
  :690-695), not rounded to nearest.

The expected words are derived here from IEEE float32 arithmetic (numpy scalars: the board's
adds and multiplies round like IEEE on the normal operands used), the exp and reciprocal ROM
lookups (pinned on their own at their knots, index boundaries and powers of two), and a
round-to-nearest-even bf16 conversion written from its definition.  Every value that the
derivation feeds through one of these operations is named, so each expected word can be followed
by hand; ``alternatives`` holds the word the competing composition would give, which each case
asserts is different.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import rtl_exact as rtl

F = np.float32
D = 128
H_Q, H_KV = 4, 1
SCALE = F(1.0 / np.sqrt(128.0))  # the transaction's default score scale at head_dim 128


def bits(x) -> int:
    return int(np.asarray(x, dtype=np.float32).view(np.uint32))


def from_bits(u: int) -> np.float32:
    return np.asarray(np.uint32(u)).view(np.float32)[()]


def word(x: float) -> int:
    """bf16 word of a value that bf16 holds exactly."""
    u = bits(F(x))
    assert u & 0xFFFF == 0, f"{x} is not a bf16 value"
    return u >> 16


def rne_word(x) -> int:
    """bf16 word nearest to the float32 value x, ties to the even word (from the definition:
    8 significant bits, the nearer of the two neighbours)."""
    x = float(F(x))
    if x == 0.0:
        return 0x8000 if np.signbit(x) else 0
    e = int(np.floor(np.log2(abs(x))))
    q = 2.0 ** (e - 7)  # bf16 spacing in x's binade
    r = np.round(x / q)  # numpy rounds halves to even
    return word(r * q)


def exp_rom(x) -> np.float32:
    """The exp table lookup of hw/rtl/core/softmax_engine.sv:570-706 (pinned on its own)."""
    return from_bits(int(rtl.exp_lookup(np.array([bits(F(x))], np.uint32))[0]))


def exp_by_hand(x, round_fraction: bool = False) -> np.float32:
    """E(x) for -8 <= x <= 0 (x a float32 with x < 0 in the interior of a table interval), derived
    step by step from hw/rtl/core/softmax_engine.sv:523-566,646-695:

    * xq = fp32_to_q8_23(x): the magnitude's 24-bit significand shifted to 2^-23 units, truncated,
      then negated: -floor(|x| 2^23);
    * n = xq + 2^26 (x + 8 in units of 2^-23); num = 1023 n; i = num >> 26 (the table interval) and
      r = num - i 2^26, the position inside it in units of 2^-26;
    * f = q26_to_fp32(r): r's leading one at bit b gives exponent b - 26 and the next 23 bits of r as
      the mantissa -- bits below bit b - 23 are dropped, i.e. the significand is truncated (with
      round_fraction: r / 2^26 rounded to nearest, the alternative the RTL does not take);
    * E = lut[i] + (lut[i+1] - lut[i]) f in fp32 (IEEE on these normal operands).
    """
    x = float(F(x))
    assert -8.0 <= x < 0.0
    xq = -int(np.floor(abs(x) * 2.0 ** 23))
    n = xq + (1 << 26)
    num = n * 1023
    i = num >> 26
    r = num - (i << 26)
    assert 0 <= i < 1023
    if round_fraction:
        f = F(r / 2.0 ** 26)
    else:
        b = r.bit_length() - 1
        kept = r if b <= 23 else (r >> (b - 23)) << (b - 23)
        f = F(kept / 2.0 ** 26)  # exact: at most 24 significant bits
    lut = rtl.exp_lut()
    lo, hi = from_bits(int(lut[i])), from_bits(int(lut[i + 1]))
    return F(lo + F(F(hi - lo) * f))


def recip_rom(l) -> np.float32:
    """R(l), the reciprocal table lookup of hw/rtl/mem/output_buffer.sv:271-286 (pinned on its own)."""
    return from_bits(int(rtl.recip_lookup(np.array([bits(F(l))], np.uint32))[0]))


def upper_half(p) -> np.float32:
    """The PV operand: P with its low 16 bits dropped."""
    return from_bits(bits(p) & 0xFFFF0000)


@dataclass
class Case:
    name: str
    L: int
    q_row: dict[int, float]          # dims of every query row (all rows and heads alike)
    k_rows: dict[int, dict[int, float]]  # key -> dims of its K row; other keys and dims are 0
    v_rows: dict[int, dict[int, float]]  # key -> dims of its V row
    out_words: dict[int, int]        # dim -> expected output word of every row; other dims 0
    m_bits: int
    l_bits: int
    alternatives: dict[str, tuple[str, int]] = field(default_factory=dict)  # plant -> (what, its word)
    catches: tuple[str, ...] = ()    # planted oracle mistakes this case must reject

    def tensors(self):
        q = np.zeros((H_Q, self.L, D), np.uint16)
        k = np.zeros((H_KV, self.L, D), np.uint16)
        v = np.zeros((H_KV, self.L, D), np.uint16)
        for d, x in self.q_row.items():
            q[:, :, d] = word(x)
        for key, row in self.k_rows.items():
            for d, x in row.items():
                k[:, key, d] = word(x)
        for key, row in self.v_rows.items():
            for d, x in row.items():
                v[:, key, d] = word(x)
        return q, k, v

    def expected_out(self) -> np.ndarray:
        out = np.zeros((H_Q, self.L, D), np.uint16)
        for d, w in self.out_words.items():
            out[:, :, d] = w
        return out


def _check_alternatives(case: Case) -> Case:
    expected = {"out": case.out_words, "m": case.m_bits, "l": case.l_bits}
    for plant, (what, alt) in case.alternatives.items():
        kind, _, dim = what.partition(":")
        want = expected[kind][int(dim)] if dim else expected[kind]
        assert alt != want, f"{case.name}: the {plant} alternative gives the same {what} word"
    return case


def p_truncation() -> Case:
    """Two keys; key 0 scores 0 (the max), key 1 scores s1 < 0, so p0 = 1 and p1 = exp(s1)."""
    b = -1.0390625  # bf16 0xBF85; q = e0, k1 = b e0
    s1 = F(F(b) * SCALE)
    p1 = exp_rom(F(s1 - F(0)))
    l = F(F(1) + p1)
    r = recip_rom(l)
    d1 = rne_word(F(upper_half(p1) * r))
    p1_rne = from_bits(rne_word(p1) << 16)
    return _check_alternatives(Case(
        "p_truncation", 2, {0: 1.0}, {1: {0: b}}, {0: {0: 1.0}, 1: {1: 1.0}},
        out_words={0: rne_word(F(F(1) * r)), 1: d1}, m_bits=0, l_bits=bits(l),
        alternatives={"p_rne": ("out:1", rne_word(F(p1_rne * r)))}, catches=("p_rne",)))


def sum_order() -> Case:
    """Q = 0: four keys with p = 1, l = 4, R(4) = 1/4 exactly.  Dim 0 holds V = (4, 2^-6, 2^-22,
    2^-22): key 0 first, each 2^-22 is half an ulp of 4 + 2^-6 and ties to it; key 3 first, the two
    make 2^-21, one ulp, and the quarter lands above the bf16 midpoint 1 + 2^-8.  Dim 1 holds the
    same values in reverse key order."""
    vals = [4.0, 2.0 ** -6, 2.0 ** -22, 2.0 ** -22]
    fwd = lambda xs: F(F(F(F(0) + F(xs[0])) + F(xs[1])) + F(xs[2])) + F(xs[3])
    l = F(4)
    r = recip_rom(l)
    assert r == F(0.25)
    d0 = rne_word(F(F(fwd(vals)) * r))
    d1 = rne_word(F(F(fwd(vals[::-1])) * r))
    rev0 = rne_word(F(F(fwd(vals[::-1])) * r))  # what dim 0 would give summed key 3 first
    pair0 = rne_word(F(F(F(vals[0]) + F(vals[1])) + F(F(vals[2]) + F(vals[3]))) * r)
    assert (d0, d1) == (0x3F80, 0x3F81) and pair0 == 0x3F81
    return _check_alternatives(Case(
        "sum_order", 4, {}, {}, {key: {0: vals[key], 1: vals[3 - key]} for key in range(4)},
        out_words={0: d0, 1: d1}, m_bits=0, l_bits=bits(l),
        alternatives={"sum_reversed": ("out:0", rev0), "pairwise": ("out:0", pair0)}, catches=("sum_reversed",)))


def subblock_delta() -> Case:
    """Q = 0: 32 keys with p = 1 in two sub-blocks, l = 32, R(32) = 2^-5.  Dim 0: key 0 = 32,
    key 1 = 2^-3 (sub-block 0), keys 16 and 17 = 2^-19 (sub-block 1).  Summed inside sub-block 1
    first, the two halves of an ulp of 32.125 make a whole one; added key by key to the running O,
    each ties back to 32.125."""
    o0 = F(F(32) + F(2.0 ** -3))
    corr = exp_rom(F(F(0) - F(0)))
    assert corr == F(1)
    delta1 = F(F(2.0 ** -19) + F(2.0 ** -19))
    o1 = F(F(o0 * corr) + delta1)
    l = F(F(F(16) * corr) + F(16))
    r = recip_rom(l)
    assert r == F(2.0 ** -5)
    flat = F(F(F(o0 * corr) + F(2.0 ** -19)) + F(2.0 ** -19))
    return _check_alternatives(Case(
        "subblock_delta", 32, {}, {}, {0: {0: 32.0}, 1: {0: 2.0 ** -3}, 16: {0: 2.0 ** -19}, 17: {0: 2.0 ** -19}},
        out_words={0: rne_word(F(o1 * r))}, m_bits=0, l_bits=bits(l),
        alternatives={"flat_accumulate": ("out:0", rne_word(F(flat * r)))}, catches=("flat_accumulate",)))


def subblock_rescale() -> Case:
    """32 keys; q = e0, key 16's K = 3 e0 scores s = 3 * scale > 0, every other key scores 0.
    Per sub-block: sub-block 0 runs at max 0 (p = 1, O = V), sub-block 1 raises the max to s and
    rescales O and l by E = exp(-s) at full fp32 precision.  Per 64-key tile, key 0 would enter PV
    as the truncated upper half of E instead.  Dim 0 carries key 0's V = 1, dim 1 key 16's V = 1."""
    s = F(F(3.0) * SCALE)
    e = exp_rom(F(F(0) - s))
    one = exp_rom(F(s - s))
    assert one == F(1)
    row_sum0 = F(0)
    for _ in range(16):
        row_sum0 = F(row_sum0 + F(1))
    row_sum1 = one  # key 16 first, then keys 17..31 at E
    for _ in range(15):
        row_sum1 = F(row_sum1 + e)
    l = F(F(row_sum0 * e) + row_sum1)
    r = recip_rom(l)
    o_d0 = F(F(F(1) * e) + F(0))
    o_d1 = F(F(F(0) * e) + F(upper_half(one) * F(1)))
    # the alternatives: one max per tile (key 0 at the upper half of E), and the row sum of
    # sub-block 1 taken from key 31 down
    tile_sum0 = F(0)
    for _ in range(16):
        tile_sum0 = F(tile_sum0 + e)
    l_tile = F(F(tile_sum0 * F(1)) + row_sum1)
    tile_d0 = rne_word(F(upper_half(e) * recip_rom(l_tile)))
    rev_sum1 = F(0)
    for _ in range(15):
        rev_sum1 = F(rev_sum1 + e)
    rev_sum1 = F(rev_sum1 + one)
    l_rev = F(F(row_sum0 * e) + rev_sum1)
    return _check_alternatives(Case(
        "subblock_rescale", 32, {0: 1.0}, {16: {0: 3.0}}, {0: {0: 1.0}, 16: {1: 1.0}},
        out_words={0: rne_word(F(o_d0 * r)), 1: rne_word(F(o_d1 * r))}, m_bits=bits(s), l_bits=bits(l),
        alternatives={"tile_rescale": ("out:0", tile_d0), "sum_reversed": ("l", bits(l_rev))},
        catches=("tile_rescale", "sum_reversed")))


def reciprocal_normalise() -> Case:
    """Q = 0: three keys with p = 1, l = 3; dim 0 holds V = (1, 1, 1.015625), O = 3.015625.
    R(3) = 0.332899... (the table's 8-bit-indexed reciprocal) puts O x R(3) below the bf16
    midpoint that O / 3 lies above."""
    o = F(F(F(F(0) + F(1)) + F(1)) + F(1.015625))
    l = F(F(F(1) + F(1)) + F(1))
    r = recip_rom(l)
    return _check_alternatives(Case(
        "reciprocal_normalise", 3, {}, {}, {0: {0: 1.0}, 1: {0: 1.0}, 2: {0: 1.015625}},
        out_words={0: rne_word(F(o * r))}, m_bits=0, l_bits=bits(l),
        alternatives={"exact_divide": ("out:0", rne_word(F(o / l)))}, catches=("exact_divide",)))


def qk_order() -> Case:
    """Two keys; q = (1, 1, 1, 0, ...), key 1's K = (4, 2^-22, 2^-22, 0, ...).  Dimension 0 first,
    each 2^-22 is half an ulp of 4 and ties back to 4; the other way round they make one ulp
    first.  m is key 1's scaled score; key 0 (K = 0) scores 0."""
    acc = F(F(F(F(0) + F(4)) + F(2.0 ** -22)) + F(2.0 ** -22))
    s1 = F(acc * SCALE)
    acc_rev = F(F(F(F(0) + F(2.0 ** -22)) + F(2.0 ** -22)) + F(4))
    p0 = exp_rom(F(F(0) - s1))
    p1 = exp_rom(F(s1 - s1))
    l = F(F(F(0) + p0) + p1)
    r = recip_rom(l)
    return _check_alternatives(Case(
        "qk_order", 2, {0: 1.0, 1: 1.0, 2: 1.0}, {1: {0: 4.0, 1: 2.0 ** -22, 2: 2.0 ** -22}},
        {0: {0: 1.0}, 1: {1: 1.0}},
        out_words={0: rne_word(F(upper_half(p0) * r)), 1: rne_word(F(upper_half(p1) * r))},
        m_bits=bits(s1), l_bits=bits(l),
        alternatives={"qk_reversed": ("m", bits(F(acc_rev * SCALE)))}, catches=("qk_reversed",)))


def exp_fraction() -> Case:
    """Two keys; q = (1, 1, 1, 0, ...).  Key 0's K = 2^-5 e0 scores t = 2^-5 x scale > 0, the max, so
    p0 = E(0) = 1.  Key 1's K = (-19.375, -0.07568359375, -0.0001659393310546875), bf16 parts that sum
    dimension 0 first to S1 = -19.4508495... exactly, scores s1 = S1 x scale, and its exp argument is
    x = s1 - t = -1.72199 (0xBFDC6A2F).  There the interpolation fraction is r / 2^26 with r >= 2^24,
    whose 24-bit significand loses r's lowest bits: truncated (the RTL) E(x) = 0x3E36FFFF, rounded to
    nearest 0x3E370000, whose upper half -- the PV operand -- is one bf16 step higher (l = 1 + p1 is
    the same word either way).  Dim 1 carries key 1's V = 1.0078125, and output word 1,
    upper(p1) x 1.0078125 x R(l), is 0x3E1C against 0x3E1D."""
    k1 = [from_bits(w << 16) for w in (0xC19B, 0xBD9B, 0xB92E)]
    S0 = F(F(F(0) + F(2.0 ** -5)) + F(0))
    S1 = F(F(F(F(0) + k1[0]) + k1[1]) + k1[2])
    t = F(S0 * SCALE)
    s1 = F(S1 * SCALE)
    x = F(s1 - t)
    assert bits(x) == 0xBFDC6A2F
    p0 = exp_rom(F(t - t))
    assert p0 == F(1)
    p1 = exp_by_hand(x)
    p1_rne = exp_by_hand(x, round_fraction=True)
    assert bits(p1) == 0x3E36FFFF and bits(p1_rne) == 0x3E370000
    l = F(F(F(0) + p0) + p1)
    r = recip_rom(l)
    l_rne = F(F(F(0) + p0) + p1_rne)
    return _check_alternatives(Case(
        "exp_fraction", 2, {0: 1.0, 1: 1.0, 2: 1.0}, {0: {0: 2.0 ** -5}, 1: {0: float(k1[0]), 1: float(k1[1]),
                                                                               2: float(k1[2])}},
        {0: {0: 1.0}, 1: {1: 1.0078125}},
        out_words={0: rne_word(F(upper_half(p0) * r)), 1: rne_word(F(F(upper_half(p1) * F(1.0078125)) * r))},
        m_bits=bits(t), l_bits=bits(l),
        alternatives={"frac_rne": ("out:1", rne_word(F(F(upper_half(p1_rne) * F(1.0078125)) * recip_rom(l_rne))))},
        catches=("frac_rne",)))


def all_cases() -> list[Case]:
    return [p_truncation(), sum_order(), subblock_delta(), subblock_rescale(), reciprocal_normalise(), qk_order(),
            exp_fraction()]
