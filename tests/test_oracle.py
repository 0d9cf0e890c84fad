"""Pins the CPU oracle against independent references before the parity tests rely on it.

* bf16 packers: hand-derived words, the algebraic closed form of the reference packer
  over every low-half pattern, and torch's bfloat16 conversion (RNE) for bf16_rne.
* attention: torch float64 scaled-dot-product attention (an independent library
  routine), pure-Python brute force on tiny shapes, and known answers.
"""
import math

import numpy as np
import pytest
import torch

from oracle import gqa_oracle as orc
from tests._gen import cancelling_kv


def words_to_f32(words):
    return np.asarray(words, dtype=np.uint32).view(np.float32)


# ---------------------------------------------------------------------------------------
# packers
# ---------------------------------------------------------------------------------------

def test_pack_hand_derived_words():
    # 1 + 2^-8 + 2^-9: RNE would give 0x3F81; the reference packer keeps 0x3F80.
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F80C000: 0x3F80,  # round bit + sticky: truncated
        0x3F808000: 0x3F80,  # tie, even
        0x3F818000: 0x3F81,  # tie, odd: still truncated
        0x3F80FFFF: 0x3F81,  # low half all ones carries
        0x3F7FFFFF: 0x3F80,  # carry into the exponent
        0x80000000: 0x8000,  # -0.0
        0xC0490FDB: 0xC049,  # -pi
        0x7F800000: 0x7F80,  # +inf
    }
    src = words_to_f32(list(cases))
    got = orc.fp32_to_bf16_u16(src)
    assert [int(x) for x in got] == list(cases.values())


def test_pack_uint16_passthrough():
    w = np.array([0, 1, 0x7F80, 0xFFFF], dtype=np.uint16)
    out = orc.fp32_to_bf16_u16(w)
    assert out.dtype == np.uint16 and np.array_equal(out, w)


def test_pack_closed_form_every_low_half():
    # The reference expression equals: upper half, plus one iff the low half is 0xFFFF.
    low = np.arange(1 << 16, dtype=np.uint32)
    for upper in (0x0000, 0x3F80, 0x3F81, 0x4049, 0xC2F7, 0x7F7F, 0x0080):
        bits = (np.uint32(upper) << np.uint32(16)) | low
        got = orc.fp32_to_bf16_u16(bits.view(np.float32)).astype(np.uint32)
        expect = (np.uint32(upper) + (low == 0xFFFF)).astype(np.uint32) & np.uint32(0xFFFF)
        assert np.array_equal(got, expect), hex(upper)


def test_unpack_matches_torch():
    rng = np.random.default_rng(0)
    words = rng.integers(0, 1 << 16, 4096, dtype=np.uint16)
    words = words[(words & 0x7F80) != 0x7F80]  # finite only
    ref = torch.from_numpy(words.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    assert np.array_equal(orc.bf16_u16_to_fp32(words), ref)


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(100000).astype(np.float32) * 3.0
    # add exact ties (low half 0x8000) with both parities
    ties = (np.array([0x3F800000, 0x3F810000, 0xBF820000, 0x40490000], dtype=np.uint32) | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, np.float32([0.0, -0.0, 1e-30, 65504.0])])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.bf16_rne(x), ref)


def test_bf16_ulp_values():
    assert orc.bf16_ulp(1.0) == 2.0 ** -7
    assert orc.bf16_ulp(1.99) == 2.0 ** -7
    assert orc.bf16_ulp(2.0) == 2.0 ** -6
    assert orc.bf16_ulp(-0.3) == 2.0 ** -9


def test_row_ulp_error_detects_planted_error():
    rng = np.random.default_rng(2)
    ref = rng.standard_normal((4, 64))
    words = orc.bf16_rne(ref.astype(np.float32))
    assert np.all(orc.row_ulp_error(words, ref) <= 0.5 + 1e-9)
    bumped = words.copy()
    bumped[1, 3] += 3  # three bf16 ulps at that element (same binade)
    err = orc.row_ulp_error(bumped, ref)
    assert err[1] > 2.0 and np.all(err[[0, 2, 3]] <= 0.5 + 1e-9)


def _bf16_p_attention(q, k, v, scale):
    """Attention whose P.V product takes each weight rounded to bf16 (RNE) while l sums the exact
    weights: the product of a bf16-P matrix-core kernel, emulated in float64."""
    s = q @ k.T * scale
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    pb = orc.bf16_u16_to_fp32(orc.bf16_rne(p.astype(np.float32))).astype(np.float64)
    return (pb @ v) / p.sum(axis=-1, keepdims=True)


def test_weight_rounding_error_bounds_a_bf16_p_product():
    """A bf16-P product stays within 2 ulp + 2^-8 * attention(|V|) on inputs whose V rows cancel,
    although the 2-ulp measure alone rejects it there; on ordinary inputs both measures pass it; an
    element off by twice the allowed error is rejected."""
    rng = np.random.default_rng(3)
    d, n = 128, 64
    q = orc.bf16_u16_to_fp32(orc.bf16_rne(rng.standard_normal((8, d)).astype(np.float32))).astype(np.float64)
    kw, vw = cancelling_kv(rng, 1, n, d)
    k = orc.bf16_u16_to_fp32(kw[0]).astype(np.float64)
    v = orc.bf16_u16_to_fp32(vw[0]).astype(np.float64)
    scale = 1 / math.sqrt(d)
    ref, _ = orc.attention(q[:, None], k[None], v[None], scale=scale)
    ref_abs, _ = orc.attention(q[:, None], k[None], np.abs(v)[None], scale=scale)
    ref, ref_abs = ref[:, 0], ref_abs[:, 0]
    out = orc.bf16_rne(_bf16_p_attention(q, k, v, scale).astype(np.float32))
    assert float(orc.weight_rounding_error(out, ref, ref_abs).max()) <= 1.0
    assert float(orc.row_ulp_error(out, ref).max()) > 2.0  # the cancellation defeats the 2-ulp measure
    # ordinary inputs: V without cancelling pairs
    v2 = orc.bf16_u16_to_fp32(orc.bf16_rne(rng.standard_normal((n, d)).astype(np.float32))).astype(np.float64)
    ref2, _ = orc.attention(q[:, None], k[None], v2[None], scale=scale)
    abs2, _ = orc.attention(q[:, None], k[None], np.abs(v2)[None], scale=scale)
    out2 = orc.bf16_rne(_bf16_p_attention(q, k, v2, scale).astype(np.float32))
    assert float(orc.row_ulp_error(out2, ref2[:, 0]).max()) <= 2.0
    assert float(orc.weight_rounding_error(out2, ref2[:, 0], abs2[:, 0]).max()) <= 1.0
    # a planted error of twice the allowed amount at one element
    mag = np.max(np.abs(ref), axis=-1)
    allowed = 2 * orc.bf16_ulp(mag[2]) + 2.0 ** -8 * ref_abs[2, 5]
    planted = out.copy()
    planted[2, 5] = orc.bf16_rne(np.float32(ref[2, 5] + 2.2 * allowed))
    err = orc.weight_rounding_error(planted, ref, ref_abs)
    assert err[2, 5] > 1.0 and float(np.delete(err.ravel(), 2 * d + 5).max()) <= 1.0


# ---------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------

def _bf16_inputs(rng, hq, hkv, lq, lk, d, amp=1.0):
    q = orc.bf16_u16_to_fp32(orc.bf16_rne(rng.standard_normal((hq, lq, d)) * amp))
    k = orc.bf16_u16_to_fp32(orc.bf16_rne(rng.standard_normal((hkv, lk, d)) * amp))
    v = orc.bf16_u16_to_fp32(orc.bf16_rne(rng.standard_normal((hkv, lk, d)) * amp))
    return q, k, v


def _torch_sdpa(q, k, v, scale, mask):
    group = q.shape[0] // k.shape[0]
    kt = torch.from_numpy(k.astype(np.float64)).repeat_interleave(group, dim=0)
    vt = torch.from_numpy(v.astype(np.float64)).repeat_interleave(group, dim=0)
    qt = torch.from_numpy(q.astype(np.float64))
    m = None if mask is None else torch.from_numpy(mask)
    o = torch.nn.functional.scaled_dot_product_attention(qt[None], kt[None], vt[None], attn_mask=m, scale=scale)
    s = (qt @ kt.transpose(-1, -2)) * scale
    if m is not None:
        s = s.masked_fill(~m, float("-inf"))
    return o[0].numpy(), torch.logsumexp(s, dim=-1).numpy()


@pytest.mark.parametrize(
    "hq,hkv,lq,lk,d,causal,qb,kb",
    [
        (32, 8, 1, 257, 128, False, 0, 0),
        (8, 2, 16, 64, 64, True, 48, 0),
        (16, 2, 33, 33, 128, True, 0, 0),
        (4, 4, 5, 40, 32, True, 100, 70),
        (64, 8, 3, 100, 128, False, 0, 0),
    ],
)
def test_attention_matches_torch_sdpa(hq, hkv, lq, lk, d, causal, qb, kb):
    rng = np.random.default_rng(hq * 1000 + lk)
    q, k, v = _bf16_inputs(rng, hq, hkv, lq, lk, d)
    scale = float(np.float32(1.0 / math.sqrt(d)))
    mask = None
    if causal:
        mask = (kb + np.arange(lk))[None, :] <= (qb + np.arange(lq))[:, None]
    o, lse = orc.attention(q, k, v, causal=causal, q_pos_base=qb, kv_pos_base=kb)
    o_ref, lse_ref = _torch_sdpa(q, k, v, scale, mask)
    rows = np.ones(lq, bool) if mask is None else mask.any(axis=1)
    np.testing.assert_allclose(o[:, rows], o_ref[:, rows], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse[:, rows], lse_ref[:, rows], rtol=1e-12, atol=1e-12)
    assert np.all(o[:, ~rows] == 0) and np.all(np.isneginf(lse[:, ~rows]))


def test_attention_brute_force_tiny():
    rng = np.random.default_rng(3)
    hq, hkv, lq, lk, d = 4, 2, 3, 5, 4
    q, k, v = _bf16_inputs(rng, hq, hkv, lq, lk, d)
    qb, kb, scale = 2, 0, 0.37
    o, lse = orc.attention(q, k, v, scale=scale, causal=True, q_pos_base=qb, kv_pos_base=kb)
    sc = float(np.float32(scale))
    for h in range(hq):
        g = h // (hq // hkv)
        for i in range(lq):
            keys = [j for j in range(lk) if kb + j <= qb + i]
            s = [sc * sum(float(q[h, i, t]) * float(k[g, j, t]) for t in range(d)) for j in keys]
            mx = max(s)
            w = [math.exp(x - mx) for x in s]
            tot = sum(w)
            for t in range(d):
                ref = sum(wj * float(v[g, j, t]) for wj, j in zip(w, keys)) / tot
                assert abs(o[h, i, t] - ref) < 1e-12
            assert abs(lse[h, i] - (mx + math.log(tot))) < 1e-12


def test_known_answers():
    rng = np.random.default_rng(4)
    d = 64
    # zero inputs -> zero output (board smoke test semantics)
    z = np.zeros((8, 5, d))
    o, _ = orc.attention(z, np.zeros((2, 5, d)), np.zeros((2, 5, d)))
    assert np.all(o == 0)
    # one key -> that key's V row exactly
    q, k, v = _bf16_inputs(rng, 8, 2, 1, 1, d)
    o, _ = orc.attention(q, k, v)
    assert np.array_equal(o[:4, 0], np.repeat(v[0, :1], 4, axis=0)) and np.array_equal(o[4:, 0], np.repeat(v[1, :1], 4, axis=0))
    # identical keys -> mean of V
    q, k, v = _bf16_inputs(rng, 4, 1, 2, 37, d)
    k[:] = k[:, :1]
    o, _ = orc.attention(q, k, v)
    np.testing.assert_allclose(o[:, 0], np.repeat(v.astype(np.float64).mean(axis=1), 4, axis=0), rtol=1e-12, atol=1e-13)
    # one dominant score -> that V row
    q, k, v = _bf16_inputs(rng, 1, 1, 1, 50, d)
    k[0, 17] = q[0, 0] * 64.0
    o, _ = orc.attention(q, k, v)
    np.testing.assert_allclose(o[0, 0], v[0, 17], atol=1e-6)


def test_gqa_head_mapping_and_permutation():
    rng = np.random.default_rng(5)
    q, k, v = _bf16_inputs(rng, 8, 2, 3, 20, 32)
    o, _ = orc.attention(q, k, v)
    k2, v2 = k.copy(), v.copy()
    k2[1] += 0.5
    v2[1] *= -1.0
    o2, _ = orc.attention(q, k2, v2)
    assert np.array_equal(o[:4], o2[:4]) and not np.allclose(o[4:], o2[4:])
    perm = rng.permutation(20)
    o3, _ = orc.attention(q, k[:, perm], v[:, perm])
    np.testing.assert_allclose(o, o3, rtol=1e-12, atol=1e-13)


def test_fully_masked_rows_are_zero_and_strict_raises():
    rng = np.random.default_rng(6)
    q, k, v = _bf16_inputs(rng, 4, 2, 4, 4, 16)
    o, lse = orc.attention(q, k, v, causal=True, q_pos_base=0, kv_pos_base=2)
    assert np.all(o[:, :2] == 0) and np.all(np.isneginf(lse[:, :2]))
    assert np.all(np.isfinite(lse[:, 2:]))
    with pytest.raises(ValueError):
        orc.attention(q, k, v, causal=True, q_pos_base=0, kv_pos_base=2, strict_rows=True)


def test_decode_matches_attention():
    rng = np.random.default_rng(7)
    B, hq, hkv, d, lcap = 3, 8, 2, 64, 64
    qw = orc.bf16_rne(rng.standard_normal((B, hq, d)))
    kc = orc.bf16_rne(rng.standard_normal((B, hkv, lcap, d)))
    vc = orc.bf16_rne(rng.standard_normal((B, hkv, lcap, d)))
    lens = np.array([64, 0, 17])
    o, lse = orc.decode(qw, kc, vc, lens)
    for b in range(B):
        if lens[b] == 0:
            assert np.all(o[b] == 0) and np.all(np.isneginf(lse[b]))
            continue
        ob, lb = orc.attention(orc.bf16_u16_to_fp32(qw[b])[:, None], orc.bf16_u16_to_fp32(kc[b, :, :lens[b]]),
                               orc.bf16_u16_to_fp32(vc[b, :, :lens[b]]))
        assert np.array_equal(o[b], ob[:, 0]) and np.array_equal(lse[b], lb[:, 0])


def test_fp32_baseline_close_to_exact():
    rng = np.random.default_rng(8)
    qw = orc.bf16_rne(rng.standard_normal((32, 9, 128)))
    kw = orc.bf16_rne(rng.standard_normal((8, 9, 128)))
    vw = orc.bf16_rne(rng.standard_normal((8, 9, 128)))
    o32 = orc.cpu_attention_numpy_fp32(qw, kw, vw, causal=True, q_pos_base=0, kv_pos_base=0)
    o64, _ = orc.attention(orc.bf16_u16_to_fp32(qw), orc.bf16_u16_to_fp32(kw), orc.bf16_u16_to_fp32(vw), causal=True)
    np.testing.assert_allclose(o32, o64, rtol=1e-4, atol=1e-5)
    u = orc.decode_fp32_baseline(qw[:4, 8], kw[0], vw[0])
    np.testing.assert_allclose(u, o64[:4, 8], rtol=1e-4, atol=1e-5)
