"""Pins the layer-input oracle (oracle/layer_oracle.py) on the CPU.

* theta: equal to the ROM image hw/data/rope_theta.hex (SHA-256 always; the file itself
  where the reference tree is present).
* RoPE: within fp32 rounding of a float64 complex rotation; position 0 is the identity;
  pair norms are kept; rotating by p1 then p2 matches p1 + p2; a half-split pairing (the
  other common RoPE layout) and a flipped sine sign both fail the complex check.
* RMSNorm: a constant row gives sign(c) * gamma * |c| / sqrt(c^2 + eps); with eps = 0 the
  result is invariant to scaling x by a power of two; the row RMS of y / gamma is 1.
* Projection bound: the float64 product rounded to bf16 satisfies it; a transposed weight
  does not.
"""
import hashlib
from pathlib import Path

import numpy as np
import pytest

from oracle import gqa_oracle as orc
from oracle import layer_oracle as lo

REF_THETA = Path("/root/reference/hw/data/rope_theta.hex")


def test_theta_equals_the_rom_image():
    text = lo.rope_theta_hex(128).encode()
    assert hashlib.sha256(text).hexdigest() == lo.ROPE_THETA_SHA256
    if REF_THETA.is_file():
        assert REF_THETA.read_bytes() == text
    th = lo.rope_theta(128)
    assert th[0] == 1.0 and np.all(np.diff(th) < 0)
    assert lo.rope_theta(64)[1] == np.float32(10000.0 ** (-2 / 64))


def _heads(rng, H, L, D, scale=1.0):
    return orc.fp32_to_bf16_u16((rng.standard_normal((H, L, D)) * scale).astype(np.float32))


def test_rope_matches_complex_rotation_within_fp32_rounding():
    rng = np.random.default_rng(0)
    h = _heads(rng, 4, 64, 128, 3.0)
    for base in (0, 7, 511, 65000):
        got = orc.bf16_u16_to_fp32(lo.apply_rope(h, base)).astype(np.float64)
        want = lo.rope_complex_exact(h, base)
        x = np.abs(orc.bf16_u16_to_fp32(h).astype(np.float64))
        pair = np.repeat(np.hypot(x[..., 0::2], x[..., 1::2]), 2, axis=-1)
        # bf16 rounding of the result plus a few fp32 roundings of the pair's magnitude
        assert np.all(np.abs(got - want) <= orc.bf16_ulp(want) * 0.5 + pair * 2.0 ** -21)


def test_rope_position_zero_is_identity_and_norms_are_kept():
    rng = np.random.default_rng(1)
    h = _heads(rng, 2, 1, 128)
    assert np.array_equal(lo.apply_rope(h, 0), h)
    h = _heads(rng, 2, 40, 128)
    r = orc.bf16_u16_to_fp32(lo.apply_rope(h, 100)).astype(np.float64)
    x = orc.bf16_u16_to_fp32(h).astype(np.float64)
    n0 = np.hypot(x[..., 0::2], x[..., 1::2])
    n1 = np.hypot(r[..., 0::2], r[..., 1::2])
    assert np.all(np.abs(n1 - n0) <= n0 * 2.0 ** -7 + 1e-30)


def test_rope_composition():
    rng = np.random.default_rng(2)
    h = _heads(rng, 1, 1, 128)
    once = lo.rope_complex_exact(lo.apply_rope(h, 0), 300)
    # rotating the exact result of position 100 by 200 in float64 equals position 300
    x = orc.bf16_u16_to_fp32(h).astype(np.float64)
    th = lo.rope_theta(128).astype(np.float64)
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(1j * np.float32(100) * th) * np.exp(1j * np.float32(200) * th)
    two = np.empty_like(x)
    two[..., 0::2], two[..., 1::2] = z.real, z.imag
    # phases are fp32 products, so 100*theta + 200*theta differs from 300*theta by ~2^-24 relative
    assert np.allclose(once, two, atol=1e-4 * np.abs(x).max())


def test_rope_planted_mistakes_fail_the_complex_check():
    rng = np.random.default_rng(3)
    h = _heads(rng, 2, 16, 128)
    want = lo.rope_complex_exact(h, 9)
    tol = orc.bf16_ulp(want) * 0.5 + 2.0 ** -21 * np.abs(want).max()
    # half-split pairing (d, d + D/2) instead of (2p, 2p + 1)
    x = orc.bf16_u16_to_fp32(h).astype(np.float64)
    th = lo.rope_theta(128).astype(np.float64)
    ph = np.float32(9 + np.arange(16))[:, None].astype(np.float64) * th[None, :]
    a, b = x[..., :64], x[..., 64:]
    half = np.concatenate([a * np.cos(ph) - b * np.sin(ph), a * np.sin(ph) + b * np.cos(ph)], axis=-1)
    assert np.any(np.abs(half - want) > tol)
    # sine sign flipped (rotation the other way)
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(-1j * ph)
    flip = np.empty_like(x)
    flip[..., 0::2], flip[..., 1::2] = z.real, z.imag
    assert np.any(np.abs(flip - want) > tol)


def test_rms_norm_closed_forms():
    eps = 1e-5
    c = -0.75
    x = orc.fp32_to_bf16_u16(np.full((3, 256), c, np.float32))
    g = orc.fp32_to_bf16_u16(np.linspace(-2, 2, 256).astype(np.float32))
    y = lo.rms_norm_exact(x, g, eps)
    gf = orc.bf16_u16_to_fp32(g).astype(np.float64)
    assert np.allclose(y, np.sign(c) * gf * abs(c) / np.sqrt(c * c + eps), rtol=1e-15, atol=0)
    rng = np.random.default_rng(4)
    x = orc.fp32_to_bf16_u16(rng.standard_normal((5, 512)).astype(np.float32))
    ones = orc.fp32_to_bf16_u16(np.ones(512, np.float32))
    y0 = lo.rms_norm_exact(x, ones, 0.0)
    x8 = orc.fp32_to_bf16_u16(orc.bf16_u16_to_fp32(x) * np.float32(8))
    assert np.allclose(lo.rms_norm_exact(x8, ones, 0.0), y0, rtol=1e-15, atol=0)
    assert np.allclose(np.sqrt(np.mean(y0 * y0, axis=-1)), 1.0, rtol=1e-12)


def test_projection_bound_accepts_rounded_exact_and_rejects_a_transpose():
    rng = np.random.default_rng(5)
    x = orc.fp32_to_bf16_u16(rng.standard_normal((8, 64)).astype(np.float32))
    w = orc.fp32_to_bf16_u16(rng.standard_normal((64, 64)).astype(np.float32))
    exact = lo.project_exact(x, w)
    bound = lo.projection_error_bound(x, w)
    rounded = orc.bf16_u16_to_fp32(orc.bf16_rne(exact.astype(np.float32))).astype(np.float64)
    assert np.all(np.abs(rounded - exact) <= bound)
    wrong = orc.bf16_u16_to_fp32(x).astype(np.float64) @ orc.bf16_u16_to_fp32(w).astype(np.float64)
    assert np.any(np.abs(wrong - exact) > bound)


@pytest.mark.parametrize("H,L,D", [(3, 5, 128), (2, 7, 64)])
def test_reshape_to_heads(H, L, D):
    cols = np.arange(L * H * D).reshape(L, H * D)
    heads = lo.reshape_to_heads(cols, H, D)
    for h in range(H):
        assert np.array_equal(heads[h], cols[:, h * D:(h + 1) * D])
