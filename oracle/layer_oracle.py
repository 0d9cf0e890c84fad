"""CPU oracle for the layer input stage of run_layer (RMSNorm, QKV projection, RoPE).

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, as the parity reference.  The
product path (``lara_amd``) never imports it.

The reference's ``run_layer`` (sw/attn_driver.py:552-586) imports ``rms_norm``,
``qkv_project``, ``reshape_to_heads`` and ``apply_rope_host`` from a ``host_attention``
module that the snapshot does not ship, so these restate the contract the RTL headers
give, with the rounding points of this engine's specification:

* ``rms_norm_exact`` -- y = x / sqrt(mean(x^2) + eps) * gamma
  (hw/rtl/ext/rms_norm/rms_norm.sv:7-8), in float64, unrounded.
* ``project_exact`` -- Q = X Wq^T with W stored out x in
  (hw/rtl/ext/qkv_projection/qkv_projection.sv:7-8), float64 products of bf16 values.
* ``reshape_to_heads`` -- [L, H*D] -> [H, L, D], head h = columns h*D .. h*D + D - 1.
* ``rope_theta`` -- theta_p = 10000^(-2p/D), rounded once to fp32; for D = 128 this is the
  ROM image hw/data/rope_theta.hex word for word (SHA-256 below).
* ``apply_rope`` -- the rotation of hw/rtl/core/rope_engine.sv:135-155 restated op for op in
  IEEE fp32 (numpy float32 arithmetic, no fused multiply-add): phase = fp32(pos * theta_p);
  c, s = cos and sin of the fp32 phase evaluated in float64 and rounded to fp32;
  a' = fp32(fp32(a c) - fp32(b s)), b' = fp32(fp32(a s) + fp32(b c)); bf16 round to nearest
  even.  The GPU kernel performs the same operations, so on the same bf16 inputs the two
  agree word for word.

Pinning (``tests/test_layer_oracle.py``): theta against the ROM image's SHA-256 (and the
file itself where the reference tree is present); RoPE against a float64 complex-number
rotation, position 0 as the identity, norm preservation, rotation composition and a planted
mistake (half-split pairing); RMSNorm against constant-row and scale-invariance closed
forms.
"""
from __future__ import annotations

import numpy as np

from .gqa_oracle import bf16_rne, bf16_u16_to_fp32

ROPE_BASE = 10000.0
# SHA-256 of the ROM image hw/data/rope_theta.hex (64 words, one per line, trailing newline).
ROPE_THETA_SHA256 = "6f111a111d89af0d8a6993de33df2228d72fe8bf4021074b4ba00dd59ad54092"


def rope_theta(head_dim: int) -> np.ndarray:
    """theta_p = 10000^(-2p/D) for p < D/2, computed in float64 and rounded to fp32."""
    p = np.arange(head_dim // 2, dtype=np.float64)
    return np.power(ROPE_BASE, -2.0 * p / head_dim).astype(np.float32)


def rope_theta_hex(head_dim: int = 128) -> str:
    """The theta table in the ROM image format: one 8-digit lower-case hex word per line."""
    return "".join(f"{int(w):08x}\n" for w in rope_theta(head_dim).view(np.uint32))


def rms_norm_exact(x_words, gamma_words, eps: float) -> np.ndarray:
    """float64 y = x / sqrt(mean(x^2) + eps) * gamma per row of x [L, hidden] (bf16 words)."""
    x = bf16_u16_to_fp32(x_words).astype(np.float64)
    g = bf16_u16_to_fp32(gamma_words).astype(np.float64).reshape(-1)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * g


def project_exact(x_words, w_words) -> np.ndarray:
    """float64 X W^T for x [L, in] and w [out, in] (bf16 words): [L, out]."""
    x = bf16_u16_to_fp32(x_words).astype(np.float64)
    w = bf16_u16_to_fp32(w_words).astype(np.float64)
    return x @ w.T


def projection_error_bound(x_words, w_words) -> np.ndarray:
    """Bound on |fp32-accumulated bf16 GEMM rounded to bf16 - exact| per output element:
    one bf16 ulp of the exact value (a rounding that lands on either neighbour) plus
    2^-20 * sum_k |x_k w_k| for the fp32 accumulation in any order (k <= 2^12 terms)."""
    from .gqa_oracle import bf16_ulp
    x = np.abs(bf16_u16_to_fp32(x_words).astype(np.float64))
    w = np.abs(bf16_u16_to_fp32(w_words).astype(np.float64))
    exact = project_exact(x_words, w_words)
    return bf16_ulp(exact) + 2.0 ** -20 * (x @ w.T)


def reshape_to_heads(cols: np.ndarray, n_heads: int, head_dim: int) -> np.ndarray:
    """[L, H*D] -> [H, L, D]."""
    L = cols.shape[0]
    return np.ascontiguousarray(cols.reshape(L, n_heads, head_dim).transpose(1, 0, 2))


def apply_rope(heads_words, pos_base: int) -> np.ndarray:
    """RoPE of bf16 heads [H, L, D] at positions pos_base + t, fp32 op for op (see header)."""
    h = np.asarray(heads_words, dtype=np.uint16)
    H, L, D = h.shape
    theta = rope_theta(D)
    pos = (np.arange(L, dtype=np.int64) + int(pos_base)).astype(np.float32)
    phase = (pos[:, None] * theta[None, :]).astype(np.float32)           # [L, D/2], fp32 product
    c = np.cos(phase.astype(np.float64)).astype(np.float32)
    s = np.sin(phase.astype(np.float64)).astype(np.float32)
    x = bf16_u16_to_fp32(h)
    a, b = x[..., 0::2], x[..., 1::2]
    r0 = (a * c).astype(np.float32) - (b * s).astype(np.float32)
    r1 = (a * s).astype(np.float32) + (b * c).astype(np.float32)
    out = np.empty_like(h)
    out[..., 0::2] = bf16_rne(r0.astype(np.float32))
    out[..., 1::2] = bf16_rne(r1.astype(np.float32))
    return out


def rope_complex_exact(heads_words, pos_base: int) -> np.ndarray:
    """float64 reference rotation (a + i b) * exp(i * phase) with the same fp32 phase."""
    h = bf16_u16_to_fp32(np.asarray(heads_words, dtype=np.uint16)).astype(np.float64)
    H, L, D = h.shape
    theta = rope_theta(D)
    pos = (np.arange(L, dtype=np.int64) + int(pos_base)).astype(np.float32)
    phase = (pos[:, None] * theta[None, :]).astype(np.float32).astype(np.float64)
    z = (h[..., 0::2] + 1j * h[..., 1::2]) * np.exp(1j * phase)
    out = np.empty_like(h)
    out[..., 0::2] = z.real
    out[..., 1::2] = z.imag
    return out
