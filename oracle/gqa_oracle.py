"""CPU oracle for the GQA streaming-attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the parity
reference or the timed CPU baseline.  The product path (``lara_amd``) never imports it and has no CPU
fallback.

What it restates (reference files, paths relative to the reference repository):

* ``fp32_to_bf16_u16`` / ``bf16_u16_to_fp32`` -- the host packing helpers of
  ``sw/attn_driver.py:88-103``, bit for bit.  Note the reference adds the round bit at
  bit 0 before masking the low half, so its packing rounds toward zero except when the
  low 16 bits are all ones; this restatement keeps that behaviour.
* ``bf16_rne`` -- the device-side output rounding ``fp32_to_bf16`` of
  ``hw/rtl/pkg/attn_pkg.sv:618-626`` (round to nearest even on the upper half).
* ``attention`` -- ``cpu_attention_numpy`` of ``sw/board_performance.py:158-192``
  generalised to any head counts, head_dim, scale, separate query/key lengths and absolute
  positions (mask: key valid iff kv_pos <= q_pos, ``hw/rtl/core/softmax_engine.sv:865-871``).
  A query row with no valid key yields zeros (``hw/rtl/mem/output_buffer.sv:276-277``),
  where ``cpu_attention_numpy`` raises; ``attention(strict_rows=True)`` raises instead.
* ``decode`` -- the same model for one query row per sequence over a resident cache
  ``[B][H_kv][L_cap][D]`` (the per-(b, h) layout of ``hw/rtl/mem/kv_cache_ram.sv:77-83``).

Pinning (``tests/test_oracle.py``): the packers against hand-derived words, torch's
bfloat16 conversion and exhaustive tables; ``attention`` against torch's float64
scaled-dot-product attention, brute-force loops on tiny shapes and the known answers
zero-in/zero-out, single key, constant keys, one-hot score, GQA head mapping, key
permutation invariance and fully masked rows.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

__all__ = [
    "fp32_to_bf16_u16",
    "bf16_u16_to_fp32",
    "bf16_rne",
    "bf16_ulp",
    "attention",
    "decode",
    "cpu_attention_numpy_fp32",
    "decode_fp32_baseline",
    "row_ulp_error",
    "weight_rounding_error",
]


# ---------------------------------------------------------------------------------------
# bf16 packing
# ---------------------------------------------------------------------------------------

def fp32_to_bf16_u16(values) -> np.ndarray:
    """Host packing of sw/attn_driver.py:88-98: uint16 input passes through unchanged."""
    arr = np.asarray(values)
    if arr.dtype == np.uint16:
        return np.ascontiguousarray(arr)
    bits = np.asarray(arr, dtype=np.float32).view(np.uint32).copy()
    low = bits & np.uint32(0xFFFF)
    odd = (bits >> np.uint32(16)) & np.uint32(1)
    half = (low >> np.uint32(15)) & np.uint32(1)
    sticky = (low & np.uint32(0x7FFF)) != 0
    increment = half & (odd | sticky.astype(np.uint32))
    packed = (bits + increment) & np.uint32(0xFFFF0000)
    return np.ascontiguousarray((packed >> np.uint32(16)).astype(np.uint16))


def bf16_u16_to_fp32(words) -> np.ndarray:
    """sw/attn_driver.py:101-103: a bf16 word is the upper half of an fp32."""
    w = np.asarray(words, dtype=np.uint16)
    return (w.astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_rne(values) -> np.ndarray:
    """fp32 -> bf16 words, round to nearest even (attn_pkg.sv:618-626)."""
    bits = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    upper = bits >> np.uint64(16)
    half = (bits >> np.uint64(15)) & np.uint64(1)
    sticky = (bits & np.uint64(0x7FFF)) != 0
    round_up = half & ((upper & np.uint64(1)) | sticky.astype(np.uint64))
    return ((upper + round_up) & np.uint64(0xFFFF)).astype(np.uint16)


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (8 significant bits); 2**-133 floor for zero."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    safe = np.where(a > 0, a, 2.0 ** -126)
    exp = np.floor(np.log2(safe))
    exp = np.maximum(exp, -126.0)
    return np.ldexp(1.0, (exp - 7).astype(np.int64))


# ---------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------

def attention(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    *,
    scale: Optional[float] = None,
    causal: bool = False,
    q_pos_base: int = 0,
    kv_pos_base: int = 0,
    dtype=np.float64,
    strict_rows: bool = False,
):
    """Exact GQA attention.  q [H_q, Lq, D], k/v [H_kv, Lk, D] real values.

    Returns (o [H_q, Lq, D], lse [H_q, Lq]) in ``dtype``; lse is the natural-log
    log-sum-exp of the scaled scores over valid keys (-inf for rows with none).
    Follows board_performance.py:158-192 (q head h reads kv head h // group).
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    hq, lq, d = q.shape
    hkv, lk, _ = k.shape
    if hq % hkv:
        raise ValueError("H_q must be a multiple of H_kv")
    group = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    scale = dtype(np.float32(scale))
    valid = None
    if causal:
        qp = q_pos_base + np.arange(lq)
        kp = kv_pos_base + np.arange(lk)
        valid = kp[None, :] <= qp[:, None]
        if strict_rows and not np.all(valid.any(axis=1)):
            raise ValueError("causal workload contains a query with no valid K/V position")
    out = np.zeros((hq, lq, d), dtype=dtype)
    lse = np.full((hq, lq), -np.inf, dtype=dtype)
    if lk == 0:
        return out, lse
    for g in range(hkv):
        qg = q[g * group:(g + 1) * group]                  # [group, Lq, D]
        s = np.matmul(qg, k[g].T) * scale                 # [group, Lq, Lk]
        if valid is not None:
            s = np.where(valid[None], s, -np.inf)
        m = np.max(s, axis=-1, keepdims=True)
        has = np.isfinite(m)
        m_safe = np.where(has, m, 0.0)
        p = np.exp(s - m_safe)
        l = np.sum(p, axis=-1, keepdims=True)
        o = np.matmul(p, v[g]) / np.where(has, l, 1.0)
        out[g * group:(g + 1) * group] = np.where(has, o, 0.0)
        lse[g * group:(g + 1) * group] = np.where(has[..., 0], (m_safe + np.log(np.where(has, l, 1.0)))[..., 0],
                                                  -np.inf)
    return out, lse


def decode(q_words, k_cache_words, v_cache_words, ctx_lens, *, scale=None, dtype=np.float64):
    """One query row per sequence against a resident cache.

    q_words [B, H_q, D], caches [B, H_kv, L_cap, D] (bf16 words); ctx_lens[b] rows attended.
    Returns (o [B, H_q, D], lse [B, H_q]).
    """
    q = bf16_u16_to_fp32(q_words)
    B, hq, d = q.shape
    out = np.zeros((B, hq, d), dtype=dtype)
    lse = np.full((B, hq), -np.inf, dtype=dtype)
    for b in range(B):
        n = int(ctx_lens[b])
        if n <= 0:
            continue
        kb = bf16_u16_to_fp32(k_cache_words[b, :, :n])
        vb = bf16_u16_to_fp32(v_cache_words[b, :, :n])
        o, l = attention(q[b][:, None, :], kb, vb, scale=scale, dtype=dtype)
        out[b] = o[:, 0]
        lse[b] = l[:, 0]
    return out, lse


# ---------------------------------------------------------------------------------------
# fp32 CPU baseline (the timed leg of bench.py)
# ---------------------------------------------------------------------------------------

def cpu_attention_numpy_fp32(q_words, k_words, v_words, *, causal, q_pos_base, kv_pos_base, scale=None):
    """board_performance.py:158-192 generalised: bf16 words in, fp32 stable softmax, fp32 out."""
    qf = bf16_u16_to_fp32(q_words)
    kf = bf16_u16_to_fp32(k_words)
    vf = bf16_u16_to_fp32(v_words)
    hq, lq, d = qf.shape
    hkv, lk, _ = kf.shape
    group = hq // hkv
    sc = np.float32(scale if scale is not None else 1.0 / np.sqrt(d))
    valid = None
    if causal:
        valid = (kv_pos_base + np.arange(lk))[None, :] <= (q_pos_base + np.arange(lq))[:, None]
    out = np.empty((hq, lq, d), dtype=np.float32)
    for g in range(hkv):
        s = np.matmul(qf[g * group:(g + 1) * group], kf[g].T) * sc
        if valid is not None:
            s = np.where(valid[None], s, -np.inf)
        s -= np.max(s, axis=-1, keepdims=True)
        np.exp(s, out=s)
        s /= np.sum(s, axis=-1, keepdims=True)
        out[g * group:(g + 1) * group] = np.matmul(s, vf[g])
    return out


def decode_fp32_baseline(q_words, k_words, v_words, *, scale=None):
    """One (sequence, kv head) decode unit in fp32: q [G, D], k/v [L, D] bf16 words."""
    qf = bf16_u16_to_fp32(q_words)
    kf = bf16_u16_to_fp32(k_words)
    vf = bf16_u16_to_fp32(v_words)
    sc = np.float32(scale if scale is not None else 1.0 / np.sqrt(qf.shape[-1]))
    s = np.matmul(qf, kf.T) * sc
    s -= np.max(s, axis=-1, keepdims=True)
    np.exp(s, out=s)
    s /= np.sum(s, axis=-1, keepdims=True)
    return np.matmul(s, vf)


# ---------------------------------------------------------------------------------------
# parity metric
# ---------------------------------------------------------------------------------------

def weight_rounding_error(out_words, ref, ref_abs_v) -> np.ndarray:
    """Per output element: |out - ref| / (2 bf16 ulp(max |ref| of the row) + 2^-8 * ref_abs_v).

    ``ref_abs_v`` is attention over |V| (sum_k p_k |v_k[d]| / l, e.g. ``attention(q, k, abs(v))``):
    a kernel that rounds each softmax weight to bf16 (relative error <= 2^-8) for the P.V product
    -- as the board does, by truncation, ``attn_top.sv:653-658`` -- is off by at most 2^-8 of it.
    Where the rows of V do not cancel that term is within the output's own magnitude, and the bound
    is the 2-ulp parity measure of ``row_ulp_error``; where they cancel it is what limits any bf16-P
    product.  An element passes when the returned value is <= 1.
    """
    out = bf16_u16_to_fp32(out_words).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    mag = np.max(np.abs(ref), axis=-1, keepdims=True)
    allowed = 2.0 * np.where(mag > 0, bf16_ulp(mag), 0.0) + 2.0 ** -8 * np.asarray(ref_abs_v, dtype=np.float64)
    err = np.abs(out - ref)
    return np.where(allowed > 0, err / np.where(allowed > 0, allowed, 1.0), np.where(err == 0, 0.0, np.inf))


def row_ulp_error(out_words, ref) -> np.ndarray:
    """Per output row (last axis = D): max |out - ref| in units of bf16 ulp(max |ref| of the row).

    This is the parity measure "max abs error <= 2 bf16 ulp of the output magnitude":
    a row passes when the returned value is <= 2.  Rows whose reference is all zero
    (no valid key) must match exactly and report 0 or inf.
    """
    out = bf16_u16_to_fp32(out_words).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.max(np.abs(out - ref), axis=-1)
    mag = np.max(np.abs(ref), axis=-1)
    ulp = bf16_ulp(mag)
    res = np.where(mag > 0, err / ulp, np.where(err == 0, 0.0, np.inf))
    return res
