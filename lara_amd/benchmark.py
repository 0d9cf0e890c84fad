"""Workload definitions and the roofline model of the GQA attention path on MI355X.

This is the counterpart of the reference's analytical model ``sw/benchmark.py``
(``tile_pairs_per_head`` :36-57, ``compute_model`` :60-133).  The board model counted
tile pairs and softmax cycles; on the GPU the path is bound by HBM bandwidth (decode) or
MFMA throughput (chunked prefill), so the model reports algorithmic bytes and FLOPs per
step and the ideal time at MI355X peak.

Algorithmic work (nothing that only exists because of the implementation is counted):

* decode step bytes = sum_b 2*H_kv*L_b*D*2 (K and V rows read)
                      + B*H_q*D*2 (Q read) + B*H_q*D*2 (O written)
                      + B*2*H_kv*D*2 (appended K and V rows written)
* decode kernel bytes (the split-KV kernel with the append fused into it) = K/V rows read + Q read
  + appended rows written (+ O written when no merge launch follows, i.e. the step bytes)
  = 512 B per (kv head, attended key) at D = 128, plus the per-sequence rows.
* FLOPs = 4*sum_b H_q*L_b*D (QK^T and PV multiply-adds);
  prefill counts causal-valid (query, key) pairs only, ops = 2*(2*H_q*pairs*D)
  (sw/board_performance.py:386-388).
"""
from __future__ import annotations

import argparse
import json
import math
from dataclasses import asdict, dataclass, field
from typing import Optional

import numpy as np

# MI355X published peaks (dense).
HBM_PEAK_GBPS = 8000.0
BF16_DENSE_TFLOPS = 2500.0
FP32_VECTOR_TFLOPS = 157.3

# Board contract, for the KV260 tile model below (sw/benchmark.py:17-28).
KV260_TILE_Q = 32
KV260_TILE_KV = 64


@dataclass(frozen=True)
class DecodeWorkload:
    """A decode configuration: every step appends one K/V row per sequence, then attends."""

    name: str
    description: str
    batch: int
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    attended: int = 0                 # keys attended per step (incl. the appended row)
    ragged: Optional[tuple] = None    # (lo, hi) inclusive: per-sequence attended lengths
    amplitude: float = 1.0            # inputs ~ N(0, 1) * amplitude
    outlier_fraction: float = 0.0     # fraction of K rows scaled by outlier_scale
    outlier_scale: float = 1.0
    scale: Optional[float] = None     # softmax scale (None: 1/sqrt(D))
    seed: int = 0

    @property
    def group(self) -> int:
        return self.n_q_heads // self.n_kv_heads

    def lengths(self) -> np.ndarray:
        if self.ragged is None:
            return np.full(self.batch, self.attended, dtype=np.int32)
        lo, hi = self.ragged
        rng = np.random.default_rng(self.seed)
        return rng.integers(lo, hi + 1, self.batch).astype(np.int32)

    @property
    def max_len(self) -> int:
        return int(self.lengths().max())


@dataclass(frozen=True)
class PrefillWorkload:
    name: str
    description: str
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    prompt: int
    chunk: int
    causal: bool = True
    seed: int = 0


# Configurations.  "attended" follows the byte counts of the measurement plan:
# The batch-1 context-4096 decode caches 4096 rows and attends 4097 after the append; the others attend the stated
# context (the appended row is the last of it).
WORKLOADS = {
    "decode-b1-d64-ctx256": DecodeWorkload("decode-b1-d64-ctx256", "board-shape decode: B1, 8q/2kv, D64, ctx 256, no mask", 1, 8, 2, 64,
                         attended=256, scale=1.0 / 8.0, seed=1),
    "decode-b1-ctx4097": DecodeWorkload("decode-b1-ctx4097", "Llama-3-8B decode: B1, 32q/8kv, D128, ctx 4096 + 1 appended", 1, 32, 8, 128,
                         attended=4097, amplitude=0.5, seed=2),
    "decode-b64-ragged": DecodeWorkload("decode-b64-ragged", "batched decode: B64, 32q/8kv, D128, L ~ U[512, 8192]", 64, 32, 8, 128,
                         ragged=(512, 8192), seed=3),
    "decode-b4-ctx131072": DecodeWorkload("decode-b4-ctx131072", "long-context decode: B4, 64q/8kv, D128, L 131072, 1% K rows x8", 4, 64, 8, 128,
                         attended=131072, outlier_fraction=0.01, outlier_scale=8.0, seed=4),
    "decode-b256-ragged": DecodeWorkload("decode-b256-ragged", "batched decode: B256, 32q/8kv, D128, L ~ U[512, 8192]",
                                         256, 32, 8, 128, ragged=(512, 8192), seed=10),
    "decode-b64-ctx8192": DecodeWorkload("decode-b64-ctx8192", "Llama-3-8B GQA decode: B64, 32q/8kv, D128, ctx 8192", 64, 32, 8, 128,
                         attended=8192, seed=5),
}

@dataclass(frozen=True)
class LayerWorkload:
    name: str
    description: str
    n_q_heads: int
    n_kv_heads: int
    head_dim: int
    hidden: int
    tokens: int
    causal: bool = True
    seed: int = 0


LAYER_WORKLOADS = {
    "layer-2048": LayerWorkload("layer-2048", "run_layer input stage + attention: Llama-3-8B shape (hidden 4096, 32q/8kv, D128), "
                                    "2048-token prompt, RMSNorm -> QKV GEMM -> RoPE -> causal attention",
                           32, 8, 128, hidden=4096, tokens=2048, seed=8),
}


def layer_projection_flops(w: LayerWorkload) -> int:
    """2 * tokens * hidden * (H_q + 2 H_kv) * D: the three projections."""
    return 2 * w.tokens * w.hidden * (w.n_q_heads + 2 * w.n_kv_heads) * w.head_dim


PREFILL_WORKLOADS = {
    "prefill-chunked-2048": PrefillWorkload("prefill-chunked-2048", "chunked prefill: B1, 32q/8kv, D128, 2048 tokens in 256-token chunks, causal",
                          32, 8, 128, prompt=2048, chunk=256, seed=6),
}


# ---------------------------------------------------------------------------------------
# work model
# ---------------------------------------------------------------------------------------

def decode_kernel_bytes(n_q_heads: int, n_kv_heads: int, head_dim: int, lengths, *, writes_output: bool = True) -> int:
    """Bytes the split-KV decode kernel moves with the append fused into it: K/V rows read, Q read,
    the appended K/V rows written, and O written when no merge launch follows (writes_output)."""
    lengths = np.asarray(lengths, dtype=np.int64)
    B = len(lengths)
    kv = int(lengths.sum()) * 2 * n_kv_heads * head_dim * 2
    q = B * n_q_heads * head_dim * 2
    append = B * 2 * n_kv_heads * head_dim * 2
    o = B * n_q_heads * head_dim * 2 if writes_output else 0
    return kv + q + append + o


def decode_step_bytes(n_q_heads: int, n_kv_heads: int, head_dim: int, lengths) -> int:
    """Bytes of one decode step: K/V read, Q read, O written, appended rows written."""
    return decode_kernel_bytes(n_q_heads, n_kv_heads, head_dim, lengths, writes_output=True)


def decode_flops(n_q_heads: int, head_dim: int, lengths) -> int:
    return 4 * n_q_heads * head_dim * int(np.asarray(lengths, dtype=np.int64).sum())


def valid_pairs(q_len: int, kv_len: int, *, causal: bool, q_pos_base: int = 0, kv_pos_base: int = 0) -> int:
    """(query, key) pairs that pass the mask (sw/board_performance.py:222-227, any lengths)."""
    if not causal:
        return q_len * kv_len
    qp = q_pos_base + np.arange(q_len, dtype=np.int64)
    # keys at kv_pos_base + j <= qp  ->  j <= qp - kv_pos_base
    per_row = np.clip(qp - kv_pos_base + 1, 0, kv_len)
    return int(per_row.sum())


def prefill_flops(n_q_heads: int, head_dim: int, pairs: int) -> int:
    return 2 * (2 * n_q_heads * pairs * head_dim)


# ---------------------------------------------------------------------------------------
# report metrics (the board harness's, sw/board_performance.py:195-273)
# ---------------------------------------------------------------------------------------

def stats(values) -> dict:
    """min / median / p95 / max of a sample (sw/board_performance.py:195-204)."""
    arr = np.asarray(list(values), dtype=np.float64)
    if arr.size == 0:
        raise ValueError("cannot summarize an empty sample")
    return {"min": float(arr.min()), "median": float(np.median(arr)), "p95": float(np.percentile(arr, 95)),
            "max": float(arr.max())}


def numeric_error(actual, reference) -> dict:
    """Error metrics of sw/board_performance.py:207-219 (relative error floored at 1e-6)."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    delta = a - r
    ref_rms = float(np.sqrt(np.mean(r * r)))
    rmse = float(np.sqrt(np.mean(delta * delta)))
    return {
        "max_abs": float(np.max(np.abs(delta))),
        "mean_abs": float(np.mean(np.abs(delta))),
        "rmse": rmse,
        "normalized_rmse": rmse / max(ref_rms, 1.0e-12),
        "max_relative_floor_1e-6": float(np.max(np.abs(delta) / np.maximum(np.abs(r), 1.0e-6))),
    }


def collect_environment() -> dict:
    """Host environment of a run (the GPU-host analogue of sw/board_performance.py:237-273)."""
    import os
    import platform
    import socket
    import sys
    from datetime import datetime, timezone

    model = None
    try:
        for line in open("/proc/cpuinfo", encoding="utf-8"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "timestamp_utc": datetime.now(timezone.utc).isoformat(),
        "hostname": socket.gethostname(),
        "platform": platform.platform(),
        "python": sys.version.split()[0],
        "numpy": np.__version__,
        "cpu_model": model,
        "os_cpu_count": os.cpu_count(),
        "process_affinity": sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
        "thread_environment": {name: os.environ.get(name) for name in
                               ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS", "NUMEXPR_NUM_THREADS",
                                "LARA_CPU_THREADS")},
    }


def prefill_chunk_schedule(w: PrefillWorkload):
    """(q_pos_base, q_len, kv_len) of every chunk of a chunked prefill."""
    out = []
    for start in range(0, w.prompt, w.chunk):
        q_len = min(w.chunk, w.prompt - start)
        out.append((start, q_len, start + q_len))
    return out


def tile_pairs_per_head(seq_len: int, causal: bool, q_pos_base: int = 0, kv_pos_base: int = 0) -> int:
    """KV260 (Q tile, KV tile) pairs of one head (sw/benchmark.py:36-57), for comparison."""
    n_q = -(-seq_len // KV260_TILE_Q)
    n_kv = -(-seq_len // KV260_TILE_KV)
    if not causal:
        return n_q * n_kv
    pairs = 0
    for t in range(n_q):
        rows = min(KV260_TILE_Q, seq_len - t * KV260_TILE_Q)
        q_end = q_pos_base + t * KV260_TILE_Q + rows - 1
        last = 0 if q_end < kv_pos_base else min((q_end - kv_pos_base) // KV260_TILE_KV, n_kv - 1)
        pairs += last + 1
    return pairs


def compute_model(name: str) -> dict:
    """Roofline summary of a workload (the GPU analogue of sw/benchmark.py:60-133)."""
    if name in WORKLOADS:
        w = WORKLOADS[name]
        lens = w.lengths()
        step = decode_step_bytes(w.n_q_heads, w.n_kv_heads, w.head_dim, lens)
        kern = decode_kernel_bytes(w.n_q_heads, w.n_kv_heads, w.head_dim, lens)
        flops = decode_flops(w.n_q_heads, w.head_dim, lens)
        return {
            "workload": asdict(w),
            "bound": "hbm",
            "step_bytes": step,
            "decode_kernel_bytes": kern,
            "flops": flops,
            "arithmetic_intensity_flop_per_byte": flops / step,
            "ideal_step_us_at_peak": step / (HBM_PEAK_GBPS * 1e3),
            "cache_resident_possible": step < 256 * 2**20,
        }
    w = PREFILL_WORKLOADS[name]
    pairs = sum(valid_pairs(ql, kl, causal=w.causal, q_pos_base=qb) for qb, ql, kl in prefill_chunk_schedule(w))
    flops = prefill_flops(w.n_q_heads, w.head_dim, pairs)
    return {
        "workload": asdict(w),
        "bound": "mfma",
        "valid_pairs_per_head": pairs,
        "flops": flops,
        "ideal_us_at_peak": flops / (BF16_DENSE_TFLOPS * 1e6),
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--workload", default="decode-b64-ctx8192", choices=sorted(WORKLOADS) + sorted(PREFILL_WORKLOADS))
    args = parser.parse_args()
    print(json.dumps(compute_model(args.workload), indent=2, sort_keys=True, default=str))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
