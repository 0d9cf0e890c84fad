#!/usr/bin/env python3
"""GQA decode on one MI355X: us/step and achieved HBM GB/s (fraction of the 8 TB/s peak).

Default workload: Llama-3-8B-shape GQA decode, batch 64, 32 query / 8 KV heads,
head_dim 128, bf16, 8192 attended keys per sequence.  One step appends one K/V row per
sequence (bit-exact row copy into the HBM cache, at a position that advances every step: a
ring over the sequence's rows) and then attends every cached row, in one
split-KV decode launch (plus a log-sum-exp merge launch when a sequence spans several
splits).  Inputs are synthetic N(0, 1) bf16 generated on the GPU and resident in HBM before
the timed region; the cache (2 GiB) is far larger than the 256 MB Infinity Cache, so the
rate is an HBM rate.

Printed: ONE JSON line.  ``value`` is the whole-step algorithmic byte rate in GB/s over the
timed steps (no per-launch events in them); ``roofline`` describes the dominant kernel (the
split-KV decode kernel, the step's only launch) from the HIP events that bracket the timed
steps on its stream, with the average of per-launch events over a second pass of the same
steps beside it; ``cpu_baseline`` times the fp32 NumPy oracle on the host on a bounded
sample of the same workload.  Other workloads (batch-1 context-4097, ragged batch-64 and
batch-4 context-131072 decode, the default decode on a paged cache; chunked prefill; one-shot
prefill; the layer input stage) are measured the same way and reported under
``other_workloads``.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
METRIC = "GQA decode µs/step + achieved HBM GB/s (% of peak) at 1 MI355X"
PROFILE_TRAFFIC = ROOT / "profiles" / "decode_b64_ctx8192_hbm_traffic.txt"
WORKLOAD_NAMES = {
    "decode-b64-ctx8192": "llama3-8b-gqa-decode-b64-ctx8192",
    "decode-b1-ctx4097": "llama3-8b-gqa-decode-b1-ctx4096+1",
    "decode-b64-ragged": "llama3-8b-gqa-decode-b64-ragged-512..8192",
    "decode-b4-ctx131072": "long-context-gqa-decode-b4-64q8kv-ctx131072",
    "decode-b1-d64-ctx256": "board-shape-gqa-decode-b1-8q2kv-d64-ctx256",
    "decode-b256-ragged": "llama3-8b-gqa-decode-b256-ragged-512..8192",
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bench_stream(dev):
    """A stream of the bench's own (default priority) for the library's launches: the timing
    events are recorded on the stream the kernels run on.  Inputs made on torch's stream are
    synchronised before the library reads them."""
    import torch

    return torch.cuda.Stream(device=dev)


_SLEEP_CYCLES_PER_US = None
MAX_GATE_US = 200_000.0  # longest hold of the gate kernel (a bounded spin)


def sleep_rate(stream) -> float:
    """Cycles per microsecond of torch.cuda._sleep (a spin kernel of a given cycle count) on this GPU."""
    global _SLEEP_CYCLES_PER_US
    if _SLEEP_CYCLES_PER_US is None:
        import torch

        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(10_000)
            e0.record(stream)
            torch.cuda._sleep(4_000_000)
            e1.record(stream)
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_US = 4_000_000 / (e0.elapsed_time(e1) * 1e3)
    return _SLEEP_CYCLES_PER_US


MIN_GATED_STEPS = 50  # steps of the gated pass, at least (per-step median and p95)


def timed_passes(lib, _lib, ctx, stream, step, steps: int, warmup: int) -> dict:
    """Warm-up, then a timed pass of `steps` calls of `step` and a gated pass of at least
    MIN_GATED_STEPS calls, on `stream`.

    Timed pass: the steps alone, back to back, between two synchronisations (wall clock) and one
    pair of events on the stream (device time per step).

    Gated pass: a spin kernel of bounded length (torch.cuda._sleep) holds the stream while the host
    queues every step with, through the library's profiling option, a start/stop event pair bound to
    each kernel launch (hipExtLaunchKernel stamps them with the dispatch's own begin and end).  The
    host needs several microseconds per timed launch, which left the GPU idle between launches when
    the steps were queued as they ran; behind the gate the queue is full before the GPU starts, so
    the launches run back to back as in the timed pass (one event pair around the whole pass checks
    that).  It gives each kernel's launch durations; a step's kernel time is the sum of its launches'
    (the steps of a workload all make the same launches).  `gate_held` says whether the gate was
    still running when the last step had been queued.
    """
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    gpu_ms = ev0.elapsed_time(ev1) / steps

    n_gated = max(steps, MIN_GATED_STEPS)
    _lib.check(lib.gqa_set_option(ctx, _lib.GQA_OPT_PROFILE, 1), "profile on")
    try:
        host_us = 0.0
        for _ in range(3):  # host cost of a profiled step: the largest of three
            t1 = time.perf_counter()
            step()
            host_us = max(host_us, (time.perf_counter() - t1) * 1e6)
            torch.cuda.synchronize()
        _lib.check(lib.gqa_set_option(ctx, _lib.GQA_OPT_PROFILE, 1), "profile restart")
        gate_us = min(MAX_GATE_US, 3.0 * host_us * n_gated + 2000.0)
        g0 = torch.cuda.Event(enable_timing=True)
        g1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(int(gate_us * sleep_rate(stream)))
        g0.record(stream)
        for _ in range(n_gated):
            step()
        g1.record(stream)
        gate_held = not g0.query()
        torch.cuda.synchronize()
        gated_gpu_ms = g0.elapsed_time(g1) / n_gated
        times = (ctypes.c_float * _lib.GQA_TIMER_COUNT)()
        counts = (ctypes.c_int32 * _lib.GQA_TIMER_COUNT)()
        _lib.check(lib.gqa_kernel_times(ctx, times, _lib.GQA_TIMER_COUNT), "kernel times")
        _lib.check(lib.gqa_kernel_launch_counts(ctx, counts, _lib.GQA_TIMER_COUNT), "counts")
        step_us = np.zeros(n_gated)
        launch_us = {}
        for slot in range(_lib.GQA_TIMER_COUNT):
            n = int(counts[slot])
            if n == 0:
                continue
            d = (ctypes.c_float * n)()
            got = ctypes.c_int32()
            _lib.check(lib.gqa_kernel_durations(ctx, slot, d, n, ctypes.byref(got)), "durations")
            per = np.frombuffer(d, dtype=np.float32).astype(np.float64)
            launch_us[slot] = per
            if n % n_gated == 0:
                step_us += per.reshape(n_gated, n // n_gated).sum(axis=1)
            else:  # launches do not split evenly over the steps: spread the mean
                step_us += per.sum() / n_gated
    finally:
        _lib.check(lib.gqa_set_option(ctx, _lib.GQA_OPT_PROFILE, 0), "profile off")
    return {"wall_ms": wall_ms, "gpu_ms": gpu_ms, "times": list(times), "counts": list(counts),
            "step_us": step_us, "gate_held": bool(gate_held), "gate_us": gate_us, "gated_steps": n_gated,
            "gated_gpu_ms": gated_gpu_ms, "launch_us": launch_us}


def step_stats(step_us) -> dict:
    """Median / p95 / mean / min / max of per-step kernel times (us) from the gated pass."""
    a = np.asarray(step_us, dtype=np.float64)
    return {"median": float(np.median(a)), "p95": float(np.percentile(a, 95)), "mean": float(a.mean()),
            "min": float(a.min()), "max": float(a.max()), "n": int(a.size)}


def rolling_positions(lens, n_steps: int) -> np.ndarray:
    """[n_steps][B] int32: the cache row step i appends to in sequence b, (L_b - 1 + i) mod L_b --
    the last row first, then a ring over the sequence's L_b rows (L_b >= 1)."""
    lens64 = np.asarray(lens, dtype=np.int64)[None, :]
    steps = np.arange(n_steps, dtype=np.int64)[:, None]
    return ((lens64 - 1 + steps) % lens64).astype(np.int32)


class DecodeBench:
    """Owns one libgqa context and HBM-resident inputs for a decode workload."""

    def __init__(self, w, device: int = 0, chunk: int = 0, page_size: int = 0, merge: int = 0):
        import torch
        from lara_amd import _lib

        self.torch = torch
        self.lib = _lib.lib()
        self._lib = _lib
        self.w = w
        self.lens = w.lengths()
        L = int(self.lens.max())
        cfg = _lib.GqaConfig(w.batch, w.n_q_heads, w.n_kv_heads, w.head_dim, L, 1, float(w.scale or 0.0), device)
        self.ctx = ctypes.c_void_p()
        if page_size:
            # Paged cache: pages handed out round robin, one page per sequence in turn, so every
            # sequence's rows are scattered over the pool.
            pages = [-(-int(n) // page_size) for n in self.lens]
            _lib.check(self.lib.gqa_create_paged(ctypes.byref(cfg), page_size, sum(pages), ctypes.byref(self.ctx)),
                       "gqa_create_paged")
            for p in range(1, max(pages) + 1):
                for b in range(w.batch):
                    if p <= pages[b]:
                        _lib.check(self.lib.gqa_paged_reserve(self.ctx, b, min(int(self.lens[b]), p * page_size)),
                                   "reserve")
        else:
            _lib.check(self.lib.gqa_create(ctypes.byref(cfg), ctypes.byref(self.ctx)), "gqa_create")
        if chunk:
            _lib.check(self.lib.gqa_set_option(self.ctx, _lib.GQA_OPT_DECODE_CHUNK, chunk), "chunk")
        _lib.check(self.lib.gqa_set_option(self.ctx, _lib.GQA_OPT_DECODE_MERGE, merge), "merge")
        dev = torch.device("cuda", device)
        self.stream = bench_stream(dev)
        sptr = ctypes.c_void_p(self.stream.cuda_stream)
        self.sptr = sptr
        g = torch.Generator(device=dev)
        g.manual_seed(w.seed)
        amp = float(w.amplitude)
        # Fill the cache sequence by sequence from device buffers.
        for b in range(w.batch):
            n = int(self.lens[b])
            k = torch.randn((w.n_kv_heads, n, w.head_dim), generator=g, device=dev) * amp
            if w.outlier_fraction > 0:
                rows = torch.rand((w.n_kv_heads, n), generator=g, device=dev) < w.outlier_fraction
                k[rows] *= w.outlier_scale
            k = k.to(torch.bfloat16)
            v = (torch.randn((w.n_kv_heads, n, w.head_dim), generator=g, device=dev) * amp).to(torch.bfloat16)
            torch.cuda.synchronize(dev)  # k, v are written on torch's stream; the copy runs on the bench stream
            _lib.check(self.lib.gqa_load_kv_device(self.ctx, b, 0, n, ctypes.c_void_p(k.data_ptr()),
                                                   ctypes.c_void_p(v.data_ptr()), sptr), "load_kv_device")
            torch.cuda.synchronize(dev)
            del k, v
        # Rolling append: step i of sequence b writes its new K/V row at cache row
        # (L_b - 1 + i) mod L_b -- a ring over the sequence's L_b rows, the oldest row giving way --
        # and attends all L_b rows, so every step attends the configured context while the append
        # position advances as in a decode loop.  Each step takes its Q and new rows from one of
        # INPUT_SETS seeded sets in turn; the position table covers POSITION_STEPS steps, then
        # starts over.
        S = self.INPUT_SETS
        self.q_sets = (torch.randn((S, w.batch, w.n_q_heads, w.head_dim), generator=g, device=dev) * amp).to(
            torch.bfloat16)
        self.k_sets = (torch.randn((S, w.batch, w.n_kv_heads, w.head_dim), generator=g, device=dev) * amp).to(
            torch.bfloat16)
        self.v_sets = (torch.randn((S, w.batch, w.n_kv_heads, w.head_dim), generator=g, device=dev) * amp).to(
            torch.bfloat16)
        self.pos_table = torch.from_numpy(rolling_positions(self.lens, self.POSITION_STEPS)).to(dev)
        self.lens_dev = torch.from_numpy(self.lens.astype(np.int32)).to(dev)
        self.o = torch.empty((w.batch, w.n_q_heads, w.head_dim), dtype=torch.bfloat16, device=dev)
        self.n_steps = 0
        # device addresses of every set and position row, so a step costs the host no tensor indexing
        c = ctypes.c_void_p
        self.set_ptrs = [(c(self.q_sets[s].data_ptr()), c(self.k_sets[s].data_ptr()), c(self.v_sets[s].data_ptr()))
                         for s in range(S)]
        self.pos_ptrs = [c(self.pos_table[i].data_ptr()) for i in range(self.POSITION_STEPS)]
        self.lens_ptr = c(self.lens_dev.data_ptr())
        self.o_ptr = c(self.o.data_ptr())
        # the fixed-pointer form (set 0, first position) for the captured graph
        self.q, self.k_new, self.v_new, self.pos = self.q_sets[0], self.k_sets[0], self.v_sets[0], self.pos_table[0]
        torch.cuda.synchronize(dev)

    INPUT_SETS = 16
    POSITION_STEPS = 1024

    def step(self) -> None:
        i = self.n_steps
        self.n_steps += 1
        q, k, v = self.set_ptrs[i % self.INPUT_SETS]
        rc = self.lib.gqa_decode_append_device(self.ctx, q, k, v, self.pos_ptrs[i % self.POSITION_STEPS],
                                               self.lens_ptr, self.o_ptr, None, self.sptr)
        if rc:
            self._lib.check(rc, "decode_append")

    def run(self, steps: int, warmup: int) -> dict:
        _lib = self._lib
        t = timed_passes(self.lib, _lib, self.ctx, self.stream, self.step, steps, warmup)
        n_dec = max(1, int(t["counts"][_lib.GQA_TIMER_DECODE]))
        merges_per_step = int(t["counts"][_lib.GQA_TIMER_COMBINE]) / n_dec
        decode_us = t["times"][_lib.GQA_TIMER_DECODE]
        combine_us = t["times"][_lib.GQA_TIMER_COMBINE]
        return {
            "wall_us_per_step": t["wall_ms"] * 1e3,
            "gpu_us_per_step": t["gpu_ms"] * 1e3,
            "step_us": step_stats(t["step_us"]),
            "gate_held": t["gate_held"],
            "gated_gpu_us_per_step": t["gated_gpu_ms"] * 1e3,
            "decode_us": decode_us,
            "decode_launches": n_dec,
            "combine_us": combine_us,
            "merges_per_step": merges_per_step,
            "kernels_us_per_step": decode_us + combine_us * merges_per_step,
        }

    def run_graph(self, steps: int, warmup: int) -> float:
        """The same step captured once into a HIP graph and replayed: wall us per step."""
        torch = self.torch
        c = ctypes.c_void_p
        graph = c()
        self._lib.check(self.lib.gqa_graph_capture_decode_append(
            self.ctx, c(self.q.data_ptr()), c(self.k_new.data_ptr()), c(self.v_new.data_ptr()), c(self.pos.data_ptr()),
            c(self.lens_dev.data_ptr()), c(self.o.data_ptr()), None, ctypes.byref(graph)), "graph capture")
        try:
            for _ in range(warmup):
                self.lib.gqa_graph_launch(graph, self.sptr)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                rc = self.lib.gqa_graph_launch(graph, self.sptr)
                if rc:
                    self._lib.check(rc, "graph launch")
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e6 / steps
        finally:
            self.lib.gqa_graph_destroy(graph)

    def close(self) -> None:
        self.lib.gqa_destroy(self.ctx)
        self.ctx = ctypes.c_void_p()


LAUNCH_BOUND = ("decode-b1-d64-ctx256", "decode-b1-ctx4097")  # workloads whose step is also timed as a replayed HIP graph
PAGED_SUFFIX = "-paged"  # a decode or chunked-prefill workload over a paged cache (64-row pages unless --page-rows)
PAGE_ROWS = 64


DECODE_MERGE = {"auto": 0, "launch": 1, "fused": 2}  # GQA_DECODE_MERGE_AUTO / _LAUNCH / _FUSED


INFINITY_CACHE_BYTES = 256 * 2**20  # MI355X last-level (MALL) cache


def residency(working_set: int, byte_rate: bool = True) -> dict:
    """Whether a workload's bytes fit the 256 MiB Infinity Cache: a step that does is served from it
    after warm-up, so a byte rate measured on it is not an HBM rate."""
    resident = working_set <= INFINITY_CACHE_BYTES
    note = "fits the 256 MiB Infinity Cache"
    if resident and byte_rate:
        note += ": GB/s is not an HBM rate (latency-bound)"
    return {"working_set_bytes": int(working_set), "cache_resident": resident,
            "residency": note if resident else "HBM (exceeds the 256 MiB Infinity Cache)"}


def measure(name: str, steps: int, warmup: int, chunk: int = 0, page_rows: int = PAGE_ROWS,
            merge: str = "auto") -> dict:
    from lara_amd.benchmark import HBM_PEAK_GBPS, WORKLOADS, decode_kernel_bytes, decode_step_bytes

    paged = name.endswith(PAGED_SUFFIX)
    w = WORKLOADS[name[: -len(PAGED_SUFFIX)] if paged else name]
    log(f"{name}: filling HBM cache")
    bench = DecodeBench(w, chunk=chunk, page_size=page_rows if paged else 0, merge=DECODE_MERGE[merge])
    try:
        log(f"{name}: warmup {warmup}, timing {steps} steps")
        r = bench.run(steps, warmup)
        if name in LAUNCH_BOUND:
            r["graph_us_per_step"] = bench.run_graph(steps, warmup)
    finally:
        bench.close()
    lens = w.lengths()
    single = r["merges_per_step"] == 0
    step_bytes = decode_step_bytes(w.n_q_heads, w.n_kv_heads, w.head_dim, lens)
    # The split kernel moves K/V, Q and the appended rows, and writes O itself when no merge follows.
    kern_bytes = decode_kernel_bytes(w.n_q_heads, w.n_kv_heads, w.head_dim, lens, writes_output=single)
    us = r["wall_us_per_step"]
    r.update(
        workload=name,
        step_bytes=step_bytes,
        decode_kernel_bytes=kern_bytes,
        us_per_step=us,
        step_gbps=step_bytes / (us * 1e-6) / 1e9,
        decode_kernel_gbps=kern_bytes / (r["decode_us"] * 1e-6) / 1e9 if r["decode_us"] > 0 else None,
        kernels_gbps=step_bytes / (r["kernels_us_per_step"] * 1e-6) / 1e9 if r["kernels_us_per_step"] > 0 else None,
        tokens_per_s=w.batch / (us * 1e-6),
        kernel_timing="gated pass: launches queued behind a bounded spin kernel and run back to back; "
                      "event pairs bound to each launch (mean over the steps)",
    )
    r["step_frac_of_peak"] = r["step_gbps"] / HBM_PEAK_GBPS
    if r["decode_kernel_gbps"]:
        r["decode_kernel_frac_of_peak"] = r["decode_kernel_gbps"] / HBM_PEAK_GBPS
    r.update(residency(step_bytes))
    log(f"{name}: {us:.1f} us/step (device {r['gpu_us_per_step']:.1f}, gated {r['gated_gpu_us_per_step']:.1f}; "
        f"kernels median {r['step_us']['median']:.1f}, p95 {r['step_us']['p95']:.1f}), step {r['step_gbps']:.0f} GB/s; "
        f"decode kernel {r['decode_us']:.1f} us = "
        f"{r.get('decode_kernel_gbps') or 0:.0f} GB/s"
        + (f", merge {r['combine_us']:.1f} us" if not single else "")
        + (f", replayed graph {r['graph_us_per_step']:.1f} us/step" if "graph_us_per_step" in r else "")
        + ("" if r["gate_held"] else " [gate released before the queue was full]"))
    return r


class PrefillBench:
    """Chunked causal prefill: every chunk appends its K/V rows, then attends the growing cache."""

    def __init__(self, w, device: int = 0, target_wgs: int = 0, page_size: int = 0):
        import torch
        from lara_amd import _lib

        self.torch = torch
        self.lib = _lib.lib()
        self._lib = _lib
        self.w = w
        self.ctx = ctypes.c_void_p()
        if page_size:
            # Paged cache: the prompt's pages alternate with a second sequence's, so its rows are
            # scattered over the pool as in a shared one.
            cfg = _lib.GqaConfig(2, w.n_q_heads, w.n_kv_heads, w.head_dim, w.prompt, w.chunk, 0.0, device)
            pages = -(-w.prompt // page_size)
            _lib.check(self.lib.gqa_create_paged(ctypes.byref(cfg), page_size, 2 * pages, ctypes.byref(self.ctx)),
                       "gqa_create_paged")
            for p in range(1, pages + 1):
                for b in range(2):
                    _lib.check(self.lib.gqa_paged_reserve(self.ctx, b, min(w.prompt, p * page_size)), "reserve")
        else:
            cfg = _lib.GqaConfig(1, w.n_q_heads, w.n_kv_heads, w.head_dim, w.prompt, w.chunk, 0.0, device)
            _lib.check(self.lib.gqa_create(ctypes.byref(cfg), ctypes.byref(self.ctx)), "gqa_create")
        if target_wgs:
            _lib.check(self.lib.gqa_set_option(self.ctx, _lib.GQA_OPT_PREFILL_WGS, target_wgs), "prefill wgs")
        dev = torch.device("cuda", device)
        self.stream = bench_stream(dev)
        self.sptr = ctypes.c_void_p(self.stream.cuda_stream)
        g = torch.Generator(device=dev)
        g.manual_seed(w.seed)
        shape_q = (w.n_q_heads, w.prompt, w.head_dim)
        shape_kv = (w.n_kv_heads, w.prompt, w.head_dim)
        q = torch.randn(shape_q, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(shape_kv, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(shape_kv, generator=g, device=dev).to(torch.bfloat16)
        from lara_amd.benchmark import prefill_chunk_schedule

        self.chunks = []
        for start, q_len, kv_len in prefill_chunk_schedule(w):
            self.chunks.append((start, q_len, kv_len, q[:, start:start + q_len].contiguous(),
                                k[:, start:start + q_len].contiguous(), v[:, start:start + q_len].contiguous()))
        self.o = torch.empty((w.n_q_heads, w.chunk, w.head_dim), dtype=torch.bfloat16, device=dev)
        torch.cuda.synchronize(dev)

    def step(self) -> None:
        c = ctypes.c_void_p
        for start, q_len, kv_len, qc, kc, vc in self.chunks:
            # One launch per chunk: place the chunk's K/V rows and attend rows 0..kv_len-1.
            rc = self.lib.gqa_prefill_append_device(self.ctx, 0, c(qc.data_ptr()), c(kc.data_ptr()),
                                                    c(vc.data_ptr()), q_len, q_len, start, kv_len, 0, 1,
                                                    c(self.o.data_ptr()), None, self.sptr)
            if rc:
                self._lib.check(rc, "prefill_append_device")

    def run(self, steps: int, warmup: int) -> dict:
        _lib = self._lib
        t = timed_passes(self.lib, _lib, self.ctx, self.stream, self.step, steps, warmup)
        prompts = t["gated_steps"]
        # mean duration of each chunk's prefill launch (launches repeat chunk by chunk, prompt by prompt)
        pre = t["launch_us"].get(_lib.GQA_TIMER_PREFILL)
        per_chunk = (pre.reshape(prompts, -1).mean(axis=0).tolist()
                     if pre is not None and pre.size % prompts == 0 else None)
        return {"wall_us_per_prompt": t["wall_ms"] * 1e3, "gpu_us_per_prompt": t["gpu_ms"] * 1e3,
                "prefill_us_per_chunk": per_chunk,
                "prompt_us": step_stats(t["step_us"]), "gate_held": t["gate_held"],
                "gated_gpu_us_per_prompt": t["gated_gpu_ms"] * 1e3,
                "prefill_us_per_prompt": t["times"][_lib.GQA_TIMER_PREFILL] * t["counts"][_lib.GQA_TIMER_PREFILL] / prompts,
                "merge_us_per_prompt": t["times"][_lib.GQA_TIMER_COMBINE] * t["counts"][_lib.GQA_TIMER_COMBINE] / prompts,
                "launches_per_prompt": (t["counts"][_lib.GQA_TIMER_PREFILL] + t["counts"][_lib.GQA_TIMER_COMBINE]) / prompts}

    def close(self) -> None:
        self.lib.gqa_destroy(self.ctx)


def measure_prefill(name: str, steps: int, warmup: int, target_wgs: int = 0, page_rows: int = PAGE_ROWS) -> dict:
    from lara_amd.benchmark import BF16_DENSE_TFLOPS, PREFILL_WORKLOADS, prefill_chunk_schedule, prefill_flops, \
        valid_pairs

    paged = name.endswith(PAGED_SUFFIX)
    w = PREFILL_WORKLOADS[name[: -len(PAGED_SUFFIX)] if paged else name]
    log(f"{name}: chunked prefill set-up")
    bench = PrefillBench(w, target_wgs=target_wgs, page_size=page_rows if paged else 0)
    try:
        r = bench.run(steps, warmup)
    finally:
        bench.close()
    sched = prefill_chunk_schedule(w)
    pairs = sum(valid_pairs(ql, kl, causal=w.causal, q_pos_base=qb) for qb, ql, kl in sched)
    flops = prefill_flops(w.n_q_heads, w.head_dim, pairs)
    kern_us = r["prefill_us_per_prompt"]
    merge_us = r["merge_us_per_prompt"]
    tflops = lambda us: flops / (us * 1e-6) / 1e12 if us > 0 else None  # noqa: E731
    out = {
        "us_per_prompt": r["wall_us_per_prompt"],
        "gpu_us_per_prompt": r["gpu_us_per_prompt"],
        "prompt_us": r["prompt_us"],
        "gated_gpu_us_per_prompt": r["gated_gpu_us_per_prompt"],
        "prefill_kernel_us_per_prompt": kern_us,
        "prefill_kernel_us_per_chunk": r["prefill_us_per_chunk"],
        "segment_merge_us_per_prompt": merge_us,
        "launches_per_prompt": r["launches_per_prompt"],
        "chunks": len(sched),
        "flops_per_prompt": flops,
        "kernel_tflops": tflops(kern_us),
        "kernels_tflops_incl_merge": tflops(kern_us + merge_us),
        "prompt_tflops": tflops(r["wall_us_per_prompt"]),
        "kernel_timing": "gated pass: launches queued behind a bounded spin kernel and run back to back; event "
                         "pairs bound to each launch (sums per prompt)",
        "gate_held": r["gate_held"],
        "tokens_per_s": w.prompt / (r["wall_us_per_prompt"] * 1e-6),
    }
    # K/V cache, the prompt's Q and its O.
    out.update(residency(2 * w.n_kv_heads * w.prompt * w.head_dim * 2 + 2 * w.n_q_heads * w.prompt * w.head_dim * 2,
                         byte_rate=False))
    out["mfma_frac_of_bf16_peak"] = out["kernel_tflops"] / BF16_DENSE_TFLOPS if out["kernel_tflops"] else None
    out["mfma_frac_incl_merge"] = (out["kernels_tflops_incl_merge"] / BF16_DENSE_TFLOPS
                                   if out["kernels_tflops_incl_merge"] else None)
    log(f"{name}: {out['us_per_prompt']:.1f} us/prompt (device {out['gpu_us_per_prompt']:.1f}, gated "
        f"{out['gated_gpu_us_per_prompt']:.1f}), prefill kernels "
        f"{kern_us:.1f} us = {out['kernel_tflops'] or 0:.1f} TFLOP/s, segment merges {merge_us:.1f} us"
        + ("" if r["gate_held"] else " [gate released before the queue was full]"))
    if r["prefill_us_per_chunk"]:
        log(f"{name}: prefill kernel per chunk (us): " + ", ".join(f"{x:.1f}" for x in r["prefill_us_per_chunk"]))
    return out


class LayerBench:
    """run_layer on the device: RMSNorm -> QKV GEMM -> RoPE/scatter (gqa_layer_qkv_device), then
    causal attention of the whole prompt (gqa_prefill_device)."""

    def __init__(self, w, device: int = 0, target_wgs: int = 0):
        import torch
        from lara_amd import _lib

        self.torch = torch
        self.lib = _lib.lib()
        self._lib = _lib
        self.w = w
        cfg = _lib.GqaConfig(1, w.n_q_heads, w.n_kv_heads, w.head_dim, w.tokens, w.tokens, 0.0, device)
        self.ctx = ctypes.c_void_p()
        _lib.check(self.lib.gqa_create(ctypes.byref(cfg), ctypes.byref(self.ctx)), "gqa_create")
        if target_wgs:
            _lib.check(self.lib.gqa_set_option(self.ctx, _lib.GQA_OPT_PREFILL_WGS, target_wgs), "prefill wgs")
        dev = torch.device("cuda", device)
        self.stream = bench_stream(dev)
        self.sptr = ctypes.c_void_p(self.stream.cuda_stream)
        g = torch.Generator(device=dev)
        g.manual_seed(w.seed)
        nq, nkv = w.n_q_heads * w.head_dim, w.n_kv_heads * w.head_dim
        s = w.hidden ** -0.5
        self.x = torch.randn((w.tokens, w.hidden), generator=g, device=dev).to(torch.bfloat16)
        # fused QKV weight [H_q + 2 H_kv][D][hidden]: the library runs one projection GEMM
        self.wqkv = (torch.randn((nq + 2 * nkv, w.hidden), generator=g, device=dev) * s).to(torch.bfloat16)
        self.wq, self.wk, self.wv = self.wqkv[:nq], self.wqkv[nq:nq + nkv], self.wqkv[nq + nkv:]
        self.gamma = (1 + 0.1 * torch.randn((w.hidden,), generator=g, device=dev)).to(torch.bfloat16)
        self.q = torch.empty((w.n_q_heads, w.tokens, w.head_dim), dtype=torch.bfloat16, device=dev)
        self.o = torch.empty_like(self.q)
        torch.cuda.synchronize(dev)

    def step(self) -> None:
        c = ctypes.c_void_p
        w = self.w
        rc = self.lib.gqa_layer_qkv_device(self.ctx, 0, c(self.x.data_ptr()), w.tokens, w.hidden, c(self.wq.data_ptr()),
                                           c(self.wk.data_ptr()), c(self.wv.data_ptr()), c(self.gamma.data_ptr()),
                                           ctypes.c_float(1e-5), 0, 0, 0, 1, c(self.q.data_ptr()), self.sptr)
        self._lib.check(rc, "gqa_layer_qkv_device")
        rc = self.lib.gqa_prefill_device(self.ctx, 0, c(self.q.data_ptr()), w.tokens, 0, w.tokens, 0, int(w.causal),
                                         c(self.o.data_ptr()), None, self.sptr)
        self._lib.check(rc, "gqa_prefill_device")

    def run(self, steps: int, warmup: int) -> dict:
        _lib = self._lib
        t = timed_passes(self.lib, _lib, self.ctx, self.stream, self.step, steps, warmup)
        n = t["gated_steps"]
        per = lambda slot: t["times"][slot] * t["counts"][slot] / n  # noqa: E731  (us per layer)
        return {"wall_us": t["wall_ms"] * 1e3, "gpu_us": t["gpu_ms"] * 1e3, "layer_us": step_stats(t["step_us"]),
                "gate_held": t["gate_held"], "norm_us": per(_lib.GQA_TIMER_NORM),
                "proj_us": per(_lib.GQA_TIMER_PROJECTION), "rope_us": per(_lib.GQA_TIMER_ROPE),
                "prefill_us": per(_lib.GQA_TIMER_PREFILL), "merge_us": per(_lib.GQA_TIMER_COMBINE)}

    def close(self) -> None:
        self.lib.gqa_destroy(self.ctx)


def copy_same_bytes(n_bytes: int, pairs: int = 8, launches: int = 40) -> dict:
    """A plain device copy (torch copy_, the runtime's copy kernel) moving n_bytes in and n_bytes out,
    the reference for a streaming kernel of that size: ``launches`` copies back to back behind a
    bounded gate, rotating over ``pairs`` source/destination pairs so that no copy finds its data in
    the L2 the previous one left behind (the footprint, 2 x pairs x n_bytes, exceeds the L2)."""
    import torch

    stream = bench_stream(torch.device("cuda", 0))
    bufs = [(torch.empty(n_bytes, dtype=torch.uint8, device="cuda"), torch.empty(n_bytes, dtype=torch.uint8,
                                                                                device="cuda")) for _ in range(pairs)]
    for src, _ in bufs:
        src.random_(0, 255)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for src, dst in bufs:
            dst.copy_(src)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(int(min(launches * 40.0, MAX_GATE_US) * sleep_rate(stream)))  # host queues ahead
        e0.record(stream)
        for i in range(launches):
            src, dst = bufs[i % pairs]
            dst.copy_(src)
        e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / launches
    return {"bytes_each_way": n_bytes, "us": us, "gbps": 2 * n_bytes / (us * 1e-6) / 1e9,
            "method": f"torch copy_ back to back over {pairs} rotating buffer pairs, {launches} launches"}


def measure_layer(name: str, steps: int, warmup: int, target_wgs: int = 0) -> dict:
    from lara_amd.benchmark import BF16_DENSE_TFLOPS, HBM_PEAK_GBPS, LAYER_WORKLOADS, layer_projection_flops, \
        prefill_flops, valid_pairs

    w = LAYER_WORKLOADS[name]
    log(f"{name}: layer set-up")
    bench = LayerBench(w, target_wgs=target_wgs)
    try:
        r = bench.run(steps, warmup)
    finally:
        bench.close()
    norm_us, proj_us, rope_us = r["norm_us"], r["proj_us"], r["rope_us"]
    proj_flops = layer_projection_flops(w)
    attn_flops = prefill_flops(w.n_q_heads, w.head_dim, valid_pairs(w.tokens, w.tokens, causal=w.causal))
    attn_us = r["prefill_us"] + r["merge_us"]
    # HBM bytes of the two streaming kernels: RMSNorm reads x and writes y (plus gamma); RoPE/scatter
    # reads the [tokens][Q|K|V] projection and writes Q and the K/V cache rows.
    norm_bytes = 2 * w.tokens * w.hidden * 2 + w.hidden * 2
    rope_bytes = 2 * w.tokens * (w.n_q_heads + 2 * w.n_kv_heads) * w.head_dim * 2
    gbps = lambda b, us: b / (us * 1e-6) / 1e9 if us > 0 else None  # noqa: E731
    out = {
        "us_per_layer": r["wall_us"],
        "gpu_us_per_layer": r["gpu_us"],
        "layer_us": r["layer_us"],
        "tokens": w.tokens,
        "rms_norm_us": norm_us,
        "rms_norm_gbps": gbps(norm_bytes, norm_us),
        "qkv_projection_us": proj_us,
        "qkv_projection_tflops": proj_flops / (proj_us * 1e-6) / 1e12 if proj_us > 0 else None,
        "rope_scatter_us": rope_us,
        "rope_scatter_gbps": gbps(rope_bytes, rope_us),
        "attention_us": attn_us,
        "attention_tflops": attn_flops / (attn_us * 1e-6) / 1e12 if attn_us > 0 else None,
        "tokens_per_s": w.tokens / (r["wall_us"] * 1e-6),
        "gate_held": r["gate_held"],
    }
    copies = {"rms_norm": copy_same_bytes(w.tokens * w.hidden * 2),
              "rope_scatter": copy_same_bytes(rope_bytes // 2)}
    for k in ("rms_norm", "rope_scatter"):
        out[f"{k}_frac_of_hbm_peak"] = out[f"{k}_gbps"] / HBM_PEAK_GBPS if out[f"{k}_gbps"] else None
        out[f"{k}_copy_same_bytes"] = copies[k]
        out[f"{k}_frac_of_copy"] = copies[k]["us"] / out[f"{k}_us"] if out[f"{k}_us"] > 0 else None
    out["qkv_projection_frac_of_bf16_peak"] = (out["qkv_projection_tflops"] / BF16_DENSE_TFLOPS
                                               if out["qkv_projection_tflops"] else None)
    log(f"{name}: {out['us_per_layer']:.1f} us/layer: norm {norm_us:.1f} us = {out['rms_norm_gbps'] or 0:.0f} GB/s, "
        f"QKV GEMM {proj_us:.1f} us = {out['qkv_projection_tflops'] or 0:.0f} TFLOP/s, RoPE {rope_us:.1f} us = "
        f"{out['rope_scatter_gbps'] or 0:.0f} GB/s, attention {attn_us:.1f} us = {out['attention_tflops'] or 0:.0f} "
        "TFLOP/s")
    log(f"{name}: a device copy of the same bytes takes {copies['rms_norm']['us']:.1f} us "
        f"({copies['rms_norm']['gbps']:.0f} GB/s; norm at {out['rms_norm_frac_of_copy']:.0%} of it) and "
        f"{copies['rope_scatter']['us']:.1f} us ({copies['rope_scatter']['gbps']:.0f} GB/s; RoPE at "
        f"{out['rope_scatter_frac_of_copy']:.0%})")
    return out


ONESHOT_PREFILL = {"prefill-8192": 8192}  # one causal prefill launch of this many tokens (32 q / 8 kv heads, D 128)
DEFAULT_OTHERS = ("decode-b1-d64-ctx256", "decode-b1-ctx4097", "decode-b64-ragged", "decode-b4-ctx131072", "prefill-chunked-2048",
                  "prefill-8192", "layer-2048", "decode-b64-ctx8192" + PAGED_SUFFIX,
                  "prefill-chunked-2048" + PAGED_SUFFIX)


def measure_prefill_oneshot(name: str, steps: int, warmup: int) -> dict:
    """One causal prefill launch over a whole prompt already in the cache (gqa_prefill_device)."""
    import torch
    from lara_amd import _lib
    from lara_amd.benchmark import BF16_DENSE_TFLOPS, prefill_flops, valid_pairs

    L = ONESHOT_PREFILL[name]
    lib = _lib.lib()
    log(f"{name}: one-shot causal prefill of {L} tokens")
    cfg = _lib.GqaConfig(1, 32, 8, 128, L, L, 0.0, 0)
    ctx = ctypes.c_void_p()
    _lib.check(lib.gqa_create(ctypes.byref(cfg), ctypes.byref(ctx)), "gqa_create")
    try:
        g = torch.Generator(device="cuda")
        g.manual_seed(9)
        q = torch.randn((32, L, 128), generator=g, device="cuda").to(torch.bfloat16)
        k = torch.randn((8, L, 128), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((8, L, 128), generator=g, device="cuda").to(torch.bfloat16)
        o = torch.empty_like(q)
        c = ctypes.c_void_p
        stream = bench_stream(torch.device("cuda", 0))
        sptr = c(stream.cuda_stream)
        torch.cuda.synchronize()
        _lib.check(lib.gqa_load_kv_device(ctx, 0, 0, L, c(k.data_ptr()), c(v.data_ptr()), sptr), "load")

        def step():
            _lib.check(lib.gqa_prefill_device(ctx, 0, c(q.data_ptr()), L, 0, L, 0, 1, c(o.data_ptr()), None, sptr),
                       "prefill")

        r = timed_passes(lib, _lib, ctx, stream, step, steps, warmup)
    finally:
        lib.gqa_destroy(ctx)
    t, n = r["times"], r["counts"]
    kern_us = (t[_lib.GQA_TIMER_PREFILL] * n[_lib.GQA_TIMER_PREFILL] + t[_lib.GQA_TIMER_COMBINE] *
               n[_lib.GQA_TIMER_COMBINE]) / r["gated_steps"]
    flops = prefill_flops(32, 128, valid_pairs(L, L, causal=True))
    out = {"tokens": L, "us_per_prompt": r["wall_ms"] * 1e3, "gpu_us_per_prompt": r["gpu_ms"] * 1e3,
           "prompt_us": step_stats(r["step_us"]), "kernel_us": kern_us, "gate_held": r["gate_held"],
           "kernel_tflops": flops / (kern_us * 1e-6) / 1e12 if kern_us > 0 else None}
    out["mfma_frac_of_bf16_peak"] = out["kernel_tflops"] / BF16_DENSE_TFLOPS if out["kernel_tflops"] else None
    log(f"{name}: {out['us_per_prompt']:.1f} us/prompt, kernels {kern_us:.1f} us = "
        f"{out['kernel_tflops'] or 0:.0f} TFLOP/s")
    return out


CONFIG_LABEL = {"decode-b1-d64-ctx256": "C1", "decode-b1-ctx4097": "C2", "decode-b64-ragged": "C3",
                "decode-b4-ctx131072": "C4", "prefill-chunked-2048": "C5", "decode-b64-ctx8192": "NS",
                "prefill-8192": "p8k", "layer-2048": "layer"}


def _fmt_us(us) -> str:
    if us is None:
        return "-"
    return f"{us / 1e3:.1f}ms" if us >= 1e4 else f"{us:.1f}us"


def _cpu_text(cpu) -> str:
    """'cpu1 <time> <rate> cpuN <time> <rate>' of a cpu_baseline entry (decode: per step; prefill: per prompt)."""
    if not cpu:
        return "cpu -"
    parts = []
    for c in (cpu, cpu.get("all_cores")):
        if not c:
            continue
        t = c.get("us_per_step", c.get("us_per_prompt"))
        rate = f"{c['value']:.1f}GB/s" if c["unit"] == "GB/s" else f"{c['value']:.2f}TF/s"
        parts.append(f"cpu{c['cores']} {_fmt_us(t)} {rate}")
    return " ".join(parts)


def compact(obj, digits: int = 5):
    """obj with every float rounded to `digits` significant digits (ints, strings and None unchanged),
    so the one JSON line stays short enough for a log tail to hold all of it."""
    if isinstance(obj, float):
        if not math.isfinite(obj):
            return obj
        if obj.is_integer() and abs(obj) >= 10**digits:
            return int(obj)  # byte counts keep every digit
        return float(f"{obj:.{digits}g}")
    if isinstance(obj, dict):
        return {k: compact(v, digits) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return [compact(v, digits) for v in obj]
    return obj


def summary_lines(main_name: str, main_r: dict, cpu, others: dict) -> list:
    """One short line per workload (GPU time per step, kernel time and rate, CPU baseline): the last
    lines the bench prints, so that a short tail of its output still holds every configuration."""
    from lara_amd.benchmark import BF16_DENSE_TFLOPS, HBM_PEAK_GBPS

    def label(name):
        base = name.removesuffix(PAGED_SUFFIX)
        tag = CONFIG_LABEL.get(base, "")
        return (tag + "-paged" if name != base and tag else tag) + " " + name

    def decode_line(name, r, c):
        gbps = r.get("kernels_gbps") or 0.0
        cache = " (in cache: latency-bound)" if r.get("cache_resident") else ""
        merge = f"+merge {r['combine_us']:.1f}" if r.get("merges_per_step") else ""
        return (f"{label(name)} {r['us_per_step']:.1f}us/step med {r['step_us']['median']:.1f} "
                f"p95 {r['step_us']['p95']:.1f} | kern {r['decode_us']:.1f}{merge}us {gbps / 1e3:.2f}TB/s "
                f"{gbps / HBM_PEAK_GBPS:.1%}{cache} | {_cpu_text(c)}")

    lines = [decode_line(main_name, main_r, cpu)]
    for name, r in others.items():
        if "us_per_step" in r:
            lines.append(decode_line(name, r, r.get("cpu_baseline")))
        elif "prefill_kernel_us_per_prompt" in r:
            tf = r.get("kernel_tflops") or 0.0
            lines.append(f"{label(name)} {r['us_per_prompt']:.1f}us/prompt | kern {r['prefill_kernel_us_per_prompt']:.1f}"
                         f"us {tf:.0f}TF/s {tf / BF16_DENSE_TFLOPS:.1%} | {_cpu_text(r.get('cpu_baseline'))}")
        elif "kernel_us" in r:
            tf = r.get("kernel_tflops") or 0.0
            lines.append(f"{label(name)} {r['us_per_prompt']:.1f}us/prompt | kern {r['kernel_us']:.1f}us {tf:.0f}TF/s "
                         f"{tf / BF16_DENSE_TFLOPS:.1%}")
        elif "us_per_layer" in r:
            tf = r.get("attention_tflops") or 0.0
            lines.append(f"{label(name)} {r['us_per_layer']:.1f}us/layer | attn {r['attention_us']:.1f}us {tf:.0f}TF/s "
                         f"{tf / BF16_DENSE_TFLOPS:.1%} norm {r['rms_norm_us']:.1f} gemm {r['qkv_projection_us']:.1f} "
                         f"rope {r['rope_scatter_us']:.1f}")
    return lines


def read_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 PMC summary, if present."""
    if not PROFILE_TRAFFIC.is_file():
        return None
    vals = dict(re.findall(r"^(\w+)\s*=\s*([0-9.eE+-]+)\s*$", PROFILE_TRAFFIC.read_text(), flags=re.M))
    try:
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def read_ceiling(gib: int = 4, launches: int = 10) -> dict:
    """Measured HBM streaming-read ceiling (gqa_stream_read_device) beside the 8 TB/s specification.

    A ``gib`` GiB buffer (16x the 256 MB Infinity Cache) is read by the probe kernel with the decode
    kernel's access pattern (16-byte nontemporal loads, 512-thread work-groups over contiguous
    shares), for loads in flight per thread x work-groups over a small grid; each configuration runs
    ``launches`` launches back to back between two events.  The best configuration is the ceiling.
    """
    import torch
    from lara_amd import _lib
    from lara_amd.benchmark import HBM_PEAK_GBPS

    lib = _lib.lib()
    n = gib << 30
    buf = torch.empty(n, dtype=torch.uint8, device="cuda")
    buf.random_(0, 255)
    sink = torch.zeros(8192, dtype=torch.int32, device="cuda")
    stream = bench_stream(torch.device("cuda", 0))
    sptr = ctypes.c_void_p(stream.cuda_stream)
    torch.cuda.synchronize()
    results = []
    for unroll in (1, 2, 4, 8):
        for wgs in (512, 1024, 2048, 4096):
            call = lambda: _lib.check(lib.gqa_stream_read_device(  # noqa: E731
                ctypes.c_void_p(buf.data_ptr()), n, wgs, unroll, ctypes.c_void_p(sink.data_ptr()), sptr), "read probe")
            call()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(launches):
                call()
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / launches
            results.append({"unroll": unroll, "work_groups": wgs, "us": us, "gbps": n / (us * 1e-6) / 1e9})
    del buf
    best = max(results, key=lambda x: x["gbps"])
    log(f"read ceiling: {best['gbps']:.0f} GB/s ({best['unroll']} loads in flight per thread, "
        f"{best['work_groups']} work-groups)")
    return {"gbps": best["gbps"], "frac_of_spec": best["gbps"] / HBM_PEAK_GBPS, "spec_gbps": HBM_PEAK_GBPS,
            "bytes": n, "best": best,
            "sweep_gbps": {f"{r['unroll']}x{r['work_groups']}": round(r["gbps"]) for r in results},
            "method": f"gqa_stream_read_device over {gib} GiB: 16-byte nontemporal loads, 512-thread work-groups, "
                      f"{launches} launches back to back between two events per configuration"}


def launch_floor(launches: int = 200) -> dict:
    """Device time per launch of a kernel that does almost nothing (the read probe over 16 bytes),
    back to back behind a bounded gate on one stream: the fixed cost every step pays per launch
    (dispatch, wave launch and the end-of-kernel cache maintenance), beside which the launch-bound
    workloads (C1, C2) are read.  Measured with 1 and with 256 work-groups."""
    import torch
    from lara_amd import _lib

    lib = _lib.lib()
    stream = bench_stream(torch.device("cuda", 0))
    sptr = ctypes.c_void_p(stream.cuda_stream)
    src = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    out = {}
    for wgs in (1, 256):
        call = lambda: _lib.check(lib.gqa_stream_read_device(  # noqa: E731
            ctypes.c_void_p(src.data_ptr()), 16 * wgs, wgs, 1, ctypes.c_void_p(sink.data_ptr()), sptr), "probe")
        for _ in range(10):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(int(min(launches * 20.0, MAX_GATE_US) * sleep_rate(stream)))  # host queues ahead
            e0.record(stream)
            for _ in range(launches):
                call()
            e1.record(stream)
        torch.cuda.synchronize()
        out[f"us_per_launch_{wgs}_wg"] = e0.elapsed_time(e1) * 1e3 / launches
    out["method"] = (f"{launches} back-to-back launches of the 16-byte-per-work-group read probe "
                     "(gqa_stream_read_device) behind a bounded gate, one event pair around them")
    log(f"launch floor: {out['us_per_launch_1_wg']:.2f} us per launch (1 work-group), "
        f"{out['us_per_launch_256_wg']:.2f} us (256 work-groups)")
    return out


def cpu_threads_all() -> int:
    """Host threads of the all-cores pass: the affinity set, capped by OMP_NUM_THREADS when set."""
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(int(env), aff)) if env.isdigit() and int(env) > 0 else aff


def _timed_repeats(fn, budget_s: float, max_repeats: int = 1000):
    """One warm-up call, then calls until budget_s seconds of timed work (at least one): the
    reference's warm-up / repeat / median method (sw/board_performance.py:295-331)."""
    fn()
    times = []
    while not times or (sum(times) < budget_s and len(times) < max_repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def decode_input_pool(name: str, max_bytes: int = 512 << 20, max_units: int = 16) -> list:
    """Seeded bf16 words for the CPU decode baseline: (q, k, v) of up to ``max_units`` units of the
    workload's longest length, at most ``max_bytes`` of K/V in all (at least two units)."""
    from lara_amd.benchmark import WORKLOADS
    from oracle.gqa_oracle import fp32_to_bf16_u16

    w = WORKLOADS[name]
    max_len = int(w.lengths().max())
    unit_bytes = 2 * max_len * w.head_dim * 2
    n_units = w.batch * w.n_kv_heads
    n_pool = max(2, min(max_units, n_units, max_bytes // unit_bytes))
    rng = np.random.default_rng(w.seed + 1000)
    draw = lambda shape: fp32_to_bf16_u16(rng.standard_normal(shape, dtype=np.float32) * np.float32(w.amplitude))  # noqa: E731
    return [(draw((w.group, w.head_dim)), draw((max_len, w.head_dim)), draw((max_len, w.head_dim)))
            for _ in range(min(n_pool, n_units))]


def cpu_decode_baseline(name: str, budget_s: float, threads: int = 1, pool=None) -> dict:
    """The fp32 NumPy oracle timed on host cores over the workload's decode step.

    A step is every (sequence, kv head) unit of the batch (the reference's CPU model works per KV
    group, sw/board_performance.py:158-192).  Inputs are seeded bf16 words (decode_input_pool)
    cycled over the step's units (the arithmetic does not depend on the values; the pool is larger
    than the last-level cache, so K/V stream from DRAM).  With ``threads`` > 1 the units run on a
    thread pool (NumPy releases the GIL in its kernels), each with one BLAS thread.  When a whole
    step would take more than a third of the budget, a sample of units is timed instead and scaled
    to the step by attended keys (the work of a unit is proportional to its keys).
    """
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    from lara_amd.benchmark import WORKLOADS, decode_step_bytes
    from oracle.gqa_oracle import decode_fp32_baseline

    w = WORKLOADS[name]
    lens = w.lengths()
    pool = pool if pool is not None else decode_input_pool(name)
    n_pool = len(pool)
    units = [(b, h) for b in range(w.batch) for h in range(w.n_kv_heads)]
    keys = np.array([int(lens[b]) for b, _ in units], dtype=np.int64)

    def unit(i: int) -> None:
        q, k, v = pool[i % n_pool]
        L = int(keys[i])
        decode_fp32_baseline(q, k[:L], v[:L], scale=w.scale)

    ex = ThreadPoolExecutor(max_workers=threads) if threads > 1 else None

    def run(sel) -> None:
        if ex is None:
            for i in sel:
                unit(i)
        else:
            list(ex.map(unit, sel))

    try:
        with threadpool_limits(limits=1):
            probe = list(range(min(len(units), threads)))
            run(probe)
            t0 = time.perf_counter()
            run(probe)
            est_step = (time.perf_counter() - t0) * keys.sum() / max(1, keys[probe].sum())
            if est_step <= budget_s / 3:
                sel = list(range(len(units)))
            else:
                n_sel = max(threads, int(len(units) * (budget_s / 3) / est_step))
                if n_sel > threads:
                    n_sel -= n_sel % threads
                sel = list(range(min(len(units), n_sel)))
            times = _timed_repeats(lambda: run(sel), budget_s)
    finally:
        if ex is not None:
            ex.shutdown()
    scale = float(keys.sum()) / float(keys[sel].sum())
    step_s = float(np.median(times)) * scale
    step_bytes = decode_step_bytes(w.n_q_heads, w.n_kv_heads, w.head_dim, lens)
    whole = len(sel) == len(units)
    return {
        "value": step_bytes / step_s / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"median of {len(times)} "
                   + ("whole steps" if whole else f"{len(sel)}/{len(units)}-unit samples x{scale:.2f} by keys")
                   + f", fp32 NumPy oracle, {threads} thread(s) x 1 BLAS, inputs cycled from {n_pool} units, "
                   f"{sum(times):.1f} s"),
        "us_per_step": step_s * 1e6,
        "us_per_step_p95": float(np.percentile(times, 95)) * scale * 1e6,
    }


def cpu_prefill_baseline(name: str, budget_s: float, threads: int = 1) -> dict:
    """The fp32 NumPy oracle timed on host cores over whole chunked prompts of the workload.

    A prompt runs every chunk's transaction (cpu_attention_numpy_fp32: per KV group, causal mask
    at the chunk's absolute positions, sw/board_performance.py:158-192 generalised) on seeded bf16
    words; BLAS uses ``threads`` threads.  Rate: causal-valid FLOPs (4 * H_q * pairs * D,
    sw/board_performance.py:386-388) per second of the median prompt.
    """
    from threadpoolctl import threadpool_limits

    from lara_amd.benchmark import PREFILL_WORKLOADS, prefill_chunk_schedule, prefill_flops, valid_pairs
    from oracle.gqa_oracle import cpu_attention_numpy_fp32, fp32_to_bf16_u16

    w = PREFILL_WORKLOADS[name]
    rng = np.random.default_rng(w.seed + 1000)
    q = fp32_to_bf16_u16(rng.standard_normal((w.n_q_heads, w.prompt, w.head_dim), dtype=np.float32))
    k = fp32_to_bf16_u16(rng.standard_normal((w.n_kv_heads, w.prompt, w.head_dim), dtype=np.float32))
    v = fp32_to_bf16_u16(rng.standard_normal((w.n_kv_heads, w.prompt, w.head_dim), dtype=np.float32))
    sched = prefill_chunk_schedule(w)

    def prompt() -> None:
        for start, q_len, kv_len in sched:
            cpu_attention_numpy_fp32(q[:, start:start + q_len], k[:, :kv_len], v[:, :kv_len], causal=w.causal,
                                     q_pos_base=start, kv_pos_base=0)

    with threadpool_limits(limits=threads):
        times = _timed_repeats(prompt, budget_s)
    pairs = sum(valid_pairs(ql, kl, causal=w.causal, q_pos_base=qb) for qb, ql, kl in sched)
    flops = prefill_flops(w.n_q_heads, w.head_dim, pairs)
    med = float(np.median(times))
    return {
        "value": flops / med / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"median of {len(times)} whole prompts ({len(sched)} chunks), fp32 NumPy oracle per KV group, "
                   f"{threads} BLAS thread(s), {sum(times):.1f} s"),
        "us_per_prompt": med * 1e6,
        "us_per_prompt_p95": float(np.percentile(times, 95)) * 1e6,
    }


def cpu_baselines(name: str, budget_s: float, all_budget_s: float) -> dict:
    """One-thread pass and all-cores pass of the CPU baseline for a decode or prefill workload."""
    from lara_amd.benchmark import PREFILL_WORKLOADS

    n_all = cpu_threads_all()
    log(f"{name}: cpu baseline, 1 thread ({budget_s:.0f} s) and {n_all} threads ({all_budget_s:.0f} s)")
    if name in PREFILL_WORKLOADS:
        one = cpu_prefill_baseline(name, budget_s, 1)
        one["all_cores"] = cpu_prefill_baseline(name, all_budget_s, n_all) if n_all > 1 else None
    else:
        pool = decode_input_pool(name)
        one = cpu_decode_baseline(name, budget_s, 1, pool)
        one["all_cores"] = cpu_decode_baseline(name, all_budget_s, n_all, pool) if n_all > 1 else None
    return one


def copy_calibration(mib: int) -> int:
    """A plain copy kernel of known size: reads and writes ``mib`` MiB per launch."""
    import torch

    n = mib * 2**20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": n, "launches": 5}), flush=True)
    return 0


def _board_cases(args, orc):
    """The matrix's transactions: board case files (--case-set LABEL=DIR) or seeded synthetic sets."""
    lengths = [int(x) for x in args.lengths.split(",") if x]
    cases = []
    if args.case_set:
        for spec in args.case_set:
            label, _, directory = spec.partition("=")
            if not directory:
                raise SystemExit(f"--case-set wants LABEL=DIR, got {spec!r}")
            paths = sorted(Path(directory).glob("case_*.npz"))
            if not paths:
                raise SystemExit(f"no case_*.npz files in {directory}")
            for path in paths:
                with np.load(path, allow_pickle=False) as d:
                    q = np.asarray(d["q_heads"], dtype=np.uint16)
                    L = int(np.asarray(d["seq_len"]).reshape(-1)[0]) if "seq_len" in d.files else q.shape[1]
                    causal = bool(np.asarray(d["causal"]).reshape(-1)[0]) if "causal" in d.files else True
                    qb = int(np.asarray(d["q_pos_base"]).reshape(-1)[0]) if "q_pos_base" in d.files else 0
                    kb = int(np.asarray(d["kv_pos_base"]).reshape(-1)[0]) if "kv_pos_base" in d.files else 0
                    if (args.lengths_given and L not in lengths) or (args.causal_only and not causal):
                        continue
                    cases.append(dict(case_id=f"{label}/{path.stem}", case_set=label, seq_len=L, causal=causal,
                                      q_pos_base=qb, kv_pos_base=kb, q=q,
                                      k=np.asarray(d["k_heads"], dtype=np.uint16),
                                      v=np.asarray(d["v_heads"], dtype=np.uint16),
                                      expected=np.asarray(d["expected_o"], dtype=np.uint16)
                                      if "expected_o" in d.files else None, input=str(path)))
        return cases
    case_sets = {"q0kv0": (0, 0), "q3kv3": (3, 3), "q31kv7": (31, 7)}
    for label, (qb, kb) in case_sets.items():
        for L in lengths:
            for causal in ((True,) if args.causal_only else (True, False)):
                rng = np.random.default_rng(len(cases) + 7919 * L)
                cases.append(dict(case_id=f"{label}_L{L}_q{qb}_kv{kb}_{'causal' if causal else 'noncausal'}",
                                  case_set=label, seq_len=L, causal=causal, q_pos_base=qb, kv_pos_base=kb,
                                  q=orc.fp32_to_bf16_u16(rng.standard_normal((32, L, 128), dtype=np.float32)),
                                  k=orc.fp32_to_bf16_u16(rng.standard_normal((8, L, 128), dtype=np.float32)),
                                  v=orc.fp32_to_bf16_u16(rng.standard_normal((8, L, 128), dtype=np.float32)),
                                  expected=None, input=None))
    return cases


def board_matrix(args) -> int:
    """The board performance matrix on the GPU (sw/board_performance.py:281-473, 573-747 re-targeted).

    For every transaction of the KV260 contract -- Q [32, L, 128], K/V [8, L, 128], bf16; from
    board case files (--case-set LABEL=DIR, the sw/board_matrix.py:117-126 format) or seeded
    N(0, 1) sets over (position bases, L, causal) -- it times ``run_attention`` (host-to-host
    and the attention kernels alone) and the fp32 NumPy CPU model on the host.  Correctness:
    with ``--numerics exact`` every row within 2 bf16 ulp of the float64 oracle; with
    ``--numerics kv260`` the output equals the C restatement of the board arithmetic word for
    word and, where a case file holds ``expected_o``, those words too (the board's
    ``fpga_bit_exact_expected``).  Writes ``performance.json`` and ``performance.csv``.
    """
    import csv

    from threadpoolctl import threadpool_limits

    from lara_amd import benchmark as bm
    from lara_amd.attn_driver import AttentionAccelerator, RunProfile
    from oracle import gqa_oracle as orc

    rtl = None
    if args.numerics == "kv260":
        from oracle import rtl_exact as rtl
    cases = _board_cases(args, orc)
    if not cases:
        raise SystemExit("board matrix: no cases selected")
    out_dir = Path(args.output_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    rows, errors = [], []
    L_max = max(max(c["seq_len"] for c in cases), 16)
    with AttentionAccelerator(max_seq_len=L_max, max_q_len=L_max, numerics=args.numerics) as acc, \
            threadpool_limits(limits=args.cpu_threads):
        for case in cases:
            case_id, L, causal = case["case_id"], case["seq_len"], case["causal"]
            qb, kb = case["q_pos_base"], case["kv_pos_base"]
            q, k, v = case["q"], case["k"], case["v"]
            log(f"board case {case_id}")
            kw = dict(q_pos_base=qb, kv_pos_base=kb, causal=causal)
            try:
                for _ in range(args.board_warmup):
                    acc.run_attention(q, k, v, seq_len=L, **kw)
                    orc.cpu_attention_numpy_fp32(q[:, :L], k[:, :L], v[:, :L], **kw)
                profiles = []
                for _ in range(args.board_repeats):
                    out = acc.run_attention(q, k, v, seq_len=L, **kw)
                    profiles.append(acc.last_profile.to_dict())
                cpu_ms = []
                for _ in range(args.board_repeats):
                    t0 = time.perf_counter_ns()
                    cpu_out = orc.cpu_attention_numpy_fp32(q[:, :L], k[:, :L], v[:, :L], **kw)
                    cpu_ms.append((time.perf_counter_ns() - t0) / 1e6)
            except (ValueError, RuntimeError) as exc:  # keep the matrix going; the case is recorded as an error
                errors.append({"case_id": case_id, "error": f"{type(exc).__name__}: {exc}"})
                continue
            exact, _ = orc.attention(orc.bf16_u16_to_fp32(q[:, :L]), orc.bf16_u16_to_fp32(k[:, :L]),
                                     orc.bf16_u16_to_fp32(v[:, :L]), **kw)
            gpu_f = orc.bf16_u16_to_fp32(out)
            ulp = float(orc.row_ulp_error(out, exact).max())
            correctness = {
                "gpu_max_row_error_bf16_ulp": ulp,
                "gpu_within_2_ulp": ulp <= 2.0,
                "gpu_bf16_vs_exact": bm.numeric_error(gpu_f, exact),
                "cpu_fp32_vs_exact": bm.numeric_error(cpu_out, exact),
                "cpu_fp32_vs_gpu_bf16": bm.numeric_error(cpu_out, gpu_f),
            }
            if rtl is not None:
                want, _, _ = rtl.attention(q[:, :L], k[:, :L], v[:, :L], **kw)
                correctness["gpu_bit_exact_kv260_model"] = bool(np.array_equal(out, want))
            if case["expected"] is not None:
                mism = int(np.count_nonzero(out != case["expected"]))
                correctness["gpu_bit_exact_expected"] = mism == 0
                correctness["expected_mismatches"] = mism
            correctness["passed"] = (correctness.get("gpu_bit_exact_kv260_model", correctness["gpu_within_2_ulp"])
                                     and correctness.get("gpu_bit_exact_expected", True))
            pairs = bm.valid_pairs(L, L, causal=causal, q_pos_base=qb, kv_pos_base=kb)
            macs = 2 * 32 * pairs * 128
            ops = 2 * macs
            h2h = bm.stats(p["attention_total_ms"] for p in profiles)
            kern = bm.stats(p["pl_mac_ms"] for p in profiles)
            cpu = bm.stats(cpu_ms)
            rows.append({
                "case_id": case_id, "case_set": case["case_set"], "input": case["input"], "seq_len": L,
                "causal": causal, "q_pos_base": qb, "kv_pos_base": kb, "numerics": args.numerics,
                "warmup": args.board_warmup, "repeats": args.board_repeats,
                "correctness": correctness,
                "work": {"valid_qk_pairs_per_q_head": pairs, "attention_macs_qk_plus_pv": macs,
                         "algorithmic_ops_two_per_mac": ops},
                "gpu": {"host_to_host_attention_ms": h2h, "attention_kernels_ms": kern,
                        "host_to_host_effective_gops_median": ops / (h2h["median"] * 1e6),
                        "kernel_effective_gops_median": ops / (kern["median"] * 1e6) if kern["median"] > 0
                        else None,
                        "profiles": profiles},
                "cpu_baseline": {"definition": "fp32 NumPy GQA attention on the GPU host; bf16 inputs; stable "
                                              "exact-exp softmax", "threads": args.cpu_threads,
                                 "wall_ms": cpu,
                                 "effective_gops_median": ops / (cpu["median"] * 1e6)},
                "speedup": {"cpu_over_gpu_host_to_host": cpu["median"] / h2h["median"],
                            "cpu_over_gpu_kernels": cpu["median"] / kern["median"] if kern["median"] > 0
                            else None},
            })
    report = {"schema": "lara-mi355x-board-performance-v1", "environment": bm.collect_environment(),
              "numerics": args.numerics, "profile_fields": list(RunProfile.__dataclass_fields__),
              "results": rows, "benchmark_errors": errors}
    (out_dir / "performance.json").write_text(json.dumps(report, indent=2) + "\n", encoding="utf-8")
    with (out_dir / "performance.csv").open("w", newline="", encoding="utf-8") as f:
        w = csv.writer(f)
        w.writerow(["case_id", "seq_len", "causal", "passed", "max_row_ulp", "gpu_h2h_ms_median",
                    "gpu_kernel_ms_median", "cpu_ms_median", "kernel_gops", "cpu_gops", "speedup_h2h",
                    "speedup_kernel"])
        for r in rows:
            w.writerow([r["case_id"], r["seq_len"], r["causal"], r["correctness"]["passed"],
                        r["correctness"]["gpu_max_row_error_bf16_ulp"],
                        r["gpu"]["host_to_host_attention_ms"]["median"], r["gpu"]["attention_kernels_ms"]["median"],
                        r["cpu_baseline"]["wall_ms"]["median"], r["gpu"]["kernel_effective_gops_median"],
                        r["cpu_baseline"]["effective_gops_median"], r["speedup"]["cpu_over_gpu_host_to_host"],
                        r["speedup"]["cpu_over_gpu_kernels"]])
    passed = sum(r["correctness"]["passed"] for r in rows)
    check = "bit-exact" if args.numerics == "kv260" else "within 2 bf16 ulp"
    print(json.dumps({"board_matrix": f"{passed}/{len(cases)} {check}", "errors": len(errors),
                      "output_dir": str(out_dir)}), flush=True)
    return 0 if passed == len(cases) and not errors else 1


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--workload", default="decode-b64-ctx8192", choices=sorted(WORKLOAD_NAMES))
    parser.add_argument("--chunk", type=int, default=0, help="keys per split-KV work-group (0 = auto)")
    parser.add_argument("--decode-merge", default="auto", choices=sorted(DECODE_MERGE),
                        help="split merge of the decode: in the decode launch (fused), a second launch, or auto "
                             "(fused while the split grid fills at most half the CUs)")
    parser.add_argument("--page-rows", type=int, default=PAGE_ROWS,
                        help="rows per page of the paged-cache workloads (power of two, >= 64)")
    parser.add_argument("--prefill-wgs", type=int, default=0,
                        help="work-groups the prefill KV segmentation aims for (0 = auto, 1 = no segments)")
    parser.add_argument("--others", default=",".join(DEFAULT_OTHERS),
                        help="extra workloads to report, comma-separated ('' = none); decode workloads also run "
                             "on a paged cache with the suffix " + PAGED_SUFFIX)
    parser.add_argument("--cpu-seconds", type=float, default=12.0,
                        help="CPU baseline budget of the headline workload's one-thread pass")
    parser.add_argument("--cpu-seconds-other", type=float, default=3.0,
                        help="CPU baseline budget of every other pass (all-cores, other workloads)")
    parser.add_argument("--no-read-ceiling", action="store_true", help="skip the streaming-read ceiling probe")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--calibrate-copy-mib", type=int, default=0,
                        help="only run a plain device-to-device copy of this many MiB (5 times) and exit; "
                             "used to scale the FETCH_SIZE / WRITE_SIZE counters")
    parser.add_argument("--board-matrix", action="store_true",
                        help="run the board transaction matrix (lengths x causal x position bases) instead")
    parser.add_argument("--lengths", default=None,
                        help="board matrix sequence lengths (default 1,16,32,64,128,512; with --case-set: all)")
    parser.add_argument("--case-set", action="append", default=[], metavar="LABEL=DIR",
                        help="board matrix: run the case_*.npz files of DIR (repeatable) instead of synthetic sets")
    parser.add_argument("--causal-only", action="store_true", help="board matrix: causal transactions only")
    parser.add_argument("--numerics", default="exact", choices=("exact", "kv260"),
                        help="board matrix: engine arithmetic (kv260 = the board's, checked word for word)")
    parser.add_argument("--board-warmup", type=int, default=1)
    parser.add_argument("--board-repeats", type=int, default=5)
    parser.add_argument("--cpu-threads", type=int, default=int(os.environ.get("LARA_CPU_THREADS", "1")))
    parser.add_argument("--output-dir", default="board_performance_results")
    args = parser.parse_args()
    from lara_amd.benchmark import LAYER_WORKLOADS, PREFILL_WORKLOADS

    known = set(WORKLOAD_NAMES) | {n + PAGED_SUFFIX for n in WORKLOAD_NAMES} | set(PREFILL_WORKLOADS) | \
        {n + PAGED_SUFFIX for n in PREFILL_WORKLOADS} | set(LAYER_WORKLOADS) | set(ONESHOT_PREFILL)
    unknown = [x for x in args.others.split(",") if x and x not in known]
    if unknown:
        parser.error(f"--others: unknown workload(s) {', '.join(unknown)}; known: {', '.join(sorted(known))}")
    args.lengths_given = args.lengths is not None
    if args.lengths is None:
        args.lengths = "1,16,32,64,128,512"

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the engine has no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        return 2

    import torch

    from lara_amd.benchmark import HBM_PEAK_GBPS, LAYER_WORKLOADS, PREFILL_WORKLOADS, WORKLOADS

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (gfx950)", file=sys.stderr)
        return 1
    if args.calibrate_copy_mib:
        return copy_calibration(args.calibrate_copy_mib)
    if args.board_matrix:
        return board_matrix(args)
    main_r = measure(args.workload, args.steps, args.warmup, args.chunk, args.page_rows, args.decode_merge)
    others = {}
    decode_keys = ("us_per_step", "gpu_us_per_step", "gated_gpu_us_per_step", "step_us", "step_gbps", "step_frac_of_peak", "decode_us",
                   "combine_us", "merges_per_step", "kernels_us_per_step", "decode_kernel_bytes",
                   "decode_kernel_gbps", "decode_kernel_frac_of_peak", "kernels_gbps", "tokens_per_s",
                   "graph_us_per_step", "gate_held", "working_set_bytes", "cache_resident")
    for name in [x for x in args.others.split(",") if x and x != args.workload]:
        if name.removesuffix(PAGED_SUFFIX) in PREFILL_WORKLOADS:
            others[name] = measure_prefill(name, max(10, args.steps // 2), max(2, args.warmup // 2), args.prefill_wgs,
                                           args.page_rows)
        elif name in ONESHOT_PREFILL:
            others[name] = measure_prefill_oneshot(name, max(5, args.steps // 10), 2)
        elif name in LAYER_WORKLOADS:
            others[name] = measure_layer(name, max(10, args.steps // 4), max(2, args.warmup // 2), args.prefill_wgs)
        else:
            r = measure(name, max(10, args.steps // 2), max(2, args.warmup // 2), page_rows=args.page_rows,
                        merge=args.decode_merge)
            others[name] = {k: r[k] for k in decode_keys if k in r}
    ceiling = None if args.no_read_ceiling else read_ceiling()
    floor = launch_floor()
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baselines(args.workload, args.cpu_seconds, args.cpu_seconds_other)
        for name in others:
            if name in WORKLOADS or name in PREFILL_WORKLOADS:
                others[name]["cpu_baseline"] = cpu_baselines(name, args.cpu_seconds_other, args.cpu_seconds_other)

    from lara_amd.benchmark import collect_environment

    w = WORKLOADS[args.workload]
    achieved = main_r["decode_kernel_gbps"]
    roofline = {
        "bound": "hbm",
        "kernel": "decode_split_kernel<128,4,8>" if w.head_dim == 128 and w.group == 4 else "decode_split_kernel",
        "achieved": achieved,
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": achieved / HBM_PEAK_GBPS if achieved else None,
        "traffic": read_traffic() if args.workload == "decode-b64-ctx8192" else None,
        "traffic_source": (f"{PROFILE_TRAFFIC.relative_to(ROOT)} (rocprofv3 FETCH_SIZE and WRITE_SIZE runs of this "
                           "kernel, scaled by a plain copy's counters); not measured in this run"
                           if args.workload == "decode-b64-ctx8192" else None),
        "algorithmic_bytes_per_launch": main_r["decode_kernel_bytes"],
        "algorithmic_bytes": "K and V rows read + Q read + appended K/V rows written + O written",
        "avg_launch_us": main_r["decode_us"],
        "launches_averaged": main_r["decode_launches"],
        "timing": main_r["kernel_timing"],
        "timed_pass_device_us_per_step": main_r["gpu_us_per_step"],
        "frac_of_measured_read_ceiling": achieved / ceiling["gbps"] if (achieved and ceiling) else None,
    }
    line = {
        "metric": METRIC,
        "value": main_r["step_gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_r["us_per_step"] * 1e-3,
        "us_per_step": main_r["us_per_step"],
        "step_us_median": main_r["step_us"]["median"],
        "step_us_p95": main_r["step_us"]["p95"],
        "frac_of_hbm_peak": main_r["step_frac_of_peak"],
        "tokens_per_s": main_r["tokens_per_s"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 generated on the GPU, resident in HBM",
        "config": {
            "workload": WORKLOAD_NAMES[args.workload],
            "batch": w.batch,
            "n_q_heads": w.n_q_heads,
            "n_kv_heads": w.n_kv_heads,
            "head_dim": w.head_dim,
            "attended_keys": int(w.lengths().max()),
            "step": "append 1 K/V row per sequence fused into the split-KV decode launch ("
                    + ("plus an LSE-merge launch: the sequences span several splits"
                       if main_r["merges_per_step"] > 0 else
                       "no merge launch: one split per sequence, or the splits merged inside the launch")
                    + "); rolling append: step i writes row (L - 1 + i) mod L of each sequence (a ring over its L "
                    "rows) and attends all L rows; "
                    f"Q and the new rows cycle over {DecodeBench.INPUT_SETS} seeded sets",
            "accumulate": "fp32",
            "working_set_bytes": main_r["working_set_bytes"],
            "residency": main_r["residency"],
        },
        "kernels_us": {"decode_step": main_r["decode_us"],
                       "merge": main_r["combine_us"] if main_r["merges_per_step"] > 0 else None,
                       "per_step": main_r["kernels_us_per_step"]},
        "roofline": roofline,
        "read_ceiling": ceiling,
        "launch_floor": floor,
        "cpu_baseline": cpu,
        "environment": collect_environment(),
        "other_workloads": {k: {f: v for f, v in r.items() if f != "residency"} for k, r in others.items()},
        "residency_note": ("cache_resident: the workload's bytes fit the 256 MiB Infinity Cache, so after warm-up "
                           "its steps are served from it and its GB/s are not HBM rates"),
    }
    line["summary"] = summary_lines(args.workload, main_r, cpu, others)
    print(json.dumps(compact(line), separators=(",", ":")), flush=True)
    for text in line["summary"]:
        print(f"[summary] {text}", file=sys.stderr, flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
