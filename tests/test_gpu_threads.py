"""Separate contexts are independent: two engines driven from two host threads at once.

ctypes releases the GIL around every library call, so the two threads' calls interleave in
the library and on the GPU.  Each thread's results must be word for word those of the same
calls made by one thread alone, and within the decode tolerance of the float64 oracle.
"""
import threading

import numpy as np
import pytest

from lara_amd.attn_driver import AttentionAccelerator
from oracle import gqa_oracle as orc
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu

SHAPES = {
    "a": dict(batch=4, n_q_heads=32, n_kv_heads=8, head_dim=128, max_seq_len=1024, max_q_len=256),
    "b": dict(batch=3, n_q_heads=16, n_kv_heads=2, head_dim=64, max_seq_len=700, max_q_len=128),
}
STEPS = 6


def workload(name):
    """Seeded inputs of one engine: a cache fill, STEPS decode steps with a fused append each,
    and one causal transaction."""
    s = SHAPES[name]
    rng = np.random.default_rng(900 + len(name) + s["head_dim"])
    B, hq, hkv, d = s["batch"], s["n_q_heads"], s["n_kv_heads"], s["head_dim"]
    lens0 = rng.integers(1, s["max_seq_len"] - STEPS, B).astype(np.int32)
    k = [bf16_normal(rng, (hkv, int(n), d)) for n in lens0]
    v = [bf16_normal(rng, (hkv, int(n), d)) for n in lens0]
    steps = []
    for t in range(STEPS):
        steps.append(dict(q=bf16_normal(rng, (B, hq, d)), k_rows=bf16_normal(rng, (B, hkv, d)),
                          v_rows=bf16_normal(rng, (B, hkv, d)), positions=(lens0 + t).astype(np.int32)))
    L = s["max_q_len"]
    txn = dict(q=bf16_normal(rng, (hq, L, d)), k=bf16_normal(rng, (hkv, L, d)), v=bf16_normal(rng, (hkv, L, d)))
    return lens0, k, v, steps, txn


def run(name, out, barrier=None):
    s = SHAPES[name]
    lens0, k, v, steps, txn = workload(name)
    res = {"decode": [], "lse": []}
    with AttentionAccelerator(**s) as eng:
        for b in range(s["batch"]):
            eng.load_kv(k[b], v[b], b=b)
        if barrier is not None:
            barrier.wait()
        for st in steps:
            o, lse = eng.decode_step(st["q"], st["positions"] + 1, k_rows=st["k_rows"], v_rows=st["v_rows"],
                                     positions=st["positions"], return_lse=True)
            res["decode"].append(o)
            res["lse"].append(lse)
        res["cache_k"], res["cache_v"] = eng.read_kv(0, 0, int(steps[-1]["positions"][0]) + 1)
    with AttentionAccelerator(n_q_heads=s["n_q_heads"], n_kv_heads=s["n_kv_heads"], head_dim=s["head_dim"],
                              max_seq_len=s["max_q_len"]) as eng:
        res["txn"] = eng.run_attention(txn["q"], txn["k"], txn["v"], causal=True)
    out[name] = res


def test_two_contexts_on_two_threads_match_serial_runs():
    serial = {}
    for name in SHAPES:
        print(f"[threads] serial run {name}", flush=True)
        run(name, serial)
    concurrent = {}
    errors = []
    barrier = threading.Barrier(len(SHAPES))

    def worker(name):
        try:
            run(name, concurrent, barrier)
        except Exception as e:  # surfaced below with the thread's name
            errors.append((name, repr(e)))
            barrier.abort()

    print("[threads] concurrent runs", flush=True)
    threads = [threading.Thread(target=worker, args=(n,)) for n in SHAPES]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    for name in SHAPES:
        a, b = serial[name], concurrent[name]
        for x, y in zip(a["decode"] + a["lse"] + [a["cache_k"], a["cache_v"], a["txn"]],
                        b["decode"] + b["lse"] + [b["cache_k"], b["cache_v"], b["txn"]]):
            assert np.array_equal(x, y), name
    # and the concurrent results are the right ones: the last decode step against the oracle
    for name in SHAPES:
        s = SHAPES[name]
        lens0, k, v, steps, _ = workload(name)
        B, hkv, d = s["batch"], s["n_kv_heads"], s["head_dim"]
        lcap = int(steps[-1]["positions"].max()) + 1
        kc = np.zeros((B, hkv, lcap, d), np.uint16)
        vc = np.zeros_like(kc)
        for bi in range(B):
            kc[bi, :, :lens0[bi]] = k[bi]
            vc[bi, :, :lens0[bi]] = v[bi]
            for st in steps:
                kc[bi, :, st["positions"][bi]] = st["k_rows"][bi]
                vc[bi, :, st["positions"][bi]] = st["v_rows"][bi]
        last = steps[-1]
        ref, _ = orc.decode(last["q"], kc, vc, last["positions"] + 1)
        assert float(np.max(orc.row_ulp_error(concurrent[name]["decode"][-1], ref))) <= 2.0, name
