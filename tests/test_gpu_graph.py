"""Replays of a prepared decode step (gqa_graph_capture_decode_append / gqa_graph_launch), and of
decode steps captured into a caller's own HIP graph.

Two engines start from the same cache.  Engine A prepares one fused append+decode step and
replays it; engine B runs the same step eagerly (gqa_decode_append_device).  Between
replays the test writes new inputs into the captured buffers in place, runs unrelated eager
GPU work and synchronises; every replay must equal the eager step word for word (output,
log-sum-exp and the appended cache rows).  The lengths make several splits per sequence, so
a step holds both the split kernel and the combine kernel.
"""
import ctypes

import numpy as np
import pytest

from lara_amd import _lib
from lara_amd.attn_driver import AttentionAccelerator
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dev(words: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(words).view(np.int16)).cuda()


@pytest.mark.parametrize("paged", [False, True])
def test_graph_replays_equal_eager_steps(paged):
    rng = np.random.default_rng(21)
    B, L_MAX = 2, 1024
    lens = np.array([300, 900], np.int32)
    kw = dict(batch=B, max_seq_len=L_MAX)
    if paged:
        kw.update(page_size=64)
    lib = _lib.lib()
    c = ctypes.c_void_p
    with AttentionAccelerator(**kw) as eng_a, AttentionAccelerator(**kw) as eng_b:
        for b in range(B):
            k = bf16_normal(rng, (8, int(lens[b]), 128))
            v = bf16_normal(rng, (8, int(lens[b]), 128))
            for eng in (eng_a, eng_b):
                if paged:
                    eng.reserve(b, L_MAX)
                eng.load_kv(k, v, b=b)
        # one set of device buffers per engine; the graph of A reads A's buffers
        bufs = {}
        for name, eng in (("a", eng_a), ("b", eng_b)):
            bufs[name] = dict(q=torch.zeros((B, 32, 128), dtype=torch.int16, device="cuda"),
                              k=torch.zeros((B, 8, 128), dtype=torch.int16, device="cuda"),
                              v=torch.zeros((B, 8, 128), dtype=torch.int16, device="cuda"),
                              pos=torch.zeros(B, dtype=torch.int32, device="cuda"),
                              lens=torch.zeros(B, dtype=torch.int32, device="cuda"),
                              o=torch.zeros((B, 32, 128), dtype=torch.int16, device="cuda"),
                              lse=torch.zeros((B, 32), dtype=torch.float32, device="cuda"))
        torch.cuda.synchronize()
        ba = bufs["a"]
        graph = c()
        rc = lib.gqa_graph_capture_decode_append(eng_a._ctx, c(ba["q"].data_ptr()), c(ba["k"].data_ptr()),
                                                 c(ba["v"].data_ptr()), c(ba["pos"].data_ptr()),
                                                 c(ba["lens"].data_ptr()), c(ba["o"].data_ptr()),
                                                 c(ba["lse"].data_ptr()), ctypes.byref(graph))
        _lib.check(rc, "gqa_graph_capture_decode_append")
        try:
            cur = lens.copy()
            for step in range(5):
                print(f"[graph] paged={paged} replay {step}", flush=True)
                q = _dev(bf16_normal(rng, (B, 32, 128)))
                k = _dev(bf16_normal(rng, (B, 8, 128)))
                v = _dev(bf16_normal(rng, (B, 8, 128)))
                pos = torch.from_numpy(cur.copy()).cuda()
                ln = torch.from_numpy((cur + 1).astype(np.int32)).cuda()
                for buf in bufs.values():
                    buf["q"].copy_(q)
                    buf["k"].copy_(k)
                    buf["v"].copy_(v)
                    buf["pos"].copy_(pos)
                    buf["lens"].copy_(ln)
                _ = torch.randn(256, 256, device="cuda") @ torch.randn(256, 256, device="cuda")  # unrelated work
                torch.cuda.synchronize()
                _lib.check(lib.gqa_graph_launch(graph, None), "gqa_graph_launch")
                bb = bufs["b"]
                _lib.check(lib.gqa_decode_append_device(eng_b._ctx, c(bb["q"].data_ptr()), c(bb["k"].data_ptr()),
                                                        c(bb["v"].data_ptr()), c(bb["pos"].data_ptr()),
                                                        c(bb["lens"].data_ptr()), c(bb["o"].data_ptr()),
                                                        c(bb["lse"].data_ptr()), None), "eager step")
                _lib.check(lib.gqa_synchronize(eng_a._ctx), "sync a")
                _lib.check(lib.gqa_synchronize(eng_b._ctx), "sync b")
                torch.cuda.synchronize()
                assert torch.equal(bufs["a"]["o"], bufs["b"]["o"]), step
                assert torch.equal(bufs["a"]["lse"], bufs["b"]["lse"]), step
                assert bool(torch.isfinite(bufs["a"]["lse"]).all())
                cur = cur + 1
            for b in range(B):
                ka, va = eng_a.read_kv(b, 0, int(cur[b]))
                kb, vb = eng_b.read_kv(b, 0, int(cur[b]))
                assert np.array_equal(ka, kb) and np.array_equal(va, vb)
        finally:
            lib.gqa_graph_destroy(graph)


def test_steps_captured_into_a_callers_graph_equal_eager_steps():
    """A caller's own stream capture (torch.cuda.graph) of gqa_decode_append_device on a context and of
    gqa_decode_append_noalloc, replayed three times with the inputs rewritten in place and the
    program's eager work and synchronisations between replays: every replay equals an eager step of
    a third engine word for word (output and log-sum-exp).  No library call allocates, synchronises or
    clears memory inside the capture."""
    rng = np.random.default_rng(22)
    B, L_MAX = 2, 1024
    lens = np.array([300, 900], np.int32)
    lib = _lib.lib()
    c = ctypes.c_void_p
    kv = [(bf16_normal(rng, (8, int(n), 128)), bf16_normal(rng, (8, int(n), 128))) for n in lens]
    with AttentionAccelerator(batch=B, max_seq_len=L_MAX) as eng_c, \
            AttentionAccelerator(batch=B, max_seq_len=L_MAX) as eng_n, \
            AttentionAccelerator(batch=B, max_seq_len=L_MAX) as eng_e:
        for eng in (eng_c, eng_n, eng_e):
            for b in range(B):
                eng.load_kv(*kv[b], b=b)
        names = ("ctx", "noalloc", "eager")
        bufs = {n: dict(q=torch.zeros((B, 32, 128), dtype=torch.int16, device="cuda"),
                        k=torch.zeros((B, 8, 128), dtype=torch.int16, device="cuda"),
                        v=torch.zeros((B, 8, 128), dtype=torch.int16, device="cuda"),
                        pos=torch.zeros(B, dtype=torch.int32, device="cuda"),
                        lens=torch.zeros(B, dtype=torch.int32, device="cuda"),
                        o=torch.zeros((B, 32, 128), dtype=torch.int16, device="cuda"),
                        lse=torch.zeros((B, 32), dtype=torch.float32, device="cuda")) for n in names}
        cfg = _lib.GqaConfig(B, 32, 8, 128, L_MAX, 1, 0.0, 0)
        kc, vc, lcap = c(), c(), ctypes.c_int32()
        _lib.check(lib.gqa_cache_pointers(eng_n._ctx, ctypes.byref(kc), ctypes.byref(vc), ctypes.byref(lcap)), "ptrs")
        ptr = lambda n, key: c(bufs[n][key].data_ptr())  # noqa: E731

        def step(n, stream):
            if n == "noalloc":
                return lib.gqa_decode_append_noalloc(ctypes.byref(cfg), kc, vc, lcap.value, ptr(n, "q"), ptr(n, "k"),
                                                     ptr(n, "v"), ptr(n, "pos"), ptr(n, "lens"), ptr(n, "o"),
                                                     ptr(n, "lse"), stream)
            eng = eng_c if n == "ctx" else eng_e
            return lib.gqa_decode_append_device(eng._ctx, ptr(n, "q"), ptr(n, "k"), ptr(n, "v"), ptr(n, "pos"),
                                                ptr(n, "lens"), ptr(n, "o"), ptr(n, "lse"), stream)

        side = torch.cuda.Stream()
        torch.cuda.synchronize()
        # the no-allocation entry point sets itself up on a device's first call, outside any capture
        # (attend only: no row is appended to the cache)
        _lib.check(lib.gqa_decode_append_noalloc(ctypes.byref(cfg), kc, vc, lcap.value, ptr("noalloc", "q"), None,
                                                 None, None, ptr("noalloc", "lens"), ptr("noalloc", "o"), None,
                                                 c(side.cuda_stream)), "noalloc set-up call")
        torch.cuda.synchronize()
        graphs = {}
        for n in ("ctx", "noalloc"):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side, capture_error_mode="thread_local"):
                _lib.check(step(n, c(side.cuda_stream)), f"capture {n}")
            graphs[n] = g
        torch.cuda.synchronize()
        cur = lens.copy()  # the captured launches did not run: the caches still hold the loaded rows
        for rep in range(3):
            print(f"[caller graph] replay {rep}", flush=True)
            q = _dev(bf16_normal(rng, (B, 32, 128)))
            k = _dev(bf16_normal(rng, (B, 8, 128)))
            v = _dev(bf16_normal(rng, (B, 8, 128)))
            pos = torch.from_numpy(cur.copy()).cuda()
            ln = torch.from_numpy((cur + 1).astype(np.int32)).cuda()
            for buf in bufs.values():
                buf["q"].copy_(q)
                buf["k"].copy_(k)
                buf["v"].copy_(v)
                buf["pos"].copy_(pos)
                buf["lens"].copy_(ln)
            _ = torch.randn(256, 256, device="cuda") @ torch.randn(256, 256, device="cuda")  # unrelated work
            torch.cuda.synchronize()
            for g in graphs.values():
                g.replay()
            _lib.check(step("eager", None), "eager step")
            _lib.check(lib.gqa_synchronize(eng_e._ctx), "sync")
            torch.cuda.synchronize()
            for n in ("ctx", "noalloc"):
                assert torch.equal(bufs[n]["o"], bufs["eager"]["o"]), (n, rep)
                assert torch.equal(bufs[n]["lse"], bufs["eager"]["lse"]), (n, rep)
            cur = cur + 1
        for b in range(B):
            want = eng_e.read_kv(b, 0, int(cur[b]))
            for eng in (eng_c, eng_n):
                got = eng.read_kv(b, 0, int(cur[b]))
                assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
