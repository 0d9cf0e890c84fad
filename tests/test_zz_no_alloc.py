"""GPU test of gqa_decode_append_noalloc, the decode entry point that allocates nothing.

It runs over caller-owned cache memory (torch tensors) with its split partials in the library's
static per-device scratch array, and is checked against gqa_decode_append_device on a context
holding the same cache words: output words, LSE and the appended cache rows must be equal word for
word (same kernels, same split plan), and the output within 2 bf16 ulp of the float64 oracle.
Two calls in a row, the second with a smaller input, so a stale scratch from the first call would
show in the second.
"""
import ctypes

import numpy as np
import pytest

from lara_amd import _lib
from oracle import gqa_oracle as orc
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu

ULP_TOL = 2.0
NAN_WORD = 0x7FC0  # stale cache words past every sequence's length


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(lib, torch, rng, B, hq, hkv, d, L_max, lens):
    print(f"[noalloc] B={B} Hq={hq} Hkv={hkv} D={d} L_max={L_max} lens={lens.tolist()}", flush=True)
    lcap = (L_max + 63) // 64 * 64
    kc = np.zeros((B, hkv, lcap, d), np.uint16)
    vc = np.zeros((B, hkv, lcap, d), np.uint16)
    kc[:, :, :L_max] = NAN_WORD
    vc[:, :, :L_max] = NAN_WORD
    for b in range(B):
        n = int(lens[b]) - 1  # the last attended row is appended by the call
        if n > 0:
            kc[b, :, :n] = bf16_normal(rng, (hkv, n, d))
            vc[b, :, :n] = bf16_normal(rng, (hkv, n, d))
    q = bf16_normal(rng, (B, hq, d))
    k_rows = bf16_normal(rng, (B, hkv, d))
    v_rows = bf16_normal(rng, (B, hkv, d))
    pos = (lens - 1).astype(np.int32)

    dev = torch.device("cuda", 0)
    as_dev = lambda a: torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)  # noqa: E731
    q_d, kr_d, vr_d, pos_d, lens_d = (as_dev(x) for x in (q, k_rows, v_rows, pos, lens.astype(np.int32)))
    o_ctx = torch.empty((B, hq, d), dtype=torch.int16, device=dev)
    o_na = torch.full((B, hq, d), -1, dtype=torch.int16, device=dev)
    lse_ctx = torch.empty((B, hq), dtype=torch.float32, device=dev)
    lse_na = torch.full((B, hq), 7.0, dtype=torch.float32, device=dev)
    kc_d, vc_d = as_dev(kc), as_dev(vc)

    cfg = _lib.GqaConfig(B, hq, hkv, d, L_max, 1, 0.0, 0)
    ctx = ctypes.c_void_p()
    _lib.check(lib.gqa_create(ctypes.byref(cfg), ctypes.byref(ctx)), "gqa_create")
    try:
        for b in range(B):
            kb = np.ascontiguousarray(kc[b, :, :L_max])
            vb = np.ascontiguousarray(vc[b, :, :L_max])
            _lib.check(lib.gqa_load_kv(ctx, b, 0, L_max, _lib.as_u16_ptr(kb), _lib.as_u16_ptr(vb)), "load_kv")
        torch.cuda.synchronize()
        _lib.check(lib.gqa_decode_append_device(ctx, _ptr(q_d), _ptr(kr_d), _ptr(vr_d), _ptr(pos_d), _ptr(lens_d),
                                                _ptr(o_ctx), _ptr(lse_ctx), None), "decode_append_device")
        _lib.check(lib.gqa_synchronize(ctx), "sync")
        _lib.check(lib.gqa_decode_append_noalloc(ctypes.byref(cfg), _ptr(kc_d), _ptr(vc_d), lcap, _ptr(q_d),
                                                 _ptr(kr_d), _ptr(vr_d), _ptr(pos_d), _ptr(lens_d), _ptr(o_na),
                                                 _ptr(lse_na), None), "decode_append_noalloc")
        torch.cuda.synchronize()
        k_ctx = np.zeros((B, hkv, L_max, d), np.uint16)
        v_ctx = np.zeros((B, hkv, L_max, d), np.uint16)
        for b in range(B):
            kb = np.zeros((hkv, L_max, d), np.uint16)
            vb = np.zeros((hkv, L_max, d), np.uint16)
            _lib.check(lib.gqa_read_kv(ctx, b, 0, L_max, _lib.as_u16_ptr(kb), _lib.as_u16_ptr(vb)), "read_kv")
            k_ctx[b], v_ctx[b] = kb, vb
    finally:
        lib.gqa_destroy(ctx)

    out_ctx = o_ctx.cpu().numpy().view(np.uint16)
    out_na = o_na.cpu().numpy().view(np.uint16)
    assert np.array_equal(out_na, out_ctx), "output words differ from gqa_decode_append_device"
    assert np.array_equal(lse_na.cpu().numpy().view(np.uint32), lse_ctx.cpu().numpy().view(np.uint32))
    k_na = kc_d.cpu().numpy().view(np.uint16)
    v_na = vc_d.cpu().numpy().view(np.uint16)
    assert np.array_equal(k_na[:, :, :L_max], k_ctx) and np.array_equal(v_na[:, :, :L_max], v_ctx)
    bidx = np.arange(B)
    assert np.array_equal(k_na[bidx, :, pos], k_rows) and np.array_equal(v_na[bidx, :, pos], v_rows)
    ref, _ = orc.decode(q, k_na, v_na, lens)
    worst = float(orc.row_ulp_error(out_na, ref).max())
    assert worst <= ULP_TOL, f"max row error {worst:.3f} bf16 ulp"


def test_noalloc_decode_matches_context_entry_point_twice():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    lib = _lib.lib()
    rng = np.random.default_rng(4242)
    # First call: several splits per sequence (partials in the scratch array), one sequence of one key.
    _case(lib, torch, rng, 3, 32, 8, 128, 5000, np.array([5000, 1, 4097], np.int32))
    # Second call, smaller: the scratch still holds the first call's partials.
    _case(lib, torch, rng, 2, 64, 8, 128, 700, np.array([700, 129], np.int32))


def test_noalloc_matches_context_on_a_ragged_one_split_batch():
    """32 sequences x 8 kv heads fill the GPU with one split each: the context entry point then takes
    its grid rows from a ticket counter (ragged lengths), the no-alloc entry point in index order; the
    words must not depend on which work-group ran which (sequence, kv head)."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    lib = _lib.lib()
    rng = np.random.default_rng(4343)
    lens = rng.integers(1, 601, 32).astype(np.int32)
    lens[0] = 600
    _case(lib, torch, rng, 32, 32, 8, 128, 600, lens)


def test_noalloc_rejects_bad_arguments():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    lib = _lib.lib()
    dev = torch.device("cuda", 0)
    cache = torch.zeros((1, 8, 128, 128), dtype=torch.int16, device=dev)
    q = torch.zeros((1, 32, 128), dtype=torch.int16, device=dev)
    lens = torch.ones((1,), dtype=torch.int32, device=dev)
    o = torch.zeros_like(q)
    cfg = _lib.GqaConfig(1, 32, 8, 128, 100, 1, 0.0, 0)
    call = lambda cfg_p, l_cap, **kw: lib.gqa_decode_append_noalloc(  # noqa: E731
        cfg_p, _ptr(cache), _ptr(cache), l_cap, _ptr(q), None, None, None, _ptr(lens), _ptr(o), None, None)
    assert call(None, 128) == _lib.GQA_ERR_NULL
    assert call(ctypes.byref(cfg), 100) == _lib.GQA_ERR_RANGE  # l_cap not a multiple of 64
    assert call(ctypes.byref(cfg), 64) == _lib.GQA_ERR_RANGE   # l_cap below max_seq_len
    bad = _lib.GqaConfig(1, 30, 8, 128, 100, 1, 0.0, 0)
    assert call(ctypes.byref(bad), 128) == _lib.GQA_ERR_BAD_CFG
    assert call(ctypes.byref(cfg), 128) == _lib.GQA_OK
    torch.cuda.synchronize()
