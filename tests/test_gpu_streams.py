"""Stream ordering of the device-pointer entry points called with stream NULL.

NULL selects the context stream, a blocking HIP stream: it is ordered both ways with the
legacy default stream (handle 0), which is PyTorch's default stream.  The default stream is
kept busy with matrix products before it writes the inputs; the library's copy must still see
the final words, and torch code that reads the library's output right after the call must
see the finished result.
"""
import ctypes

import numpy as np
import pytest

from lara_amd import _lib
from lara_amd.attn_driver import AttentionAccelerator
from oracle import gqa_oracle as orc
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _busy_default_stream():
    a = torch.randn(4096, 4096, device="cuda")
    for _ in range(6):
        a = (a @ a) * 1e-3
    return a


def test_null_stream_calls_are_ordered_with_the_default_stream():
    rng = np.random.default_rng(31)
    L = 2048
    kw = bf16_normal(rng, (8, L, 128))
    vw = bf16_normal(rng, (8, L, 128))
    q = bf16_normal(rng, (1, 32, 128))
    c = ctypes.c_void_p
    lib = _lib.lib()
    with AttentionAccelerator(batch=1, max_seq_len=L) as acc:
        kd = torch.from_numpy(kw.view(np.int16)).cuda()
        vd = torch.from_numpy(vw.view(np.int16)).cuda()
        qd = torch.from_numpy(q.view(np.int16)).cuda()
        lens = torch.tensor([L], dtype=torch.int32, device="cuda")
        k = torch.zeros_like(kd)
        v = torch.zeros_like(vd)
        od = torch.zeros_like(qd)
        torch.cuda.synchronize()
        print("[streams] default stream busy, then inputs written; library copy with stream NULL", flush=True)
        _busy_default_stream()
        k.copy_(kd)
        v.copy_(vd)
        _lib.check(lib.gqa_load_kv_device(acc._ctx, 0, 0, L, c(k.data_ptr()), c(v.data_ptr()), None), "load")
        _lib.check(lib.gqa_decode_device(acc._ctx, c(qd.data_ptr()), c(lens.data_ptr()), c(od.data_ptr()), None,
                                         None), "decode")
        o_first = od.clone()  # default-stream read right after the call
        torch.cuda.synchronize()
        kr, vr = acc.read_kv(0, 0, L)
    assert np.array_equal(kr, kw) and np.array_equal(vr, vw)
    o = o_first.cpu().numpy().view(np.uint16)
    ref, _ = orc.attention(orc.bf16_u16_to_fp32(q[0][:, None]), orc.bf16_u16_to_fp32(kw), orc.bf16_u16_to_fp32(vw),
                           causal=False)
    assert float(orc.row_ulp_error(o[0][:, None], ref).max()) <= 2.0


def test_device_entry_points_refuse_misaligned_vector_operands():
    # Q, appended K/V rows and the prefill output are moved in 16-byte vectors: a pointer off a
    # 16-byte boundary is refused on the host (GQA_ERR_RANGE) before anything is launched.
    c = ctypes.c_void_p
    lib = _lib.lib()
    with AttentionAccelerator(batch=2, max_seq_len=256, max_q_len=64) as acc:
        buf = torch.zeros(1 << 20, dtype=torch.int16, device="cuda")  # 256-byte aligned base
        ok, off = buf.data_ptr(), buf.data_ptr() + 8
        lens = torch.tensor([16, 16], dtype=torch.int32, device="cuda")
        pos = torch.tensor([15, 15], dtype=torch.int32, device="cuda")
        o = ok + (1 << 19)
        lp = c(lens.data_ptr())
        assert lib.gqa_decode_device(acc._ctx, c(off), lp, c(o), None, None) == _lib.GQA_ERR_RANGE
        assert lib.gqa_decode_append_device(acc._ctx, c(ok), c(off), c(ok), c(pos.data_ptr()), lp, c(o), None,
                                            None) == _lib.GQA_ERR_RANGE
        assert lib.gqa_prefill_device(acc._ctx, 0, c(ok), 16, 0, 16, 0, 1, c(o + 8), None, None) == _lib.GQA_ERR_RANGE
        assert lib.gqa_prefill_append_device(acc._ctx, 0, c(ok), c(ok), c(off), 16, 16, 0, 16, 0, 1, c(o), None,
                                             None) == _lib.GQA_ERR_RANGE
        # the aligned forms of the same calls run
        _lib.check(lib.gqa_decode_device(acc._ctx, c(ok), lp, c(o), None, None), "aligned decode")
        _lib.check(lib.gqa_prefill_device(acc._ctx, 0, c(ok), 16, 0, 16, 0, 1, c(o), None, None), "aligned prefill")
        torch.cuda.synchronize()
