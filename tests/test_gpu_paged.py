"""GPU parity of the paged K/V cache (gqa_create_paged).

A paged engine runs the same kernels as a contiguous one and only reads and writes through
the block tables, so on the same inputs every output word and every cache row must equal
the contiguous engine's (bit-exact), and the attention must be within 2 bf16 ulp per row of
the float64 oracle.  Pages are handed out interleaved across sequences and recycled, so a
sequence's rows are scattered over the pool and freed pages hold stale words.
"""
import ctypes

import numpy as np
import pytest

from lara_amd import _lib
from lara_amd.attn_driver import AttentionAccelerator
from oracle import gqa_oracle as orc
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu

P = 64
LENS = [1, 63, 64, 65, 700, 1500]
B = len(LENS)
L_MAX = 1536


def engines(**kw):
    cont = AttentionAccelerator(batch=B, max_seq_len=L_MAX, max_q_len=256, **kw)
    paged = AttentionAccelerator(batch=B, max_seq_len=L_MAX, max_q_len=256, page_size=P,
                                 n_pages=B * (L_MAX // P) + 4, **kw)
    return cont, paged


def scatter_reserve(acc, lens, step=P):
    """Grow every sequence one page at a time, round robin, so their pages interleave."""
    target = list(lens)
    grown = [0] * len(target)
    while any(g < t for g, t in zip(grown, target)):
        for b, t in enumerate(target):
            if grown[b] < t:
                grown[b] = min(t, grown[b] + step)
                acc.reserve(b, grown[b])


def fill(accs, rng, lens):
    ks, vs = [], []
    for b, L in enumerate(lens):
        k = bf16_normal(rng, (8, L, 128))
        v = bf16_normal(rng, (8, L, 128))
        for acc in accs:
            acc.load_kv(k, v, b=b)
        ks.append(k)
        vs.append(v)
    return ks, vs


def test_pages_are_scattered_and_recycled():
    _, paged = engines()
    with paged:
        scatter_reserve(paged, LENS)
        info = paged.page_info()
        assert info["page_size"] == P and info["max_pages"] == L_MAX // P
        tables = [paged.page_table(b) for b in range(B)]
        used = np.concatenate([t[t >= 0] for t in tables])
        assert len(used) == len(set(used.tolist())) == sum(-(-L // P) for L in LENS)
        assert info["free_pages"] == info["n_pages"] - len(used)
        assert any(np.any(np.diff(t[t >= 0]) != 1) for t in tables)  # not one contiguous run
        paged.release(4)
        assert np.all(paged.page_table(4) == -1)
        assert paged.page_info()["free_pages"] == info["free_pages"] + -(-LENS[4] // P)


def test_decode_paged_equals_contiguous_and_oracle():
    rng = np.random.default_rng(11)
    cont, paged = engines()
    with cont, paged:
        scatter_reserve(paged, LENS)
        ks, vs = fill([cont, paged], rng, LENS)
        q = bf16_normal(rng, (B, 32, 128))
        o_c, lse_c = cont.decode_step(q, LENS, return_lse=True)
        o_p, lse_p = paged.decode_step(q, LENS, return_lse=True)
        for b in range(B):
            kb, vb = paged.read_kv(b, 0, LENS[b])
            assert np.array_equal(kb, ks[b]) and np.array_equal(vb, vs[b])
    assert np.array_equal(o_p, o_c) and np.array_equal(lse_p, lse_c)
    for b, L in enumerate(LENS):
        ref, _ = orc.attention(orc.bf16_u16_to_fp32(q[b][:, None]), orc.bf16_u16_to_fp32(ks[b]),
                               orc.bf16_u16_to_fp32(vs[b]), causal=False)
        assert float(orc.row_ulp_error(o_p[b][:, None], ref).max()) <= 2.0


def test_fused_decode_append_over_a_page_boundary():
    """Rows 63, 64, 65 of a sequence cross from one page into the next."""
    rng = np.random.default_rng(12)
    lens = [63] * B
    cont, paged = engines()
    with cont, paged:
        scatter_reserve(paged, [66] * B)
        fill([cont, paged], rng, lens)
        for step in range(3):
            pos = np.full(B, 63 + step, np.int32)
            pos[1] = -1  # one sequence appends nothing
            q = bf16_normal(rng, (B, 32, 128))
            k = bf16_normal(rng, (B, 8, 128))
            v = bf16_normal(rng, (B, 8, 128))
            ctx = np.where(pos >= 0, pos + 1, 63 + step).astype(np.int32)
            o_c = cont.decode_step(q, ctx, k_rows=k, v_rows=v, positions=pos)
            o_p = paged.decode_step(q, ctx, k_rows=k, v_rows=v, positions=pos)
            assert np.array_equal(o_p, o_c), step
        for b in range(B):
            kc, vc = cont.read_kv(b, 0, 66)
            kp, vp = paged.read_kv(b, 0, 66)
            assert np.array_equal(kp, kc) and np.array_equal(vp, vc)


@pytest.mark.parametrize("kernel", ["auto", "shared", "paired"])
def test_chunked_prefill_into_pages(kernel):
    """Chunks of 256 rows take the row-block kernel (auto) or the GQA-shared one, unpaired or paired
    (forced): each reads the pages' block-table entries through the scalar cache."""
    rng = np.random.default_rng(13)
    prompt, chunk = 640, 256
    cont, paged = engines()
    code = {"auto": _lib.GQA_PREFILL_KERNEL_AUTO, "shared": _lib.GQA_PREFILL_KERNEL_SHARED,
            "paired": _lib.GQA_PREFILL_KERNEL_PAIRED}[kernel]
    with cont, paged:
        for acc in (cont, paged):
            _lib.check(acc._lib.gqa_set_option(acc._ctx, _lib.GQA_OPT_PREFILL_KERNEL, code), "prefill kernel")
        paged.reserve(2, prompt)
        paged.reserve(0, 3 * P)  # sequence 0 sits between sequence 2's pages
        paged.reserve(2, prompt)
        for start in range(0, prompt, chunk):
            n = min(chunk, prompt - start)
            q = bf16_normal(rng, (32, n, 128))
            k = bf16_normal(rng, (8, n, 128))
            v = bf16_normal(rng, (8, n, 128))
            kw = dict(b=2, q_pos_base=start, kv_len=start + n, causal=True, k_rows=k, v_rows=v, return_lse=True)
            o_c, l_c = cont.prefill_chunk(q, **kw)
            o_p, l_p = paged.prefill_chunk(q, **kw)
            assert np.array_equal(o_p, o_c) and np.array_equal(l_p, l_c), start
            if kernel != "auto":  # the forced decomposition ran, paired in one KV segment
                for acc in (cont, paged):
                    assert acc.last_prefill_plan()[0] == kernel
                    assert kernel != "paired" or acc.last_prefill_plan()[1] == 1
        kc, vc = cont.read_kv(2, 0, prompt)
        kp, vp = paged.read_kv(2, 0, prompt)
    assert np.array_equal(kp, kc) and np.array_equal(vp, vc)


def test_run_attention_and_layer_on_a_paged_engine():
    rng = np.random.default_rng(14)
    L = 200
    q = bf16_normal(rng, (32, L, 128))
    k = bf16_normal(rng, (8, L, 128))
    v = bf16_normal(rng, (8, L, 128))
    x = bf16_normal(rng, (L, 512))
    w = [bf16_normal(rng, (n, 512), 512 ** -0.5) for n in (4096, 1024, 1024)]
    with AttentionAccelerator() as cont, AttentionAccelerator(page_size=P) as paged:
        assert np.array_equal(paged.run_attention(q, k, v, q_pos_base=3, kv_pos_base=3),
                              cont.run_attention(q, k, v, q_pos_base=3, kv_pos_base=3))
        assert np.array_equal(paged.run_layer(x, *w, q_pos_base=1, kv_pos_base=1),
                              cont.run_layer(x, *w, q_pos_base=1, kv_pos_base=1))
        assert all(np.array_equal(a, b) for a, b in zip(paged.read_kv(0, 0, L), cont.read_kv(0, 0, L)))


def test_host_calls_refuse_unmapped_rows_and_the_pool_limit():
    rng = np.random.default_rng(15)
    with AttentionAccelerator(batch=3, max_seq_len=512, page_size=P, n_pages=6) as acc:
        acc.reserve(0, 100)  # 2 pages
        with pytest.raises(RuntimeError):  # rows 128..199 have no page
            acc.load_kv(bf16_normal(rng, (8, 200, 128)), bf16_normal(rng, (8, 200, 128)), b=0)
        with pytest.raises(RuntimeError):
            acc.decode_step(bf16_normal(rng, (3, 32, 128)), [129, 0, 0])
        with pytest.raises(MemoryError):
            acc.reserve(1, 5 * P)  # 5 pages > 4 free
        assert acc.page_info()["free_pages"] == 4 and np.all(acc.page_table(1) == -1)
        acc.reserve(1, 2 * P)
        acc.reserve(2, 2 * P)
        acc.reserve(0, 100)  # a use of sequence 0: sequence 1 is now the least recently used
        assert acc.evict_lru(2, pinned=[2]) == [1]
        with pytest.raises(MemoryError):
            acc.evict_lru(6, pinned=[0, 2])
        assert acc.evict_lru(6) == [2, 0]  # least recently used first
        assert acc.page_info()["free_pages"] == 6


def test_recycled_pages_hold_stale_words_that_never_leak():
    """A sequence that reuses another's freed pages attends only its own rows."""
    rng = np.random.default_rng(16)
    with AttentionAccelerator(batch=2, max_seq_len=512, page_size=P, n_pages=8) as acc:
        acc.reserve(0, 512)
        nan_rows = np.full((8, 512, 128), 0x7FC1, np.uint16)  # NaN words everywhere
        acc.load_kv(nan_rows, nan_rows, b=0)
        acc.release(0)
        L = 100  # inside the first two recycled pages; rows 100..127 still hold NaNs
        acc.reserve(1, L)
        k = bf16_normal(rng, (8, L, 128))
        v = bf16_normal(rng, (8, L, 128))
        acc.load_kv(k, v, b=1)
        q = bf16_normal(rng, (2, 32, 128))
        o = acc.decode_step(q, [0, L])
        q2 = bf16_normal(rng, (32, 40, 128))
        o2 = acc.prefill_chunk(q2, b=1, q_pos_base=L - 40, kv_len=L, causal=True)
    ref, _ = orc.attention(orc.bf16_u16_to_fp32(q[1][:, None]), orc.bf16_u16_to_fp32(k), orc.bf16_u16_to_fp32(v),
                           causal=False)
    assert float(orc.row_ulp_error(o[1][:, None], ref).max()) <= 2.0 and not o[0].any()
    ref2, _ = orc.attention(orc.bf16_u16_to_fp32(q2), orc.bf16_u16_to_fp32(k), orc.bf16_u16_to_fp32(v),
                            causal=True, q_pos_base=L - 40)
    assert float(orc.row_ulp_error(o2, ref2).max()) <= 2.0


def test_device_decode_reads_unmapped_pages_as_zero_rows():
    """The device form cannot validate device-resident lengths: rows of unmapped pages read as
    zeros (and the fused append skips them) instead of touching memory outside the pool."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(17)
    L_mapped, L_asked = 64, 130
    with AttentionAccelerator(batch=1, max_seq_len=256, page_size=P, n_pages=4) as acc:
        acc.reserve(0, L_mapped)
        k = bf16_normal(rng, (8, L_mapped, 128))
        v = bf16_normal(rng, (8, L_mapped, 128))
        acc.load_kv(k, v, b=0)
        q = bf16_normal(rng, (1, 32, 128))
        qd = torch.from_numpy(q.view(np.int16)).cuda()
        lens = torch.tensor([L_asked], dtype=torch.int32, device="cuda")
        od = torch.empty_like(qd)
        torch.cuda.synchronize()
        c = ctypes.c_void_p
        rc = _lib.lib().gqa_decode_device(acc._ctx, c(qd.data_ptr()), c(lens.data_ptr()), c(od.data_ptr()), None,
                                          None)
        assert rc == 0
        _lib.check(_lib.lib().gqa_synchronize(acc._ctx), "sync")
        o = od.cpu().numpy().view(np.uint16)
    kz = np.concatenate([k, np.zeros((8, L_asked - L_mapped, 128), np.uint16)], axis=1)
    vz = np.concatenate([v, np.zeros((8, L_asked - L_mapped, 128), np.uint16)], axis=1)
    ref, _ = orc.attention(orc.bf16_u16_to_fp32(q[0][:, None]), orc.bf16_u16_to_fp32(kz), orc.bf16_u16_to_fp32(vz),
                           causal=False)
    assert float(orc.row_ulp_error(o[0][:, None], ref).max()) <= 2.0
