"""GPU parity of K/V append and split-KV decode against the CPU oracle.

Tolerance (stated once, used everywhere): for every output row (one query head of one
sequence) the max abs error against the float64 oracle is <= 2 bf16 ulp of the row's
largest |output| ("2 bf16 ulp of output magnitude"); the softmax sum l, recovered from
the returned log-sum-exp, is within rtol 1e-2; K/V append and read-back are bit-exact.
"""
import ctypes

import numpy as np
import pytest

from lara_amd import _lib
from lara_amd.attn_driver import AttentionAccelerator
from oracle import gqa_oracle as orc
from tests._gen import bf16_normal, kv_with_outliers

pytestmark = pytest.mark.gpu

ULP_TOL = 2.0
L_RTOL = 1e-2


def make_engine(B, hq, hkv, d, max_len, **kw):
    print(f"[engine] B={B} Hq={hq} Hkv={hkv} D={d} L={max_len}", flush=True)
    return AttentionAccelerator(batch=B, n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=max_len,
                                max_q_len=kw.pop("max_q_len", min(max_len, 512)), **kw)


def check_decode(out, lse, q, kc, vc, lens, scale):
    ref, ref_lse = orc.decode(q, kc, vc, lens, scale=scale)
    err = orc.row_ulp_error(out, ref)
    worst = float(np.max(err))
    assert worst <= ULP_TOL, f"max row error {worst:.3f} bf16 ulp > {ULP_TOL}"
    if lse is not None:
        live = np.isfinite(ref_lse)
        assert np.array_equal(np.isneginf(lse), ~live)
        # l = exp(lse - m): compare the sums relative to a common max via the lse difference
        rel = np.abs(np.expm1(lse[live].astype(np.float64) - ref_lse[live]))
        assert float(rel.max(initial=0.0)) <= L_RTOL
    return worst


def fill_cache(eng, rng, B, hkv, d, lens, amp=1.0, outliers=(0.0, 1.0), lcap=None):
    lcap = lcap or int(max(lens.max(), 1))
    kc = np.zeros((B, hkv, lcap, d), np.uint16)
    vc = np.zeros((B, hkv, lcap, d), np.uint16)
    for b in range(B):
        n = int(lens[b])
        if n == 0:
            continue
        kc[b, :, :n] = kv_with_outliers(rng, (hkv, n, d), amp, *outliers)
        vc[b, :, :n] = bf16_normal(rng, (hkv, n, d), amp)
        eng.load_kv(kc[b, :, :n], vc[b, :, :n], b=b)
    return kc, vc


def test_append_and_load_bit_exact():
    rng = np.random.default_rng(100)
    B, hq, hkv, d, L = 3, 32, 8, 128, 300
    with make_engine(B, hq, hkv, d, L) as eng:
        k = rng.integers(0, 1 << 16, (hkv, 200, d), dtype=np.uint16)  # arbitrary words, NaN patterns included
        v = rng.integers(0, 1 << 16, (hkv, 200, d), dtype=np.uint16)
        eng.load_kv(k, v, b=1, start_pos=50)
        kr, vr = eng.read_kv(1, 50, 200)
        assert np.array_equal(kr, k) and np.array_equal(vr, v)
        rows_k = rng.integers(0, 1 << 16, (B, hkv, d), dtype=np.uint16)
        rows_v = rng.integers(0, 1 << 16, (B, hkv, d), dtype=np.uint16)
        eng.append_kv(rows_k, rows_v, np.array([7, 299, -1], np.int32))
        k0, v0 = eng.read_kv(0, 7, 1)
        assert np.array_equal(k0[:, 0], rows_k[0]) and np.array_equal(v0[:, 0], rows_v[0])
        k1, v1 = eng.read_kv(1, 299, 1)
        assert np.array_equal(k1[:, 0], rows_k[1]) and np.array_equal(v1[:, 0], rows_v[1])
        # untouched rows unchanged, skipped sequence unchanged
        kr, vr = eng.read_kv(1, 50, 200)
        assert np.array_equal(kr, k) and np.array_equal(vr, v)
        k2, v2 = eng.read_kv(2, 0, 300)
        assert not k2.any() and not v2.any()
        with pytest.raises(ValueError):
            eng.append_kv(rows_k, rows_v, np.array([0, 300, 0], np.int32))


def test_decode_c1_board_shape():
    # B1, 8q/2kv, D64, ctx 256, scale 1/8, no mask
    rng = np.random.default_rng(101)
    B, hq, hkv, d, L = 1, 8, 2, 64, 256
    with make_engine(B, hq, hkv, d, L, scale=0.125) as eng:
        lens = np.array([L], np.int32)
        kc, vc = fill_cache(eng, rng, B, hkv, d, lens)
        q = bf16_normal(rng, (B, hq, d))
        out, lse = eng.decode_step(q, lens, return_lse=True)
        check_decode(out, lse, q, kc, vc, lens, 0.125)


def test_decode_c2_append_then_attend():
    # B1, 32q/8kv, D128: 4096 cached rows, each step appends one and attends 4097.
    rng = np.random.default_rng(102)
    B, hq, hkv, d = 1, 32, 8, 128
    with make_engine(B, hq, hkv, d, 4200) as eng:
        lens = np.array([4096], np.int32)
        kc, vc = fill_cache(eng, rng, B, hkv, d, lens, amp=0.5, lcap=4200)
        for step in range(3):
            pos = 4096 + step
            nk = bf16_normal(rng, (B, hkv, d), 0.5)
            nv = bf16_normal(rng, (B, hkv, d), 0.5)
            eng.append_kv(nk, nv, np.array([pos], np.int32))
            kc[:, :, pos], vc[:, :, pos] = nk, nv
            q = bf16_normal(rng, (B, hq, d), 0.5)
            cur = np.array([pos + 1], np.int32)
            out, lse = eng.decode_step(q, cur, return_lse=True)
            check_decode(out, lse, q, kc, vc, cur, None)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 8, 128), (64, 4, 128), (16, 4, 64), (32, 4, 64)])
def test_decode_ragged_edges(hq, hkv, d):
    # lengths at round (16), chunk (256) and empty boundaries
    rng = np.random.default_rng(hq + hkv + d)
    lens = np.array([0, 1, 15, 16, 17, 255, 256, 257, 1000, 2049], np.int32)
    B = len(lens)
    with make_engine(B, hq, hkv, d, 2100) as eng:
        kc, vc = fill_cache(eng, rng, B, hkv, d, lens, lcap=2100)
        q = bf16_normal(rng, (B, hq, d))
        out, lse = eng.decode_step(q, lens, return_lse=True)
        check_decode(out, lse, q, kc, vc, lens, None)
        assert not out[0].any()


@pytest.mark.parametrize("B", [64, 65, 200])
def test_decode_longest_first_order_is_invisible(B):
    # Sequences are dispatched longest first, ranked inside the kernel: exactly up to 64 sequences
    # (ties in index order), by length bucket above.  Either way every sequence's output must be
    # the oracle's, and word for word the same when the batch is listed in another order.
    rng = np.random.default_rng(600 + B)
    hq, hkv, d = 32, 8, 128
    lens = rng.choice(np.array([0, 1, 16, 17, 100, 256, 257, 300, 511, 600], np.int32), size=B)
    lens[:4] = 600  # ties at the top
    with make_engine(B, hq, hkv, d, 640) as eng:
        kc, vc = fill_cache(eng, rng, B, hkv, d, lens, lcap=640)
        q = bf16_normal(rng, (B, hq, d))
        out, lse = eng.decode_step(q, lens, return_lse=True)
        check_decode(out, lse, q, kc, vc, lens, None)
    perm = rng.permutation(B)
    with make_engine(B, hq, hkv, d, 640) as eng:
        for i, b in enumerate(perm):
            if lens[b]:
                eng.load_kv(kc[b, :, :lens[b]], vc[b, :, :lens[b]], b=i)
        out_p, lse_p = eng.decode_step(q[perm], lens[perm], return_lse=True)
    assert np.array_equal(out_p, out[perm])
    assert np.array_equal(lse_p, lse[perm])


def test_decode_ragged_rows_by_ticket_over_repeated_steps():
    """A ragged batch of one split per (sequence, kv head) takes its rows from a counter that the
    launch's last taker resets: repeated steps, with steps of an equal-length batch (rows in grid
    order, counter untouched) between them, give the same words every time, and the oracle's."""
    rng = np.random.default_rng(611)
    B, hq, hkv, d = 64, 32, 8, 128
    lens = rng.integers(1, 600, size=B).astype(np.int32)
    lens[[3, 40]] = 600
    lens[7] = 0
    with make_engine(B, hq, hkv, d, 640) as eng:
        kc, vc = fill_cache(eng, rng, B, hkv, d, lens, lcap=640)
        q = bf16_normal(rng, (B, hq, d))
        out0, lse0 = eng.decode_step(q, lens, return_lse=True)
        check_decode(out0, lse0, q, kc, vc, lens, None)
        even = np.full(B, 500, np.int32)
        even_out = None
        for step in range(4):
            out, lse = eng.decode_step(q, lens, return_lse=True)
            assert np.array_equal(out, out0), f"ragged step {step}"
            assert np.array_equal(lse.view(np.uint32), lse0.view(np.uint32))
            out_e = eng.decode_step(q, even)
            if even_out is None:
                even_out = out_e
                check_decode(out_e, None, q, kc, vc, even, None)
            assert np.array_equal(out_e, even_out), f"equal-length step {step}"


def test_decode_split_invariance():
    rng = np.random.default_rng(103)
    B, hq, hkv, d = 2, 32, 8, 128
    lens = np.array([3000, 1777], np.int32)
    with make_engine(B, hq, hkv, d, 3072) as eng:
        kc, vc = fill_cache(eng, rng, B, hkv, d, lens, lcap=3072)
        q = bf16_normal(rng, (B, hq, d))
        outs = []
        for chunk in (256, 512, 1024, 3072, 0):
            _lib.check(eng._lib.gqa_set_option(eng._ctx, _lib.GQA_OPT_DECODE_CHUNK, chunk), "set chunk")
            out, lse = eng.decode_step(q, lens, return_lse=True)
            check_decode(out, lse, q, kc, vc, lens, None)
            outs.append(out)
        # different split counts differ by at most the rounding of the final bf16
        for o in outs[1:]:
            diff = np.abs(orc.bf16_u16_to_fp32(o).astype(np.float64) - orc.bf16_u16_to_fp32(outs[0]))
            assert float(diff.max()) <= float(orc.bf16_ulp(np.abs(orc.bf16_u16_to_fp32(outs[0])).max()))


def test_decode_group8_outliers():
    # Long-context shape (64q/8kv, 1% of K rows x8) at a length the oracle checks in seconds
    rng = np.random.default_rng(104)
    B, hq, hkv, d, L = 2, 64, 8, 128, 20000
    with make_engine(B, hq, hkv, d, L) as eng:
        lens = np.array([L, 12345], np.int32)
        kc, vc = fill_cache(eng, rng, B, hkv, d, lens, outliers=(0.01, 8.0), lcap=L)
        q = bf16_normal(rng, (B, hq, d))
        out, lse = eng.decode_step(q, lens, return_lse=True)
        check_decode(out, lse, q, kc, vc, lens, None)


def test_decode_constant_v_is_exact():
    # softmax weights sum to 1: a constant V row must come back exactly
    rng = np.random.default_rng(105)
    B, hq, hkv, d, L = 2, 32, 8, 128, 5000
    with make_engine(B, hq, hkv, d, L) as eng:
        for b in range(B):
            k = bf16_normal(rng, (hkv, L, d))
            v = np.broadcast_to(bf16_normal(rng, (hkv, 1, d)), (hkv, L, d)).copy()
            eng.load_kv(k, v, b=b)
            if b == 0:
                v0 = v[:, 0]
        q = bf16_normal(rng, (B, hq, d))
        out = eng.decode_step(q, np.array([L, L], np.int32))
        assert np.array_equal(out[0], np.repeat(v0, hq // hkv, axis=0))


def _full_size(name, page_size=0):
    from lara_amd.benchmark import WORKLOADS
    w = WORKLOADS[name]
    rng = np.random.default_rng(w.seed)
    lens = w.lengths()
    paged = dict(page_size=page_size, n_pages=int(sum(-(-int(n) // page_size) for n in lens)) + 1) if page_size else {}
    with make_engine(w.batch, w.n_q_heads, w.n_kv_heads, w.head_dim, int(lens.max()), max_q_len=1,
                     scale=w.scale, **paged) as eng:
        if page_size:  # every sequence grows a page at a time, round robin: their pages interleave
            grown = [0] * w.batch
            while any(g < n for g, n in zip(grown, lens)):
                for b, n in enumerate(lens):
                    if grown[b] < n:
                        grown[b] = min(int(n), grown[b] + page_size)
                        eng.reserve(b, grown[b])
        kc, vc = fill_cache(eng, rng, w.batch, w.n_kv_heads, w.head_dim, lens, w.amplitude,
                            (w.outlier_fraction, w.outlier_scale))
        q = bf16_normal(rng, (w.batch, w.n_q_heads, w.head_dim), w.amplitude)
        print(f"[{name}] decode", flush=True)
        out, lse = eng.decode_step(q, lens, return_lse=True)
        print(f"[{name}] oracle check", flush=True)
        worst = check_decode(out, lse, q, kc, vc, lens, w.scale)
        print(f"[{name}] worst row error {worst:.3f} ulp", flush=True)


def test_decode_full_size_ns():
    _full_size("decode-b64-ctx8192")


def test_decode_full_size_ns_on_scattered_pages():
    """The north-star decode on a paged cache of 64-row pages, every sequence's pages interleaved
    with the others' (the bench's NS-paged line), against the oracle at full size."""
    _full_size("decode-b64-ctx8192", page_size=64)


def test_decode_full_size_c3_ragged():
    _full_size("decode-b64-ragged")


def test_decode_full_size_c4_long_context():
    _full_size("decode-b4-ctx131072")


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (64, 8, 128), (16, 8, 64)])
def test_fused_append_decode_matches_two_launches(hq, hkv, d):
    """decode_step with rows = append_kv + decode_step, bit for bit, over repeated steps.

    A small split size gives many splits per sequence, so every step exercises the
    combine launch and the split that reads the appended row from k_new/v_new.
    """
    rng = np.random.default_rng(200 + hq + d)
    B = 3
    lens = np.array([700, 1, 1500], np.int32)
    cap = 1600
    with make_engine(B, hq, hkv, d, cap) as fused, make_engine(B, hq, hkv, d, cap) as split:
        kc, vc = fill_cache(fused, rng, B, hkv, d, lens, lcap=cap)
        for b in range(B):
            split.load_kv(kc[b, :, :lens[b]], vc[b, :, :lens[b]], b=b)
        for eng in (fused, split):
            _lib.check(eng._lib.gqa_set_option(eng._ctx, _lib.GQA_OPT_DECODE_CHUNK, 256), "chunk")
        cur = lens.copy()
        for step in range(4):
            nk = bf16_normal(rng, (B, hkv, d))
            nv = bf16_normal(rng, (B, hkv, d))
            pos = cur.copy()
            pos[1] = -1 if step == 2 else pos[1]  # a sequence that skips the append this step
            q = bf16_normal(rng, (B, hq, d))
            attend = np.where(pos >= 0, pos + 1, cur).astype(np.int32)
            out_f, lse_f = fused.decode_step(q, attend, k_rows=nk, v_rows=nv, positions=pos, return_lse=True)
            split.append_kv(nk, nv, pos)
            out_s, lse_s = split.decode_step(q, attend, return_lse=True)
            assert np.array_equal(out_f, out_s)
            assert np.array_equal(lse_f.view(np.uint32), lse_s.view(np.uint32))
            for b in range(B):
                if pos[b] >= 0:
                    kc[b, :, pos[b]], vc[b, :, pos[b]] = nk[b], nv[b]
                    kr, vr = fused.read_kv(b, int(pos[b]), 1)
                    assert np.array_equal(kr[:, 0], nk[b]) and np.array_equal(vr[:, 0], nv[b])
            check_decode(out_f, lse_f, q, kc, vc, attend, None)
            cur = attend


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (64, 8, 128)])
def test_decode_fused_merge_matches_merge_launch(hq, hkv, d):
    """The in-launch merge (last split to arrive) and the separate merge launch fold the same
    partials in the same order: equal words and LSE, over repeated steps (the arrival counters
    reset themselves) with sequences of one split, several splits and no key."""
    rng = np.random.default_rng(300 + hq)
    B = 4
    lens = np.array([3000, 129, 0, 2049], np.int32)
    cap = 3072
    with make_engine(B, hq, hkv, d, cap) as fused, make_engine(B, hq, hkv, d, cap) as launch:
        kc, vc = fill_cache(fused, rng, B, hkv, d, lens, lcap=cap)
        for b in range(B):
            if lens[b]:
                launch.load_kv(kc[b, :, :lens[b]], vc[b, :, :lens[b]], b=b)
        _lib.check(fused._lib.gqa_set_option(fused._ctx, _lib.GQA_OPT_DECODE_MERGE, _lib.GQA_DECODE_MERGE_FUSED), "m")
        _lib.check(launch._lib.gqa_set_option(launch._ctx, _lib.GQA_OPT_DECODE_MERGE, _lib.GQA_DECODE_MERGE_LAUNCH),
                   "m")
        for eng in (fused, launch):
            _lib.check(eng._lib.gqa_set_option(eng._ctx, _lib.GQA_OPT_DECODE_CHUNK, 256), "chunk")
        for step in range(3):
            q = bf16_normal(rng, (B, hq, d))
            out_f, lse_f = fused.decode_step(q, lens, return_lse=True)
            out_l, lse_l = launch.decode_step(q, lens, return_lse=True)
            assert np.array_equal(out_f, out_l), f"step {step}"
            assert np.array_equal(lse_f.view(np.uint32), lse_l.view(np.uint32))
            check_decode(out_f, lse_f, q, kc, vc, lens, None)


def test_decode_cancelling_v_rows_within_the_weight_rounding_bound():
    """V rows in cancelling pairs with near-equal weights: the products take P rounded to bf16 (as the
    board takes it truncated), so each element is within 2 bf16 ulp of its row's largest |output|
    plus 2^-8 of attention over |V| at that element (oracle.weight_rounding_error), the stated bound
    of the EXACT mode; the softmax sum stays within rtol 1e-2."""
    from tests._gen import cancelling_kv

    rng = np.random.default_rng(160)
    B, hq, hkv, d = 2, 32, 8, 128
    lens = np.array([64, 300], np.int32)
    with make_engine(B, hq, hkv, d, 300) as eng:
        kc = np.zeros((B, hkv, 300, d), np.uint16)
        vc = np.zeros((B, hkv, 300, d), np.uint16)
        for b in range(B):
            kc[b, :, :lens[b]], vc[b, :, :lens[b]] = cancelling_kv(rng, hkv, int(lens[b]), d)
            eng.load_kv(kc[b, :, :lens[b]], vc[b, :, :lens[b]], b=b)
        q = bf16_normal(rng, (B, hq, d))
        out, lse = eng.decode_step(q, lens, return_lse=True)
    ref, ref_lse = orc.decode(q, kc, vc, lens)
    ref_abs, _ = orc.decode(q, kc, vc & np.uint16(0x7FFF), lens)
    err = orc.weight_rounding_error(out, ref, ref_abs)
    print(f"[cancel] decode: bound use {err.max():.3f}, 2-ulp measure {orc.row_ulp_error(out, ref).max():.2f}",
          flush=True)
    assert float(err.max()) <= 1.0
    rel = np.abs(np.expm1(lse.astype(np.float64) - ref_lse))
    assert float(rel.max()) <= L_RTOL


def _merge_launches(eng):
    counts = (ctypes.c_int32 * _lib.GQA_TIMER_COUNT)()
    _lib.check(eng._lib.gqa_kernel_launch_counts(eng._ctx, counts, _lib.GQA_TIMER_COUNT), "counts")
    return int(counts[_lib.GQA_TIMER_COMBINE]), int(counts[_lib.GQA_TIMER_DECODE])


@pytest.mark.parametrize("B,hq,hkv,d,L,twice", [(1, 32, 8, 128, 4097, True), (2, 32, 8, 128, 2049, True),
                                                (4, 32, 8, 128, 1025, True), (8, 32, 8, 128, 513, True),
                                                (1, 32, 8, 128, 2049, False), (1, 8, 2, 64, 2049, False)])
def test_decode_auto_plan_merges_small_grids_in_launch(B, hq, hkv, d, L, twice):
    """Small split grids under GQA_DECODE_MERGE_AUTO on 256 CUs: up to 16 splits within half the CUs
    merge inside the decode launch, and a plan of the shortest splits (128 keys) that would need the
    merge launch takes 256-key splits instead ("twice"), equal word for word to those splits merged by
    the merge launch.  Every step is checked against the oracle."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(700 + B * 10 + d + L)
    lens = np.full(B, L, np.int32)
    lens[-1] = L - 37 if B > 1 else L  # one shorter sequence: its split count differs
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    with make_engine(B, hq, hkv, d, L) as auto, make_engine(B, hq, hkv, d, L) as ref:
        kc, vc = fill_cache(auto, rng, B, hkv, d, lens, lcap=L)
        for b in range(B):
            ref.load_kv(kc[b, :, :lens[b]], vc[b, :, :lens[b]], b=b)
        _lib.check(ref._lib.gqa_set_option(ref._ctx, _lib.GQA_OPT_DECODE_MERGE, _lib.GQA_DECODE_MERGE_LAUNCH), "m")
        _lib.check(ref._lib.gqa_set_option(ref._ctx, _lib.GQA_OPT_DECODE_CHUNK, 256), "chunk")
        _lib.check(auto._lib.gqa_set_option(auto._ctx, _lib.GQA_OPT_PROFILE, 1), "profile")
        for step in range(2):
            q = bf16_normal(rng, (B, hq, d))
            out_a, lse_a = auto.decode_step(q, lens, return_lse=True)
            check_decode(out_a, lse_a, q, kc, vc, lens, None)
            if twice and n_cu == 256:
                out_r, lse_r = ref.decode_step(q, lens, return_lse=True)
                assert np.array_equal(out_a, out_r), f"step {step}"
                assert np.array_equal(lse_a.view(np.uint32), lse_r.view(np.uint32))
        merges, decodes = _merge_launches(auto)
        assert decodes == 2
        if n_cu == 256:
            assert merges == 0, "the automatic plan took the merge launch"
