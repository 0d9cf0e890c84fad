"""GPU parity of the MFMA prefill path (run_attention transactions and chunked prefill).

Tolerance, as for decode: every output row (one query head, one query position) is within
2 bf16 ulp of the row's largest |output| of the float64 oracle; the softmax sum l, recovered
from the returned log-sum-exp, is within rtol 1e-2; rows with no valid key are exactly zero.
"""
import numpy as np
import pytest

from lara_amd import attn_driver as drv
from lara_amd.attn_driver import AttentionAccelerator
from oracle import gqa_oracle as orc
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu

ULP_TOL = 2.0
L_RTOL = 1e-2


def check_rows(out_words, lse, ref, ref_lse):
    err = orc.row_ulp_error(out_words, ref)
    worst = float(np.max(err)) if err.size else 0.0
    assert worst <= ULP_TOL, f"max row error {worst:.3f} bf16 ulp > {ULP_TOL}"
    if lse is not None:
        live = np.isfinite(ref_lse)
        assert np.array_equal(np.isneginf(lse), ~live)
        rel = np.abs(np.expm1(lse[live].astype(np.float64) - ref_lse[live]))
        assert float(rel.max(initial=0.0)) <= L_RTOL
    return worst


def oracle_for(q, k, v, **kw):
    return orc.attention(orc.bf16_u16_to_fp32(q), orc.bf16_u16_to_fp32(k), orc.bf16_u16_to_fp32(v), **kw)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("L,qb,kb", [(1, 0, 0), (16, 0, 0), (32, 3, 3), (64, 31, 7), (128, 0, 0), (200, 5, 9),
                                     (512, 0, 0)])
def test_run_attention_board_contract(L, qb, kb, causal):
    """sw/attn_driver.py:469-550 at the KV260 shape: Q [32, L, 128], K/V [8, L, 128]."""
    print(f"[run_attention] L={L} q_pos_base={qb} kv_pos_base={kb} causal={causal}", flush=True)
    rng = np.random.default_rng(1000 + L + qb + kb + causal)
    q = bf16_normal(rng, (32, L, 128))
    k = bf16_normal(rng, (8, L, 128))
    v = bf16_normal(rng, (8, L, 128))
    with AttentionAccelerator() as acc:
        out = acc.run_attention(q, k, v, seq_len=L, q_pos_base=qb, kv_pos_base=kb, causal=causal)
        assert out.dtype == np.uint16 and out.shape == (32, L, 128)
        prof = acc.last_profile.to_dict()
        assert prof["seq_len"] == L and prof["attention_total_ms"] > 0
    ref, _ = oracle_for(q, k, v, causal=causal, q_pos_base=qb, kv_pos_base=kb)
    check_rows(out, None, ref, None)


def test_run_attention_float_inputs_are_packed_like_the_board():
    rng = np.random.default_rng(7)
    L = 48
    qf = rng.standard_normal((32, L, 128)).astype(np.float32)
    kf = rng.standard_normal((8, L, 128)).astype(np.float32)
    vf = rng.standard_normal((8, L, 128)).astype(np.float32)
    with AttentionAccelerator() as acc:
        out_f = acc.run_attention(qf, kf, vf, causal=True)
        out_w = acc.run_attention(drv.fp32_to_bf16_u16(qf), drv.fp32_to_bf16_u16(kf), drv.fp32_to_bf16_u16(vf),
                                  causal=True)
    assert np.array_equal(out_f, out_w)


def test_zero_input_gives_zero_output():
    """Board smoke test (sw/board_test.py:44-48): all-zero Q/K/V must give all-zero O."""
    L = 64
    with AttentionAccelerator() as acc:
        z = np.zeros((32, L, 128), np.uint16)
        zk = np.zeros((8, L, 128), np.uint16)
        out = acc.run_attention(z, zk, zk, causal=True)
    assert not out.any()


def test_transaction_protocol_and_busy_start():
    rng = np.random.default_rng(8)
    L = 96
    q = bf16_normal(rng, (32, L, 128))
    k = bf16_normal(rng, (8, L, 128))
    v = bf16_normal(rng, (8, L, 128))
    with AttentionAccelerator() as acc:
        acc.load_kv(k, v)
        acc.submit_query(q, kv_len=L, causal=False)
        assert acc.status() & drv.STATUS_START_READY
        acc.start()
        acc.wait_done(q, k, v, L, timeout_ms=10000)
        assert acc.status() & drv.STATUS_DONE
        out = acc.read_output()
        perf = acc.read_perf()
        assert perf["cycles"] >= perf["mac_cycles"] > 0
        with pytest.raises(RuntimeError):
            acc.readback_o(L + 1)  # CSR_RESULT_LEN mismatch
    ref, _ = oracle_for(q, k, v, causal=False)
    check_rows(out, None, ref, None)


def set_prefill_kernel(acc, kernel):
    """Force the prefill decomposition: 'auto', 'shared' (GQA-shared tiles + KV segments), 'rows' or
    'paired' (shared tiles, a long and a short causal row block per work-group)."""
    from lara_amd import _lib
    code = {"auto": _lib.GQA_PREFILL_KERNEL_AUTO, "shared": _lib.GQA_PREFILL_KERNEL_SHARED,
            "rows": _lib.GQA_PREFILL_KERNEL_ROWS, "paired": _lib.GQA_PREFILL_KERNEL_PAIRED}[kernel]
    _lib.check(acc._lib.gqa_set_option(acc._ctx, _lib.GQA_OPT_PREFILL_KERNEL, code), "prefill kernel")


@pytest.mark.parametrize("kernel", ["auto", "shared"])
def test_chunked_prefill_c5(kernel):
    """2048-token prompt in 256-token chunks against a growing cache, causal (32q/8kv, D 128)."""
    rng = np.random.default_rng(5)
    P, C = 2048, 256
    q = bf16_normal(rng, (32, P, 128))
    k = bf16_normal(rng, (8, P, 128))
    v = bf16_normal(rng, (8, P, 128))
    with AttentionAccelerator(max_seq_len=P, max_q_len=C) as acc:
        set_prefill_kernel(acc, kernel)
        for c in range(P // C):
            s = c * C
            print(f"[c5] chunk {c}", flush=True)
            acc.load_kv(k[:, s:s + C], v[:, s:s + C], start_pos=s)
            out, lse = acc.prefill_chunk(q[:, s:s + C], q_pos_base=s, kv_len=s + C, causal=True, return_lse=True)
            ref, ref_lse = oracle_for(q[:, s:s + C], k[:, :s + C], v[:, :s + C], causal=True, q_pos_base=s)
            check_rows(out, lse, ref, ref_lse)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 128), (16, 8, 128), (64, 8, 128), (64, 4, 128),
                                      (8, 2, 64), (16, 16, 64), (32, 4, 64), (32, 2, 64)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("kernel", ["rows", "shared"])
def test_prefill_shapes_ragged(hq, hkv, d, causal, kernel):
    """Every compiled (head_dim, group), ragged q_len / kv_len, absolute position bases, both
    decompositions."""
    rng = np.random.default_rng(hq * 7 + hkv * 3 + d + causal)
    q_len, kv_len, qb, kb = 77, 333, 300, 40
    print(f"[prefill] hq={hq} hkv={hkv} d={d} causal={causal} kernel={kernel}", flush=True)
    q = bf16_normal(rng, (hq, q_len, d))
    k = bf16_normal(rng, (hkv, kv_len, d))
    v = bf16_normal(rng, (hkv, kv_len, d))
    with AttentionAccelerator(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=kv_len, max_q_len=q_len) as acc:
        set_prefill_kernel(acc, kernel)
        acc.load_kv(k, v)
        out, lse = acc.prefill_chunk(q, q_pos_base=qb, kv_len=kv_len, kv_pos_base=kb, causal=causal,
                                     return_lse=True)
    ref, ref_lse = oracle_for(q, k, v, causal=causal, q_pos_base=qb, kv_pos_base=kb)
    check_rows(out, lse, ref, ref_lse)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 128), (16, 8, 128), (64, 8, 128), (64, 4, 128),
                                      (8, 2, 64), (16, 16, 64), (32, 4, 64), (32, 2, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_shared_one_segment_every_group(hq, hkv, d, causal):
    """The GQA-shared kernel writing its rows itself (one KV segment: rows staged in the free ring
    stages and stored whole) for every compiled (head_dim, group): ragged q_len (a partial last row
    block), work-groups whose last waves have no task (group 1 and 2), position bases."""
    rng = np.random.default_rng(hq * 11 + hkv * 5 + d + causal)
    q_len, kv_len, qb, kb = 77, 333, 300, 40
    print(f"[shared, one segment] hq={hq} hkv={hkv} d={d} causal={causal}", flush=True)
    q = bf16_normal(rng, (hq, q_len, d))
    k = bf16_normal(rng, (hkv, kv_len, d))
    v = bf16_normal(rng, (hkv, kv_len, d))
    with AttentionAccelerator(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=kv_len, max_q_len=q_len) as acc:
        set_prefill_kernel(acc, "shared")
        drv._lib.check(acc._lib.gqa_set_option(acc._ctx, drv._lib.GQA_OPT_PREFILL_WGS, 1), "wgs")
        acc.load_kv(k, v)
        out, lse = acc.prefill_chunk(q, q_pos_base=qb, kv_len=kv_len, kv_pos_base=kb, causal=causal,
                                     return_lse=True)
        assert acc.last_prefill_plan() == ("shared", 1)
    ref, ref_lse = oracle_for(q, k, v, causal=causal, q_pos_base=qb, kv_pos_base=kb)
    check_rows(out, lse, ref, ref_lse)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 4, 64)])
@pytest.mark.parametrize("q_len,kv_len,qb,kb", [(33, 33, 0, 0), (64, 64, 0, 0), (96, 96, 0, 0), (333, 333, 0, 0),
                                                (200, 700, 500, 0), (257, 300, 43, 0), (160, 230, 100, 30),
                                                (64, 200, 0, 150)])
def test_prefill_paired_causal(hq, hkv, d, q_len, kv_len, qb, kb):
    """Paired row blocks (group 4): work-group p owns row blocks n-1-p and p; the short block's waves
    move to the long block's keys at the first block past their own and the two halves of the long
    block merge in LDS.  Odd row-block counts (a work-group without a short block), a partial last
    row block, position bases (rows with no key, chunks after history) and a short block whose keys
    end in the long block's last block, against the oracle; the short blocks' rows are computed as
    by the unpaired kernel, word for word."""
    rng = np.random.default_rng(4000 + q_len + kv_len + qb + kb + d)
    print(f"[paired] hq={hq} hkv={hkv} d={d} q_len={q_len} kv_len={kv_len} qb={qb} kb={kb}", flush=True)
    q = bf16_normal(rng, (hq, q_len, d))
    k = bf16_normal(rng, (hkv, kv_len, d))
    v = bf16_normal(rng, (hkv, kv_len, d))
    outs = {}
    for kernel in ("paired", "shared"):
        with AttentionAccelerator(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=kv_len,
                                  max_q_len=q_len) as acc:
            set_prefill_kernel(acc, kernel)
            if kernel == "shared":  # the unpaired kernel in one KV segment, as the paired one runs
                drv._lib.check(acc._lib.gqa_set_option(acc._ctx, drv._lib.GQA_OPT_PREFILL_WGS, 1), "wgs")
            acc.load_kv(k, v)
            outs[kernel] = acc.prefill_chunk(q, q_pos_base=qb, kv_len=kv_len, kv_pos_base=kb, causal=True,
                                             return_lse=True)
            # the forced decomposition is the one that ran, in one KV segment
            assert acc.last_prefill_plan() == (kernel, 1)
    ref, ref_lse = oracle_for(q, k, v, causal=True, q_pos_base=qb, kv_pos_base=kb)
    check_rows(*outs["paired"], ref, ref_lse)
    short = (q_len // 32 + (q_len % 32 > 0)) // 2 * 32  # rows of the short row blocks
    assert np.array_equal(outs["paired"][0][:, :short], outs["shared"][0][:, :short])
    assert np.array_equal(outs["paired"][1][:, :short], outs["shared"][1][:, :short])


@pytest.mark.parametrize("P", [1024, 1536, 2048])
def test_prefill_whole_causal_prompt_pairs_by_default(P):
    """A whole causal prompt of 1024-2048 tokens (32q/8kv, D 128: 128-256 work-groups, one dispatch
    round) takes the paired kernel under AUTO; against the oracle, with fused append of its rows."""
    rng = np.random.default_rng(4100 + P)
    q = bf16_normal(rng, (32, P, 128))
    k = bf16_normal(rng, (8, P, 128))
    v = bf16_normal(rng, (8, P, 128))
    with AttentionAccelerator(max_seq_len=P, max_q_len=P) as acc:
        out, lse = acc.prefill_chunk(q, q_pos_base=0, kv_len=P, causal=True, k_rows=k, v_rows=v, return_lse=True)
        assert acc.last_prefill_plan() == ("paired", 1)
        kr, vr = acc.read_kv(0, 0, P)
    assert np.array_equal(kr, k) and np.array_equal(vr, v)
    ref, ref_lse = oracle_for(q, k, v, causal=True)
    check_rows(out, lse, ref, ref_lse)


@pytest.mark.parametrize("paged", [False, True])
def test_prefill_chunk_after_history_pairs_when_the_grid_fills_the_gpu(paged):
    """A causal 2048-row chunk after 192 cached rows (32q/8kv, D 128): its shared grid is one
    work-group per CU, so AUTO takes the paired kernel in one segment although earlier keys exist;
    against the oracle, and on a paged cache (scattered pages) word for word equal to the contiguous
    engine."""
    rng = np.random.default_rng(4200)
    H, C = 192, 2048
    q = bf16_normal(rng, (32, C, 128))
    k = bf16_normal(rng, (8, H + C, 128))
    v = bf16_normal(rng, (8, H + C, 128))
    outs = []
    for use_pages in ([False, True] if paged else [False]):
        kw = dict(page_size=64, n_pages=2 * (H + C) // 64 + 2, batch=2) if use_pages else {}
        with AttentionAccelerator(max_seq_len=H + C, max_q_len=C, **kw) as acc:
            b = 1 if use_pages else 0
            if use_pages:  # sequence 1's pages alternate with sequence 0's
                for n in range(64, H + C + 1, 64):
                    acc.reserve(0, n)
                    acc.reserve(1, n)
            acc.load_kv(k[:, :H], v[:, :H], b=b)
            print(f"[paired-after-history] paged={use_pages}", flush=True)
            outs.append(acc.prefill_chunk(q, b=b, q_pos_base=H, kv_len=H + C, causal=True, k_rows=k[:, H:],
                                          v_rows=v[:, H:], return_lse=True))
            assert acc.last_prefill_plan() == ("paired", 1)
    if paged:
        assert np.array_equal(outs[1][0], outs[0][0]) and np.array_equal(outs[1][1], outs[0][1])
    else:
        ref, ref_lse = oracle_for(q, k, v, causal=True, q_pos_base=H)
        check_rows(*outs[0], ref, ref_lse)


def test_one_causal_8192_token_prompt_sampled_rows():
    """One causal prefill launch over an 8192-token prompt already in the cache (32q/8kv, D 128: the
    bench's one-shot shape, several dispatch rounds of the GQA-shared kernel): rows at the start, at
    the middle and at the end of the prompt, every query head, against the float64 oracle over all
    their keys; every output row finite."""
    rng = np.random.default_rng(8192)
    P = 8192
    q = bf16_normal(rng, (32, P, 128))
    k = bf16_normal(rng, (8, P, 128))
    v = bf16_normal(rng, (8, P, 128))
    with AttentionAccelerator(max_seq_len=P, max_q_len=P) as acc:
        acc.load_kv(k, v)
        print("[p8k] one causal launch over 8192 rows", flush=True)
        out, lse = acc.prefill_chunk(q, q_pos_base=0, kv_len=P, causal=True, return_lse=True)
        print(f"[p8k] plan {acc.last_prefill_plan()}", flush=True)
    assert np.isfinite(orc.bf16_u16_to_fp32(out)).all() and np.isfinite(lse).all()
    for r0 in (0, 4064, 8128):  # 64 rows each: the first blocks, a middle pair of blocks, the last
        ref, ref_lse = oracle_for(q[:, r0:r0 + 64], k[:, :r0 + 64], v[:, :r0 + 64], causal=True, q_pos_base=r0)
        check_rows(out[:, r0:r0 + 64], lse[:, r0:r0 + 64], ref, ref_lse)


def test_prefill_rows_without_keys_are_zero():
    rng = np.random.default_rng(9)
    q_len, kv_len = 50, 120
    q = bf16_normal(rng, (32, q_len, 128))
    k = bf16_normal(rng, (8, kv_len, 128))
    v = bf16_normal(rng, (8, kv_len, 128))
    with AttentionAccelerator(max_seq_len=kv_len, max_q_len=q_len) as acc:
        acc.load_kv(k, v)
        # queries at positions 0..49, keys at 20..139: rows 0..19 see no key
        out, lse = acc.prefill_chunk(q, q_pos_base=0, kv_len=kv_len, kv_pos_base=20, causal=True, return_lse=True)
    assert not out[:, :20].any() and np.all(np.isneginf(lse[:, :20]))
    ref, ref_lse = oracle_for(q, k, v, causal=True, q_pos_base=0, kv_pos_base=20)
    check_rows(out, lse, ref, ref_lse)


def test_prefill_stale_cache_rows_do_not_leak():
    """Rows past kv_len hold NaN words; the result must not see them."""
    rng = np.random.default_rng(10)
    q_len, kv_len = 40, 70
    q = bf16_normal(rng, (32, q_len, 128))
    k = bf16_normal(rng, (8, kv_len, 128))
    v = bf16_normal(rng, (8, kv_len, 128))
    nan = np.full((8, 58, 128), 0x7FC0, np.uint16)
    with AttentionAccelerator(max_seq_len=128, max_q_len=q_len) as acc:
        acc.load_kv(nan, nan, start_pos=70)
        acc.load_kv(k, v)
        out = acc.prefill_chunk(q, q_pos_base=kv_len - q_len, kv_len=kv_len, causal=True)
    ref, _ = oracle_for(q, k, v, causal=True, q_pos_base=kv_len - q_len)
    check_rows(out, None, ref, None)


def test_single_row_prefill_matches_decode():
    rng = np.random.default_rng(11)
    L = 700
    k = bf16_normal(rng, (8, L, 128))
    v = bf16_normal(rng, (8, L, 128))
    q = bf16_normal(rng, (32, 1, 128))
    with AttentionAccelerator(max_seq_len=L, max_q_len=1) as acc:
        acc.load_kv(k, v)
        pre, lse_p = acc.prefill_chunk(q, q_pos_base=L - 1, kv_len=L, causal=True, return_lse=True)
        dec, lse_d = acc.decode_step(q[:, 0][None], np.array([L], np.int32), return_lse=True)
    ref, ref_lse = oracle_for(q, k, v, causal=False)
    check_rows(pre, lse_p, ref, ref_lse)
    check_rows(dec[0][:, None], lse_d[0][:, None], ref, ref_lse)


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 2, 64)])
@pytest.mark.parametrize("kernel", ["rows", "shared"])
def test_fused_chunk_append_matches_load_then_prefill(hq, hkv, d, kernel):
    """prefill_chunk with k_rows/v_rows = load_kv + prefill_chunk, bit for bit, chunk by chunk."""
    rng = np.random.default_rng(300 + hq + d)
    P, C = 700, 192  # the last chunk is partial
    q = bf16_normal(rng, (hq, P, d))
    k = bf16_normal(rng, (hkv, P, d))
    v = bf16_normal(rng, (hkv, P, d))
    kw = dict(n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=P, max_q_len=C)
    with AttentionAccelerator(**kw) as fused, AttentionAccelerator(**kw) as split:
        set_prefill_kernel(fused, kernel)
        set_prefill_kernel(split, kernel)
        for s in range(0, P, C):
            e = min(P, s + C)
            print(f"[fused chunk] {s}..{e}", flush=True)
            out_f, lse_f = fused.prefill_chunk(q[:, s:e], q_pos_base=s, kv_len=e, k_rows=k[:, s:e], v_rows=v[:, s:e],
                                               return_lse=True)
            split.load_kv(k[:, s:e], v[:, s:e], start_pos=s)
            out_s, lse_s = split.prefill_chunk(q[:, s:e], q_pos_base=s, kv_len=e, return_lse=True)
            assert np.array_equal(out_f, out_s)
            assert np.array_equal(lse_f.view(np.uint32), lse_s.view(np.uint32))
            kr, vr = fused.read_kv(0, s, e - s)
            assert np.array_equal(kr, k[:, s:e]) and np.array_equal(vr, v[:, s:e])
            ref, ref_lse = oracle_for(q[:, s:e], k[:, :e], v[:, :e], causal=True, q_pos_base=s)
            check_rows(out_f, lse_f, ref, ref_lse)


@pytest.mark.parametrize("wgs", [1, 64, 0, 4096])
def test_prefill_segmentation_invariance(wgs):
    """Results for any KV segmentation agree with the oracle (1 = one segment)."""
    rng = np.random.default_rng(400 + wgs)
    q_len, kv_len = 256, 1536
    q = bf16_normal(rng, (32, q_len, 128))
    k = bf16_normal(rng, (8, kv_len, 128))
    v = bf16_normal(rng, (8, kv_len, 128))
    with AttentionAccelerator(max_seq_len=kv_len, max_q_len=q_len) as acc:
        from lara_amd import _lib
        _lib.check(acc._lib.gqa_set_option(acc._ctx, _lib.GQA_OPT_PREFILL_WGS, wgs), "prefill wgs")
        acc.load_kv(k, v)
        out, lse = acc.prefill_chunk(q, q_pos_base=kv_len - q_len, kv_len=kv_len, return_lse=True)
    ref, ref_lse = oracle_for(q, k, v, causal=True, q_pos_base=kv_len - q_len)
    check_rows(out, lse, ref, ref_lse)


@pytest.mark.parametrize("v_scale", [1e30, 1e-30, 1e-39, "mixed", "weighted"])
def test_segment_partials_at_extreme_magnitudes(v_scale):
    """KV segments hand their rows to the merge as fp16 O / l divided by the row's largest
    |O / l|: outputs of very large or very small magnitude, and rows mixing both, keep the
    2-ulp bound with many segments."""
    seeds = {"mixed": 500, "weighted": 501}
    rng = np.random.default_rng(seeds.get(v_scale) or int(np.log10(v_scale)) + 600)
    q_len, kv_len = 128, 1024
    q = bf16_normal(rng, (32, q_len, 128))
    k = bf16_normal(rng, (8, kv_len, 128))
    if v_scale == "mixed":
        v32 = rng.standard_normal((8, kv_len, 128), dtype=np.float32)
        v32[:, ::7] *= np.float32(1e20)  # every 7th key's row dominates the rows that see it
        v = orc.fp32_to_bf16_u16(v32)
    elif v_scale == "weighted":
        # The first 256 keys carry V ~ 1e30 but scores far below the rest (scores 0 against about
        # 130: weight ~ e^-130 after the softmax), the later keys V ~ 1e-10: the segments with the
        # largest |O| contribute almost nothing, and must not flush the segments that do.
        k32 = orc.bf16_u16_to_fp32(k).copy()
        k32[:, :256] = 0.0
        k = orc.fp32_to_bf16_u16(k32)
        q32 = np.abs(orc.bf16_u16_to_fp32(q)) + np.float32(1.0)
        q = orc.fp32_to_bf16_u16(q32)
        k32 = orc.bf16_u16_to_fp32(k).copy()
        k32[:, 256:] = np.abs(k32[:, 256:]) * np.float32(8.0)  # scores of the later keys >> 0
        k = orc.fp32_to_bf16_u16(k32)
        v32 = rng.standard_normal((8, kv_len, 128), dtype=np.float32) * np.float32(1e-10)
        v32[:, :256] = rng.standard_normal((8, 256, 128), dtype=np.float32) * np.float32(1e30)
        v = orc.fp32_to_bf16_u16(v32)
    else:
        v = bf16_normal(rng, (8, kv_len, 128), v_scale)
    outs = []
    for wgs in (1024, 1):  # many KV segments, then one (no partials)
        with AttentionAccelerator(max_seq_len=kv_len, max_q_len=q_len) as acc:
            from lara_amd import _lib
            _lib.check(acc._lib.gqa_set_option(acc._ctx, _lib.GQA_OPT_PREFILL_WGS, wgs), "prefill wgs")
            acc.load_kv(k, v)
            outs.append(acc.prefill_chunk(q, q_pos_base=kv_len - q_len, kv_len=kv_len, return_lse=True))
    out, lse = outs[0]
    assert np.all(np.isfinite(drv.bf16_u16_to_fp32(out)))
    ref, ref_lse = oracle_for(q, k, v, causal=True, q_pos_base=kv_len - q_len)
    check_rows(out, lse, ref, ref_lse)
    check_rows(outs[1][0], outs[1][1], ref, ref_lse)


@pytest.mark.parametrize("kernel", ["rows", "shared", "paired"])
def test_prefill_scores_climbing_past_the_reference_max(kernel):
    """Scores that climb block after block far past the first block's max (positive Q, K rows
    scaled by a ramp: about 140 log2 units over the prompt) with V of magnitude 1e20.  The kernels
    take a block's weights against the row's reference max while a lane's weights sum to at most
    2^16 and otherwise move the max and rescale; both paths run here, and every output row is within
    the 2-ulp bound and finite."""
    rng = np.random.default_rng(777)
    hq, hkv, d, L = 32, 8, 128, 512
    print(f"[climb] kernel={kernel} L={L}", flush=True)
    q = orc.fp32_to_bf16_u16(np.abs(rng.standard_normal((hq, L, d), dtype=np.float32)) + np.float32(1.0))
    ramp = np.linspace(0.0, 6.0, L, dtype=np.float32)[None, :, None]
    k = orc.fp32_to_bf16_u16(np.abs(rng.standard_normal((hkv, L, d), dtype=np.float32)) * ramp)
    v = bf16_normal(rng, (hkv, L, d), 1e20)
    with AttentionAccelerator(max_seq_len=L, max_q_len=L) as acc:
        set_prefill_kernel(acc, kernel)
        acc.load_kv(k, v)
        out, lse = acc.prefill_chunk(q, q_pos_base=0, kv_len=L, causal=True, return_lse=True)
        assert acc.last_prefill_plan()[0] == kernel
    assert np.all(np.isfinite(drv.bf16_u16_to_fp32(out)))
    ref, ref_lse = oracle_for(q, k, v, causal=True)
    check_rows(out, lse, ref, ref_lse)


@pytest.mark.parametrize("kernel", ["rows", "shared"])
def test_prefill_cancelling_v_rows_within_the_weight_rounding_bound(kernel):
    """Causal prefill over V rows in cancelling pairs: within 2 ulp of the row's largest |output| plus
    2^-8 of attention over |V| per element (P rounded to bf16 for the PV product), the stated bound
    of the EXACT mode; l within rtol 1e-2."""
    from tests._gen import cancelling_kv

    rng = np.random.default_rng(4300)
    q_len, kv_len = 64, 256
    q = bf16_normal(rng, (32, q_len, 128))
    k, v = cancelling_kv(rng, 8, kv_len, 128)
    with AttentionAccelerator(max_seq_len=kv_len, max_q_len=q_len) as acc:
        set_prefill_kernel(acc, kernel)
        acc.load_kv(k, v)
        out, lse = acc.prefill_chunk(q, q_pos_base=kv_len - q_len, kv_len=kv_len, causal=True, return_lse=True)
    ref, ref_lse = oracle_for(q, k, v, causal=True, q_pos_base=kv_len - q_len)
    ref_abs, _ = oracle_for(q, k, v & np.uint16(0x7FFF), causal=True, q_pos_base=kv_len - q_len)
    err = orc.weight_rounding_error(out, ref, ref_abs)
    print(f"[cancel] prefill {kernel}: bound use {err.max():.3f}, 2-ulp measure "
          f"{orc.row_ulp_error(out, ref).max():.2f}", flush=True)
    assert float(err.max()) <= 1.0
    rel = np.abs(np.expm1(lse.astype(np.float64) - ref_lse))
    assert float(rel.max()) <= L_RTOL
