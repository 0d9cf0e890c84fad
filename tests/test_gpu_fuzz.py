"""Randomised GPU parity: seeded decode and prefill cases drawn over the compiled shapes, cache
kinds (contiguous / paged with interleaved pages), split plans, merge paths and prefill
decompositions, each against the float64 oracle with the tolerances of test_gpu_decode and
test_gpu_prefill (every output row within 2 bf16 ulp of its largest |output|, the softmax sum
within rtol 1e-2, rows without a valid key exactly 0), and the paged engine word for word equal
to a contiguous one running the same case with the same options.  Every case prints its draw
before it runs; the seed is the test id.
"""
import numpy as np
import pytest

from lara_amd import _lib
from lara_amd.attn_driver import AttentionAccelerator
from oracle import gqa_oracle as orc
from tests._gen import bf16_normal

pytestmark = pytest.mark.gpu

ULP_TOL = 2.0
L_RTOL = 1e-2
PAGE = 64
DECODE_SHAPES = [(32, 8, 128), (16, 8, 128), (64, 8, 128), (64, 4, 128), (32, 16, 128), (16, 4, 64), (32, 4, 64),
                 (8, 4, 64)]
PREFILL_SHAPES = [(32, 8, 128), (8, 8, 128), (64, 8, 128), (32, 4, 128), (16, 2, 64), (32, 4, 64), (16, 16, 64)]


def check(out, lse, ref, ref_lse):
    err = orc.row_ulp_error(out, ref)
    worst = float(np.max(err)) if err.size else 0.0
    assert worst <= ULP_TOL, f"max row error {worst:.3f} bf16 ulp > {ULP_TOL}"
    live = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(lse), ~live)
    rel = np.abs(np.expm1(lse[live].astype(np.float64) - ref_lse[live]))
    assert float(rel.max(initial=0.0)) <= L_RTOL


def set_option(acc, option, value):
    _lib.check(acc._lib.gqa_set_option(acc._ctx, option, value), "gqa_set_option")


def reserve_interleaved(acc, lens):
    """Grow the sequences one page at a time in turn, so their pages interleave in the pool."""
    grown = [0] * len(lens)
    while any(g < t for g, t in zip(grown, lens)):
        for b, t in enumerate(lens):
            if grown[b] < t:
                grown[b] = min(t, grown[b] + PAGE)
                acc.reserve(b, grown[b])


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_steps(seed):
    rng = np.random.default_rng(9100 + seed)
    hq, hkv, d = DECODE_SHAPES[rng.integers(len(DECODE_SHAPES))]
    B = int(rng.integers(1, 7))
    L_max = 1024
    lens = rng.integers(0, L_max - 2, B).astype(np.int32)  # rows already cached
    chunk = int(rng.choice([0, 256, 512]))
    merge = int(rng.choice([_lib.GQA_DECODE_MERGE_AUTO, _lib.GQA_DECODE_MERGE_FUSED, _lib.GQA_DECODE_MERGE_LAUNCH]))
    steps = 2
    print(f"[fuzz-decode] seed={seed} hq={hq} hkv={hkv} d={d} B={B} lens={lens.tolist()} chunk={chunk} "
          f"merge={merge}", flush=True)
    kc = np.zeros((B, hkv, L_max, d), np.uint16)
    vc = np.zeros((B, hkv, L_max, d), np.uint16)
    for b in range(B):
        kc[b, :, :lens[b]] = bf16_normal(rng, (hkv, int(lens[b]), d))
        vc[b, :, :lens[b]] = bf16_normal(rng, (hkv, int(lens[b]), d))
    kw = dict(batch=B, n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=L_max, max_q_len=64)
    with AttentionAccelerator(**kw) as cont, \
            AttentionAccelerator(page_size=PAGE, n_pages=B * (L_max // PAGE), **kw) as paged:
        reserve_interleaved(paged, [int(n) + steps for n in lens])
        for acc in (cont, paged):
            if chunk:
                set_option(acc, _lib.GQA_OPT_DECODE_CHUNK, chunk)
            set_option(acc, _lib.GQA_OPT_DECODE_MERGE, merge)
            for b in range(B):
                if lens[b]:
                    acc.load_kv(kc[b, :, :lens[b]], vc[b, :, :lens[b]], b=b)
        for step in range(steps):
            pos = lens + step
            k_new = bf16_normal(rng, (B, hkv, d))
            v_new = bf16_normal(rng, (B, hkv, d))
            kc[np.arange(B), :, pos] = k_new
            vc[np.arange(B), :, pos] = v_new
            q = bf16_normal(rng, (B, hq, d))
            ctx = pos + 1
            o_c, l_c = cont.decode_step(q, ctx, k_rows=k_new, v_rows=v_new, positions=pos, return_lse=True)
            o_p, l_p = paged.decode_step(q, ctx, k_rows=k_new, v_rows=v_new, positions=pos, return_lse=True)
            assert np.array_equal(o_p, o_c) and np.array_equal(l_p, l_c), step
            ref, ref_lse = orc.decode(q, kc, vc, ctx)
            check(o_c, l_c, ref, ref_lse)


@pytest.mark.parametrize("seed", range(24))
def test_random_prefill_chunks(seed):
    rng = np.random.default_rng(9200 + seed)
    hq, hkv, d = PREFILL_SHAPES[rng.integers(len(PREFILL_SHAPES))]
    q_len = int(rng.integers(1, 200))
    prefix = int(rng.integers(0, 400))
    kv_len = prefix + q_len
    causal = bool(rng.integers(2))
    kv_pos_base = int(rng.integers(0, 40))
    q_pos_base = kv_pos_base + prefix  # the chunk's queries sit at its own keys' positions
    kernel = str(rng.choice(["auto", "rows", "shared"]))
    print(f"[fuzz-prefill] seed={seed} hq={hq} hkv={hkv} d={d} q_len={q_len} prefix={prefix} causal={causal} "
          f"kv_pos_base={kv_pos_base} kernel={kernel}", flush=True)
    code = {"auto": _lib.GQA_PREFILL_KERNEL_AUTO, "rows": _lib.GQA_PREFILL_KERNEL_ROWS,
            "shared": _lib.GQA_PREFILL_KERNEL_SHARED}[kernel]
    q = bf16_normal(rng, (hq, q_len, d))
    k = bf16_normal(rng, (hkv, kv_len, d))
    v = bf16_normal(rng, (hkv, kv_len, d))
    kw = dict(batch=2, n_q_heads=hq, n_kv_heads=hkv, head_dim=d, max_seq_len=640, max_q_len=256)
    with AttentionAccelerator(**kw) as cont, \
            AttentionAccelerator(page_size=PAGE, n_pages=2 * (640 // PAGE), **kw) as paged:
        reserve_interleaved(paged, [kv_len, kv_len])
        outs = []
        for acc in (cont, paged):
            set_option(acc, _lib.GQA_OPT_PREFILL_KERNEL, code)
            if prefix:
                acc.load_kv(k[:, :prefix], v[:, :prefix], b=1)
            outs.append(acc.prefill_chunk(q, b=1, q_pos_base=q_pos_base, kv_len=kv_len, kv_pos_base=kv_pos_base,
                                          causal=causal, k_rows=k[:, prefix:], v_rows=v[:, prefix:],
                                          return_lse=True))
            kr, vr = acc.read_kv(1, 0, kv_len)
            assert np.array_equal(kr, k) and np.array_equal(vr, v)  # the chunk's rows were placed exactly
    (o_c, l_c), (o_p, l_p) = outs
    assert np.array_equal(o_p, o_c) and np.array_equal(l_p, l_c)
    ref, ref_lse = orc.attention(orc.bf16_u16_to_fp32(q), orc.bf16_u16_to_fp32(k), orc.bf16_u16_to_fp32(v),
                                 causal=causal, q_pos_base=q_pos_base, kv_pos_base=kv_pos_base)
    check(o_c, l_c, ref, ref_lse)
