"""GPU parity of the multi-layer paged K/V cache (gqa_create_paged_layers).

All layers of a model share one block table per sequence and one page allocator; each layer has
its own pools and GQA_OPT_LAYER picks the one the entry points address.  On the same inputs,
every output word and cache row of a layer must equal those of a single-layer paged engine that
holds only that layer (bit-exact), writing one layer must leave the others' rows untouched, and
page management must act on all layers at once.
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
N_LAYERS = 3
LENS = [1, 65, 300, 700]
B = len(LENS)
L_MAX = 768


def layered(**kw):
    return AttentionAccelerator(batch=B, max_seq_len=L_MAX, max_q_len=256, page_size=P,
                                n_pages=B * (L_MAX // P), n_layers=N_LAYERS, **kw)


def single(**kw):
    return AttentionAccelerator(batch=B, max_seq_len=L_MAX, max_q_len=256, page_size=P,
                                n_pages=B * (L_MAX // P), **kw)


def reserve_round_robin(acc, lens):
    grown = [0] * len(lens)
    while any(g < t for g, t in zip(grown, lens)):
        for b, t in enumerate(lens):
            if grown[b] < t:
                grown[b] = min(t, grown[b] + P)
                acc.reserve(b, grown[b])


def test_layers_share_one_block_table_and_keep_their_own_rows():
    rng = np.random.default_rng(31)
    kv = [[(bf16_normal(rng, (8, L, 128)), bf16_normal(rng, (8, L, 128))) for L in LENS] for _ in range(N_LAYERS)]
    q = [bf16_normal(rng, (B, 32, 128)) for _ in range(N_LAYERS)]
    print(f"[layers] B={B} layers={N_LAYERS} lens={LENS}", flush=True)
    with layered() as acc, single() as ref:
        assert acc.n_layers == N_LAYERS and acc.layer == 0
        reserve_round_robin(acc, LENS)
        reserve_round_robin(ref, LENS)
        # one allocation serves every layer: the tables and free count are a single layer's
        assert acc.page_info() == ref.page_info()
        assert all(np.array_equal(acc.page_table(b), ref.page_table(b)) for b in range(B))
        for layer in range(N_LAYERS):
            acc.select_layer(layer)
            for b in range(B):
                acc.load_kv(*kv[layer][b], b=b)
        for layer in range(N_LAYERS):
            acc.select_layer(layer)
            assert acc.layer == layer
            for b in range(B):
                ref.load_kv(*kv[layer][b], b=b)
                got = acc.read_kv(b, 0, LENS[b])
                assert np.array_equal(got[0], kv[layer][b][0]) and np.array_equal(got[1], kv[layer][b][1])
            o, lse = acc.decode_step(q[layer], LENS, return_lse=True)
            o_ref, lse_ref = ref.decode_step(q[layer], LENS, return_lse=True)
            assert np.array_equal(o, o_ref) and np.array_equal(lse, lse_ref), layer
            k0, v0 = kv[layer][3]
            want, _ = orc.attention(orc.bf16_u16_to_fp32(q[layer][3][:, None]), orc.bf16_u16_to_fp32(k0),
                                    orc.bf16_u16_to_fp32(v0), causal=False)
            assert float(orc.row_ulp_error(o[3][:, None], want).max()) <= 2.0
        # release unmaps the sequence in every layer at once
        acc.release(2)
        for layer in range(N_LAYERS):
            acc.select_layer(layer)
            assert np.all(acc.page_table(2) == -1)
        assert acc.page_info()["free_pages"] == ref.page_info()["free_pages"] + -(-LENS[2] // P)
        with pytest.raises(ValueError):
            acc.select_layer(N_LAYERS)


def test_model_flow_prefill_then_decode_layer_by_layer():
    """A 3-layer model: chunked prefill of a prompt into every layer, then fused decode steps
    over all layers; each layer equals its own single-layer engine step for step."""
    rng = np.random.default_rng(32)
    prompt, chunk, steps = 320, 128, 3
    with layered() as acc:
        refs = [single() for _ in range(N_LAYERS)]
        try:
            acc.reserve(1, prompt + steps)
            for r in refs:
                r.reserve(1, prompt + steps)
            for start in range(0, prompt, chunk):
                n = min(chunk, prompt - start)
                for layer in range(N_LAYERS):
                    q = bf16_normal(rng, (32, n, 128))
                    k = bf16_normal(rng, (8, n, 128))
                    v = bf16_normal(rng, (8, n, 128))
                    kw = dict(b=1, q_pos_base=start, kv_len=start + n, causal=True, k_rows=k, v_rows=v)
                    acc.select_layer(layer)
                    assert np.array_equal(acc.prefill_chunk(q, **kw), refs[layer].prefill_chunk(q, **kw)), (start, layer)
            for step in range(steps):
                pos = np.full(B, -1, np.int32)
                pos[1] = prompt + step
                ctx = np.zeros(B, np.int32)
                ctx[1] = prompt + step + 1
                for layer in range(N_LAYERS):
                    q = bf16_normal(rng, (B, 32, 128))
                    k = bf16_normal(rng, (B, 8, 128))
                    v = bf16_normal(rng, (B, 8, 128))
                    acc.select_layer(layer)
                    o = acc.decode_step(q, ctx, k_rows=k, v_rows=v, positions=pos)
                    o_ref = refs[layer].decode_step(q, ctx, k_rows=k, v_rows=v, positions=pos)
                    assert np.array_equal(o[1], o_ref[1]), (step, layer)
            for layer in range(N_LAYERS):
                acc.select_layer(layer)
                got = acc.read_kv(1, 0, prompt + steps)
                want = refs[layer].read_kv(1, 0, prompt + steps)
                assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), layer
        finally:
            for r in refs:
                r.close()


def test_transaction_reads_the_layer_it_was_submitted_on():
    rng = np.random.default_rng(33)
    L = 96
    q = bf16_normal(rng, (32, L, 128))
    kv = [(bf16_normal(rng, (8, L, 128)), bf16_normal(rng, (8, L, 128))) for _ in range(2)]
    with AttentionAccelerator(max_seq_len=256, page_size=P, n_layers=2) as acc:
        acc.reserve(0, L)
        for layer in range(2):
            acc.select_layer(layer)
            acc.load_kv(*kv[layer], b=0)
        lib, ctx = _lib.lib(), acc._ctx
        acc.select_layer(1)
        _lib.check(lib.gqa_submit(ctx, 0, _lib.as_u16_ptr(q), L, 0, L, 0, 1), "gqa_submit")
        acc.select_layer(0)  # after submission: the transaction still reads layer 1
        _lib.check(lib.gqa_start(ctx), "gqa_start")
        _lib.check(lib.gqa_wait(ctx, 10000), "gqa_wait")
        out = np.empty_like(q)
        _lib.check(lib.gqa_read_output(ctx, _lib.as_u16_ptr(out), out.size), "gqa_read_output")
        assert acc.layer == 0
    want, _ = orc.attention(orc.bf16_u16_to_fp32(q), orc.bf16_u16_to_fp32(kv[1][0]), orc.bf16_u16_to_fp32(kv[1][1]),
                            causal=True)
    assert float(orc.row_ulp_error(out, want).max()) <= 2.0
    other, _ = orc.attention(orc.bf16_u16_to_fp32(q), orc.bf16_u16_to_fp32(kv[0][0]), orc.bf16_u16_to_fp32(kv[0][1]),
                             causal=True)
    assert float(orc.row_ulp_error(out, other).max()) > 2.0


def test_layer_option_and_creation_limits():
    cfg = _lib.GqaConfig(1, 32, 8, 128, 256, 256, 0.0, 0)
    lib = _lib.lib()
    ctx = ctypes.c_void_p()
    for n_layers in (0, _lib.GQA_MAX_LAYERS + 1):
        assert lib.gqa_create_paged_layers(ctypes.byref(cfg), P, 4, n_layers, ctypes.byref(ctx)) == _lib.GQA_ERR_BAD_CFG
    with AttentionAccelerator(max_seq_len=256, page_size=P, n_layers=4) as acc:
        assert lib.gqa_set_option(acc._ctx, _lib.GQA_OPT_LAYER, 4) == _lib.GQA_ERR_RANGE
        assert lib.gqa_set_option(acc._ctx, _lib.GQA_OPT_LAYER, -1) == _lib.GQA_ERR_RANGE
        acc.select_layer(3)
        n, cur = ctypes.c_int32(0), ctypes.c_int32(0)
        _lib.check(lib.gqa_paged_layers(acc._ctx, ctypes.byref(n), ctypes.byref(cur)), "gqa_paged_layers")
        assert (n.value, cur.value) == (4, 3)
        k_ptr, v_ptr = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(lib.gqa_cache_pointers(acc._ctx, ctypes.byref(k_ptr), ctypes.byref(v_ptr), None), "ptrs")
        acc.select_layer(0)
        k0, v0 = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(lib.gqa_cache_pointers(acc._ctx, ctypes.byref(k0), ctypes.byref(v0), None), "ptrs")
        layer_bytes = acc.page_info()["n_pages"] * 8 * P * 128 * 2
        assert k_ptr.value - k0.value == 3 * layer_bytes and v_ptr.value - v0.value == 3 * layer_bytes
    with AttentionAccelerator(max_seq_len=256) as contiguous:
        assert lib.gqa_paged_layers(contiguous._ctx, None, None) == _lib.GQA_ERR_UNSUPPORTED
        assert lib.gqa_set_option(contiguous._ctx, _lib.GQA_OPT_LAYER, 0) == _lib.GQA_OK


def test_reserved_rows_never_written_read_as_zero_on_every_layer():
    """Creation clears every layer's pool, not only layer 0's: a reserved row that no call has
    written reads as zero words on each layer (first dirtying device memory that the engine's
    allocation may reuse)."""
    import torch

    junk = torch.full((64 << 20,), -1, dtype=torch.int32, device="cuda")  # 256 MiB of 0xFFFFFFFF words
    torch.cuda.synchronize()
    del junk
    torch.cuda.empty_cache()
    with layered() as acc:
        acc.reserve(0, 2 * P)
        for layer in range(N_LAYERS):
            acc.select_layer(layer)
            k, v = acc.read_kv(0, 0, 2 * P)
            assert not k.any() and not v.any(), layer
