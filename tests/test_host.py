"""Host-side logic of the drop-in driver and the roofline model (no GPU needed)."""
import numpy as np
import pytest

from lara_amd import attn_driver as drv
from lara_amd import benchmark as bm
from oracle import gqa_oracle as orc


def test_product_packer_matches_oracle():
    rng = np.random.default_rng(10)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(7.0),
        (rng.integers(0, 1 << 32, 200000, dtype=np.uint64).astype(np.uint32)).view(np.float32),
        np.float32([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40]),
    ])
    assert np.array_equal(drv.fp32_to_bf16_u16(x), orc.fp32_to_bf16_u16(x))
    w = rng.integers(0, 1 << 16, 5000, dtype=np.uint16)
    assert np.array_equal(drv.fp32_to_bf16_u16(w), w)
    assert np.array_equal(drv.bf16_u16_to_fp32(w).view(np.uint32), orc.bf16_u16_to_fp32(w).view(np.uint32))


def test_product_packer_float64_input():
    x = np.array([1.0 + 2 ** -8 + 2 ** -9, -3.25], dtype=np.float64)
    assert np.array_equal(drv.fp32_to_bf16_u16(x), orc.fp32_to_bf16_u16(x))


def test_board_constants():
    assert drv.GQA_GROUP_SIZE == 4 and drv.N_Q_HEADS == 32 and drv.N_KV_HEADS == 8 and drv.HEAD_DIM == 128
    assert drv.MAX_KV_HEAD_BYTES == 512 * 128 * 2 and drv.Q_TILE_BYTES == 32 * 128 * 2
    assert drv.DMA_MAX_TRANSFER_BYTES == (1 << 26) - 1
    assert (drv.ERR_BAD_CFG, drv.ERR_BUSY_START, drv.ERR_STREAM_LEN, drv.ERR_STREAM_DEST, drv.ERR_RESULT_LEN) == (
        0x01, 0x02, 0x10, 0x11, 0x12)


def test_byte_counts_and_validation():
    c = drv.AttentionAccelerator.byte_counts(16)
    assert c == drv.TensorByteCounts(32 * 16 * 256, 8 * 16 * 256, 8 * 16 * 256, 32 * 16 * 256)
    for bad in (0, 513, -1):
        with pytest.raises(ValueError):
            drv.AttentionAccelerator.byte_counts(bad)


def test_mock_request_protocol_self_test(capsys):
    drv._self_test()
    assert "PASSED" in capsys.readouterr().out


def test_mock_request_words():
    m = drv.MockMMIO()
    m.prepare(40)  # two 32-row Q tiles
    assert m.read(drv.CSR_STATUS) == drv.STATUS_START_READY
    m.write(drv.CSR_CTRL, drv.CTRL_START)
    assert m.read(drv.CSR_STATUS) == drv.STATUS_BUSY | drv.STATUS_KV_LOAD_REQ
    assert m.read(drv.CSR_LOAD_REQ) == 0x1  # KV request, group 0
    m.transfer_complete(drv.DEST_K_CACHE)
    m.transfer_complete(drv.DEST_V_CACHE)
    # group 0, head 0, tile 0 then tile 1 (bank 1)
    assert m.read(drv.CSR_LOAD_REQ) == 0x2
    m.transfer_complete(drv.DEST_Q_BUF)
    assert m.read(drv.CSR_LOAD_REQ) == 0x2 | (1 << 2) | (1 << 16)
    m.write(drv.CSR_CTRL, drv.CTRL_CLEAR_STATUS)
    assert m.regs[drv.CSR_ERROR_CODE] == drv.ERR_NONE


def test_run_profile_fields():
    p = drv.RunProfile("t", "g", None, 1.0, 16, True, 0, 0)
    d = p.to_dict()
    for name in ("input_pack_ms", "request_service_ms", "kv_dma_bytes", "q_dma_transfers", "pl_total_cycles",
                 "pl_core_active_ms_excluding_stalls", "attention_total_ms"):
        assert name in d


def test_valid_pairs_brute_force():
    for q_len, kv_len, qb, kb in [(256, 512, 256, 0), (16, 16, 0, 0), (5, 40, 100, 70), (3, 3, 0, 2)]:
        brute = sum(1 for i in range(q_len) for j in range(kv_len) if kb + j <= qb + i)
        assert bm.valid_pairs(q_len, kv_len, causal=True, q_pos_base=qb, kv_pos_base=kb) == brute
    assert bm.valid_pairs(7, 9, causal=False) == 63


def test_tile_pairs_per_head_brute_force():
    for L in (1, 16, 32, 33, 64, 100, 512):
        n_q, n_kv = -(-L // 32), -(-L // 64)
        brute = 0
        for t in range(n_q):
            q_end = t * 32 + min(32, L - t * 32) - 1
            brute += min(q_end // 64, n_kv - 1) + 1
        assert bm.tile_pairs_per_head(L, True) == brute
        assert bm.tile_pairs_per_head(L, False) == n_q * n_kv


def test_roofline_bytes_match_measurement_plan():
    ns = bm.compute_model("decode-b64-ctx8192")
    # the fused decode launch moves every byte of the step: K/V read, Q read, O and appended rows written
    assert ns["decode_kernel_bytes"] == ns["step_bytes"] == 2 ** 31 + int(1.25 * 2 ** 20)
    # with a merge launch after it, the split kernel does not write O
    lens = np.full(64, 8192)
    assert bm.decode_kernel_bytes(32, 8, 128, lens, writes_output=False) == 2 ** 31 + int(0.75 * 2 ** 20)
    c2 = bm.compute_model("decode-b1-ctx4097")
    assert c2["step_bytes"] - 2 * 8 * 128 * 2 - 2 * 32 * 128 * 2 == 16781312
    c5 = bm.compute_model("prefill-chunked-2048")
    assert abs(c5["flops"] / 1e9 - 34.38) < 0.01


def test_workload_lengths():
    c3 = bm.WORKLOADS["decode-b64-ragged"].lengths()
    assert c3.shape == (64,) and c3.min() >= 512 and c3.max() <= 8192
    assert np.array_equal(c3, bm.WORKLOADS["decode-b64-ragged"].lengths())
    assert np.all(bm.WORKLOADS["decode-b64-ctx8192"].lengths() == 8192)
    sched = bm.prefill_chunk_schedule(bm.PREFILL_WORKLOADS["prefill-chunked-2048"])
    assert len(sched) == 8 and sched[-1] == (1792, 256, 2048)


def test_report_metrics_closed_forms():
    s = bm.stats([3.0, 1.0, 2.0, 4.0])
    assert s["min"] == 1.0 and s["max"] == 4.0 and s["median"] == 2.5
    assert abs(s["p95"] - 3.85) < 1e-12
    e = bm.numeric_error(np.array([1.0, 2.0, 0.0]), np.array([1.0, 1.0, 0.0]))
    assert e["max_abs"] == 1.0 and abs(e["mean_abs"] - 1 / 3) < 1e-15
    assert abs(e["rmse"] - np.sqrt(1 / 3)) < 1e-15
    assert abs(e["normalized_rmse"] - np.sqrt(1 / 3) / np.sqrt(2 / 3)) < 1e-15
    assert e["max_relative_floor_1e-6"] == 1.0
    env = bm.collect_environment()
    assert env["os_cpu_count"] >= 1 and "thread_environment" in env
