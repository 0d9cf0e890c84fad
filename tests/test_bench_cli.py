"""bench.py's command-line contract on a host without a GPU.

The measurement itself needs an MI355X; these checks cover what does not: the one-GPU refusal
(the engine has no multi-GPU path, so any N > 1 exits with a message instead of timing one GPU
and calling it N), the option surface its callers rely on, and the workload names.
"""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT, env=env)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_world_size_above_one_is_refused():
    import os

    env = dict(os.environ, WORLD_SIZE="2")
    r = run_bench(env=env)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_help_lists_the_contract_options():
    r = run_bench("--help")
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--workload", "--others", "--no-cpu-baseline", "--board-matrix",
                "--page-rows", "--prefill-wgs", "--chunk"):
        assert opt in r.stdout, opt


def test_unknown_other_workload_is_rejected_before_any_gpu_work():
    r = run_bench("--others", "decode-b64-ctx8192,no-such-workload")
    assert r.returncode == 2
    assert "no-such-workload" in r.stderr


def test_workload_names_say_what_they_measure():
    r = run_bench("--help")
    for name in ("decode-b64-ctx8192", "decode-b1-ctx4097", "decode-b64-ragged", "decode-b4-ctx131072",
                 "decode-b1-d64-ctx256"):
        assert name in r.stdout, name


def _fake_results():
    """Result dicts shaped like bench.py's, for every default workload."""
    dec = {"us_per_step": 309.3, "step_us": {"median": 308.1, "p95": 315.2}, "decode_us": 306.9, "combine_us": 4.2,
           "merges_per_step": 0, "kernels_gbps": 6950.0, "cache_resident": False}
    cpu_dec = {"value": 6.0, "unit": "GB/s", "cores": 1, "us_per_step": 356000.0,
               "all_cores": {"value": 26.2, "unit": "GB/s", "cores": 16, "us_per_step": 82000.0}}
    pre = {"us_per_prompt": 96.7, "prefill_kernel_us_per_prompt": 90.6, "kernel_tflops": 379.6,
           "cpu_baseline": {"value": 0.14, "unit": "TFLOP/s", "cores": 1, "us_per_prompt": 250000.0,
                            "all_cores": {"value": 0.17, "unit": "TFLOP/s", "cores": 16, "us_per_prompt": 200000.0}}}
    one = {"us_per_prompt": 575.2, "kernel_us": 532.1, "kernel_tflops": 1033.0}
    layer = {"us_per_layer": 173.3, "attention_us": 49.4, "attention_tflops": 696.0, "rms_norm_us": 7.6,
             "qkv_projection_us": 89.2, "rope_scatter_us": 13.0}
    others = {}
    for name in ("decode-b1-d64-ctx256", "decode-b1-ctx4097", "decode-b64-ragged", "decode-b4-ctx131072",
                 "decode-b64-ctx8192-paged"):
        others[name] = dict(dec, merges_per_step=1 if name == "decode-b4-ctx131072" else 0,
                            cache_resident=name.startswith("decode-b1"), cpu_baseline=cpu_dec)
    others["prefill-chunked-2048"] = pre
    others["prefill-chunked-2048-paged"] = {k: v for k, v in pre.items() if k != "cpu_baseline"}
    others["prefill-8192"] = one
    others["layer-2048"] = layer
    return dec, cpu_dec, others


def test_summary_names_every_config_and_fits_a_short_tail():
    """The summary lines are the bench's last output: a 2000-character tail of stderr must hold
    C1-C5 and the headline with their GPU and CPU figures."""
    sys.path.insert(0, str(ROOT))
    import bench

    dec, cpu_dec, others = _fake_results()
    assert set(bench.DEFAULT_OTHERS) <= set(others) | {"decode-b64-ctx8192"}
    lines = bench.summary_lines("decode-b64-ctx8192", dec, cpu_dec, others)
    text = "".join(f"[summary] {x}\n" for x in lines)
    assert len(text) <= 2000, len(text)
    for tag in ("NS ", "C1 ", "C2 ", "C3 ", "C4 ", "C5 ", "p8k ", "layer "):
        assert any(x.startswith(tag) for x in lines), tag
    for x in lines:
        if x.split()[0] in ("NS", "C1", "C2", "C3", "C4", "C5"):
            assert "cpu1 " in x and "cpu16 " in x, x


def test_rolling_append_positions_form_a_ring():
    """Step i appends at row (L - 1 + i) mod L of a sequence of L attended rows: the first step writes
    the last row, every row is written once per L steps, and the position never reaches L."""
    import numpy as np

    sys.path.insert(0, str(ROOT))
    import bench

    lens = np.array([1, 5, 256, 4097], dtype=np.int32)
    pos = bench.rolling_positions(lens, 3 * 4097).astype(np.int64)
    assert pos.shape == (3 * 4097, 4)
    assert (pos[0] == lens - 1).all()
    assert (pos >= 0).all() and (pos < lens[None, :]).all()
    for j, L in enumerate(lens):
        assert sorted(pos[:L, j].tolist()) == list(range(L))


def test_compact_rounds_floats_and_keeps_counts_whole():
    """The printed line rounds floats to 5 significant digits; whole byte counts stored as floats keep
    every digit, and ints, strings, None and non-finite values pass through."""
    import math

    sys.path.insert(0, str(ROOT))
    import bench

    out = bench.compact({"v": 6934.080491501775, "f": 0.8676560901833921, "t": 2148915777.0, "n": 7,
                         "s": "x", "z": None, "inf": math.inf, "l": [1.23456789, {"u": 309.56884765625}]})
    assert out["v"] == 6934.1 and out["f"] == 0.86766 and out["l"] == [1.2346, {"u": 309.57}]
    assert out["t"] == 2148915777 and isinstance(out["t"], int)
    assert out["n"] == 7 and out["s"] == "x" and out["z"] is None and out["inf"] == math.inf
