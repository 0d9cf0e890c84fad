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
