"""bench.py's command-line contract on a host without a GPU.

The measurement itself needs an MI355X; these checks cover what does not: the one-GPU refusal
(this build has no multi-GPU path, so any N > 1 exits with a message instead of timing one GPU
and calling it N), and the option surface the round-end driver and the docs rely on.
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
