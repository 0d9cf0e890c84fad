"""The full-validation orchestrator's host logic (lara_amd/validation.py) on the CPU.

Mirrors what sw/run_board_full_validation.py guarantees: stages run in their own process
group with their output logged, a stage that overruns is reaped with its children, the run
directory must be empty, pass counts need every selected case, and a failing stage leaves a
manifest that says FAIL and why.
"""
import json
import os
import sys
import textwrap
import time
from pathlib import Path

import pytest

from lara_amd import validation as val

CASES = Path(__file__).resolve().parent / "golden" / "board_cases"


def test_stage_logs_output_and_status(tmp_path):
    ok = val.run_stage([sys.executable, "-c", "print('alpha'); print('beta')"], tmp_path / "a.log")
    assert ok["status"] == "PASS" and ok["return_code"] == 0 and not ok["timed_out"]
    assert (tmp_path / "a.log").read_text().splitlines() == ["alpha", "beta"]
    bad = val.run_stage([sys.executable, "-c", "import sys; print('x'); sys.exit(3)"], tmp_path / "b.log")
    assert bad["status"] == "FAIL" and bad["return_code"] == 3


def _alive(pid: int) -> bool:
    try:
        os.kill(pid, 0)
    except ProcessLookupError:
        return False
    try:  # a zombie still answers signal 0; it is gone for our purpose
        with open(f"/proc/{pid}/stat") as f:
            return f.read().split(")")[-1].split()[0] != "Z"
    except FileNotFoundError:
        return False


def test_overrunning_stage_is_reaped_with_its_children(tmp_path):
    pidfile = tmp_path / "child.pid"
    script = textwrap.dedent(f"""
        import subprocess, sys, time
        child = subprocess.Popen([sys.executable, "-c", "import time; time.sleep(60)"])
        open({str(pidfile)!r}, "w").write(str(child.pid))
        print("started", flush=True)
        time.sleep(60)
    """)
    t0 = time.monotonic()
    rec = val.run_stage([sys.executable, "-c", script], tmp_path / "c.log", timeout_s=3.0, grace_s=2.0)
    assert time.monotonic() - t0 < 30
    assert rec["timed_out"] and rec["return_code"] == 124 and rec["status"] == "FAIL"
    grandchild = int(pidfile.read_text())
    for _ in range(50):
        if not _alive(grandchild):
            break
        time.sleep(0.1)
    assert not _alive(grandchild)


def test_output_directory_must_be_empty(tmp_path):
    val.require_empty_output(tmp_path / "new")
    (tmp_path / "new" / "x").write_text("1")
    with pytest.raises(FileExistsError):
        val.require_empty_output(tmp_path / "new")


def test_summaries_need_every_selected_case(tmp_path):
    f = tmp_path / "summary.json"
    f.write_text(json.dumps([{"status": "PASS"}, {"status": "PASS"}]))
    assert val.functional_summary(f, 2)["all_passed"]
    assert not val.functional_summary(f, 3)["all_passed"]  # a case that never ran is a failure
    f.write_text(json.dumps([{"status": "PASS"}, {"status": "FAIL"}]))
    assert val.functional_summary(f, 2)["passed"] == 1
    p = tmp_path / "performance.json"
    p.write_text(json.dumps({"results": [{"correctness": {"passed": True}}], "benchmark_errors": []}))
    assert val.performance_summary(p, 1)["all_passed"]
    p.write_text(json.dumps({"results": [{"correctness": {"passed": True}}],
                             "benchmark_errors": [{"case_id": "x", "error": "boom"}]}))
    assert not val.performance_summary(p, 1)["all_passed"]


def test_case_selection_and_case_set_parsing():
    every = val.select_cases(CASES, None, False)
    assert len(every) >= 3
    lengths = {val._case_meta(p)[0] for p in every}
    one = sorted(lengths)[0]
    assert all(val._case_meta(p)[0] == one for p in val.select_cases(CASES, [one], False))
    assert all(val._case_meta(p)[1] for p in val.select_cases(CASES, None, True))
    sets = val.parse_case_sets([f"a={CASES}", f"b={CASES}"])
    assert list(sets) == ["a", "b"]
    with pytest.raises(ValueError):
        val.parse_case_sets([str(CASES)])
    with pytest.raises(ValueError):
        val.parse_case_sets([f"a={CASES}", f"a={CASES}"])


def test_failed_probe_leaves_a_fail_manifest(tmp_path, monkeypatch):
    """Without a GPU the init stage fails; the manifest must say FAIL with the reason and the
    provenance hashes, and no functional stage may run."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU suite runs the full orchestrator")
    out = tmp_path / "run"
    rc = val.main(["--output-dir", str(out), "--skip-performance", f"--case-set=board={CASES}"])
    assert rc == 1
    manifest = json.loads((out / "run_manifest.json").read_text())
    assert manifest["status"] == "FAIL" and "probe" in manifest["error"]
    assert [s["kind"] for s in manifest["stages"]] == ["init"]
    names = {Path(f["source"]).name for f in manifest["provenance"]["files"]}
    assert {"attn_driver.py", "validation.py"} <= names
    assert len(manifest["provenance"]["cases"]["board"]) == len(val.select_cases(CASES, None, False))
    assert all(len(c["sha256"]) == 64 for c in manifest["provenance"]["cases"]["board"])
