"""The full-validation orchestrator's host logic (lara_amd/validation.py) on the CPU.

What sw/run_board_full_validation.py guarantees, checked against the step executor: a step's
output is logged as it arrives, a step past its deadline is ended with its whole session, the run
directory must be new or empty, pass counts come from the artifacts and need every selected case,
and a failing step leaves a manifest that says FAIL, why, and the provenance hashes.
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


def test_execute_logs_output_and_status(tmp_path):
    ok = val.execute([sys.executable, "-c", "print('alpha'); print('beta')"], tmp_path / "a.log", echo=False)
    assert ok["status"] == "PASS" and ok["return_code"] == 0 and not ok["timed_out"]
    assert (tmp_path / "a.log").read_text().splitlines() == ["alpha", "beta"]
    bad = val.execute([sys.executable, "-c", "import sys; print('x'); sys.exit(3)"], tmp_path / "b.log", echo=False)
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


def test_step_past_its_deadline_is_ended_with_its_children(tmp_path):
    pidfile = tmp_path / "child.pid"
    script = textwrap.dedent(f"""
        import subprocess, sys, time
        child = subprocess.Popen([sys.executable, "-c", "import time; time.sleep(60)"])
        open({str(pidfile)!r}, "w").write(str(child.pid))
        print("started", flush=True)
        time.sleep(60)
    """)
    t0 = time.monotonic()
    rec = val.execute([sys.executable, "-c", script], tmp_path / "c.log", deadline_s=3.0, grace_s=2.0, echo=False)
    assert time.monotonic() - t0 < 30
    assert rec["timed_out"] and rec["return_code"] == 124 and rec["status"] == "FAIL"
    assert "started" in (tmp_path / "c.log").read_text()
    grandchild = int(pidfile.read_text())
    for _ in range(50):
        if not _alive(grandchild):
            break
        time.sleep(0.1)
    assert not _alive(grandchild)


def test_step_that_ignores_sigint_is_still_ended(tmp_path):
    script = "import signal, time; signal.signal(signal.SIGINT, signal.SIG_IGN); print('up', flush=True); time.sleep(60)"
    t0 = time.monotonic()
    rec = val.execute([sys.executable, "-c", script], tmp_path / "d.log", deadline_s=2.0, grace_s=1.0, echo=False)
    assert rec["timed_out"] and time.monotonic() - t0 < 20


def test_output_directory_must_be_new_or_empty(tmp_path):
    val.prepare_output_dir(tmp_path / "new")
    val.prepare_output_dir(tmp_path / "new")  # still empty
    (tmp_path / "new" / "x").write_text("1")
    with pytest.raises(FileExistsError):
        val.prepare_output_dir(tmp_path / "new")


def test_ledger_is_rewritten_whole(tmp_path):
    ledger = val.Ledger(tmp_path / "m.json", {"status": "RUNNING", "stages": []})
    ledger.add_stage({"kind": "probe", "status": "PASS"})
    ledger.record["status"] = "PASS"
    ledger.flush()
    assert json.loads((tmp_path / "m.json").read_text()) == {"status": "PASS",
                                                             "stages": [{"kind": "probe", "status": "PASS"}]}
    assert [p.name for p in tmp_path.iterdir()] == ["m.json"]  # no temporary file left behind


def _step(kind, path, count):
    return val.Step(kind, "x", [], path, count)


def test_pass_counts_need_every_selected_case(tmp_path):
    f = tmp_path / "summary.json"
    f.write_text(json.dumps([{"passed": True}, {"passed": True}]))
    assert val.tally(_step("functional", f, val.count_functional), 2)["all_passed"]
    assert not val.tally(_step("functional", f, val.count_functional), 3)["all_passed"]  # a case that never ran
    f.write_text(json.dumps([{"passed": True}, {"passed": False}]))
    t = val.tally(_step("functional", f, val.count_functional), 2)
    assert t["passed"] == 1 and not t["all_passed"]
    missing = val.tally(_step("functional", tmp_path / "absent.json", val.count_functional), 2)
    assert missing["passed"] == 0 and not missing["all_passed"]
    p = tmp_path / "performance.json"
    p.write_text(json.dumps({"results": [{"correctness": {"passed": True}}], "benchmark_errors": []}))
    assert val.tally(_step("performance", p, val.count_performance), 1)["all_passed"]
    p.write_text(json.dumps({"results": [{"correctness": {"passed": True}}],
                             "benchmark_errors": [{"case_id": "x", "error": "boom"}]}))
    assert not val.tally(_step("performance", p, val.count_performance), 1)["all_passed"]


def test_case_selection_and_case_set_parsing():
    every = val.pick_cases(CASES, None, False)
    assert len(every) >= 3
    lengths = {val.case_params(p)[0] for p in every}
    one = sorted(lengths)[0]
    assert all(val.case_params(p)[0] == one for p in val.pick_cases(CASES, [one], False))
    assert all(val.case_params(p)[1] for p in val.pick_cases(CASES, None, True))
    sets = val.case_sets_from([f"a={CASES}", f"b={CASES}"])
    assert list(sets) == ["a", "b"]
    with pytest.raises(ValueError):
        val.case_sets_from([str(CASES)])
    with pytest.raises(ValueError):
        val.case_sets_from([f"a={CASES}", f"a={CASES}"])


def test_plan_has_one_step_per_case_set_and_thread_count(tmp_path):
    args = val.argparse.Namespace(numerics="kv260", causal_only=True, lengths=[16, 32], skip_performance=False,
                                  cpu_threads=[1, 4], warmup=0, repeats=1)
    plan = val.build_plan(args, {"a": CASES, "b": CASES}, tmp_path)
    assert [s.name for s in plan] == ["probe", "functional:a", "functional:b", "performance:cpu1",
                                      "performance:cpu4"]
    func = plan[1].argv
    assert func[func.index("--lengths") + 1:func.index("--lengths") + 3] == ["16", "32"]
    assert "--causal-only" in func and plan[1].artifact == tmp_path / "functional" / "a" / "summary.json"
    perf = plan[4].argv
    assert perf[perf.index("--lengths") + 1] == "16,32" and plan[4].env["OMP_NUM_THREADS"] == "4"
    assert f"--case-set=b={CASES}" in perf


def test_failed_probe_leaves_a_fail_manifest(tmp_path):
    """Without a GPU the probe step fails; the manifest must say FAIL with the reason and the
    provenance hashes, and no functional step may run."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU suite runs the full orchestrator")
    out = tmp_path / "run"
    rc = val.main(["--output-dir", str(out), "--skip-performance", f"--case-set=board={CASES}"])
    assert rc == 1
    manifest = json.loads((out / "run_manifest.json").read_text())
    assert manifest["status"] == "FAIL" and "probe" in manifest["error"]
    assert [s["kind"] for s in manifest["stages"]] == ["probe"]
    assert not (out / "consolidated_results.json").exists()
    for key in ("schema", "started_utc", "ended_utc", "working_directory", "output_directory", "configuration"):
        assert key in manifest
    names = {Path(f["source"]).name for f in manifest["provenance"]["files"]}
    assert {"attn_driver.py", "validation.py"} <= names
    assert len(manifest["provenance"]["cases"]["board"]) == len(val.pick_cases(CASES, None, False))
    assert all(len(c["sha256"]) == 64 for c in manifest["provenance"]["cases"]["board"])
