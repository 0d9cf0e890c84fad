"""The full-validation orchestrator end to end on the GPU (sw/run_board_full_validation.py re-targeted).

Runs ``python -m lara_amd.validation`` as a child process over the committed board-format
cases: the device probe, the functional matrix (KV260 numerics, word for word against
``expected_o``) and the performance matrix (one CPU-thread setting, one repeat) must all
pass, and the consolidated counts must cover every case.
"""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CASES = ROOT / "tests" / "golden" / "board_cases"

pytestmark = pytest.mark.gpu


@pytest.mark.timeout(400)
def test_full_validation_run_passes(tmp_path):
    out = tmp_path / "run"
    cmd = [sys.executable, "-u", "-m", "lara_amd.validation", f"--case-set=board={CASES}", "--output-dir", str(out),
           "--warmup", "0", "--repeats", "1", "--cpu-threads", "1", "--stage-timeout", "150"]
    print("validation run:", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=380)
    print(proc.stdout[-4000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0
    manifest = json.loads((out / "run_manifest.json").read_text())
    assert manifest["status"] == "PASS"
    assert [s["kind"] for s in manifest["stages"]] == ["probe", "functional", "performance"]
    consolidated = json.loads((out / "consolidated_results.json").read_text())
    n = len(list(CASES.glob("case_*.npz")))
    assert consolidated["overall_status"] == "PASS"
    assert consolidated["functional"]["board"]["passed"] == n
    perf = consolidated["performance"]["cpu1"]
    assert perf["passed"] == perf["total"] == perf["expected"] == n
    report = json.loads((out / "performance" / "cpu1" / "performance.json").read_text())
    assert all(r["correctness"]["gpu_bit_exact_expected"] and r["correctness"]["gpu_bit_exact_kv260_model"]
               for r in report["results"])
