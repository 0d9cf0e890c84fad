"""Full validation of the GPU engine on one MI355X.

Covers what the board's ``sw/run_board_full_validation.py`` covers for the KV260 (a device check,
the functional case matrix, the performance matrix, a provenance manifest), organised as a plan of
steps run by a small executor:

* ``build_plan`` turns the options into ``Step``s: a ``probe`` (the library loads, a gfx950 device
  answers, a zero transaction returns zeros), one ``functional`` step per case set
  (``python -m lara_amd.board_matrix``: every output word against ``expected_o``) and one
  ``performance`` step per CPU-baseline thread count (``bench.py --board-matrix``).  Each step names
  the artifact it must leave and how to count the cases that passed in it.
* ``execute`` runs one step as a child in a session of its own, copies its output to the console
  and to the step's log as it arrives (``selectors`` on the pipe), and ends the whole session
  (SIGINT, SIGTERM, then SIGKILL, a grace period apart) when the step passes its deadline or the
  run is interrupted.
* ``run_plan`` executes the steps in order, stops at the first failing one, records every result in
  the ledger, and finally counts passes from the artifacts: the run passes only when every step
  exited 0 and every selected case appears as passed.

Outputs in a new or empty directory: ``run_manifest.json`` (schema, status, started_utc,
ended_utc, working_directory, output_directory, configuration, environment, provenance -- SHA-256
of the library, the driver sources and every selected case file -- and stages: the manifest keys
are the board runs' data format), ``consolidated_results.json`` (overall status and pass counts),
``logs/`` and the steps' own outputs.

    python -m lara_amd.validation --case-set board=tests/golden/board_cases [--output-dir DIR]
        [--lengths 1 16 32 64 128] [--causal-only] [--numerics kv260|exact] [--cpu-threads 1 4]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import selectors
import signal
import subprocess
import sys
import tempfile
import time
from dataclasses import dataclass, field
from datetime import datetime, timezone
from pathlib import Path
from typing import Any, Callable

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SCHEMA = "lara-mi355x-full-validation-v1"
TRACKED_SOURCES = ("attn_driver.py", "_lib.py", "board_matrix.py", "benchmark.py", "validation.py", "libgqa.so")


def utc_now() -> str:
    return datetime.now(timezone.utc).isoformat()


def file_sha256(path: Path) -> str:
    """SHA-256 of a file, read through one reusable buffer."""
    h = hashlib.sha256()
    buf = bytearray(1 << 20)
    view = memoryview(buf)
    with open(path, "rb", buffering=0) as f:
        while True:
            n = f.readinto(buf)
            if not n:
                break
            h.update(view[:n])
    return h.hexdigest()


def prepare_output_dir(path: Path) -> Path:
    """The run's directory: created if missing; one that already holds files is refused, so results
    of different runs never mix."""
    path = Path(path)
    if path.is_dir() and next(path.iterdir(), None) is not None:
        raise FileExistsError(f"refusing to write into {path}: it already holds files")
    path.mkdir(parents=True, exist_ok=True)
    return path


class Ledger:
    """The run manifest, rewritten atomically (temporary file + rename) after every change."""

    def __init__(self, path: Path, record: dict[str, Any]):
        self.path = Path(path)
        self.record = record
        self.flush()

    def flush(self) -> None:
        fd, tmp = tempfile.mkstemp(prefix=".manifest-", dir=self.path.parent)
        with os.fdopen(fd, "w", encoding="utf-8") as f:
            json.dump(self.record, f, indent=2)
            f.write("\n")
        os.replace(tmp, self.path)

    def add_stage(self, result: dict[str, Any]) -> None:
        self.record["stages"].append(result)
        self.flush()


@dataclass
class Step:
    """One child command of the plan and the artifact whose passes it contributes."""

    kind: str
    label: str
    argv: list[str]
    artifact: Path | None = None
    count: Callable[[Path], tuple[int, int]] | None = None  # artifact -> (passed, recorded)
    env: dict[str, str] | None = None
    extra: dict[str, Any] = field(default_factory=dict)

    @property
    def name(self) -> str:
        return f"{self.kind}:{self.label}" if self.label else self.kind


def end_session(proc: subprocess.Popen, grace_s: float) -> None:
    """Signal the child's whole session, escalating until it is gone."""
    for sig in (signal.SIGINT, signal.SIGTERM, signal.SIGKILL):
        if proc.poll() is not None:
            return
        try:
            os.killpg(proc.pid, sig)
        except ProcessLookupError:
            return
        try:
            proc.wait(timeout=grace_s)
        except subprocess.TimeoutExpired:
            pass


def execute(argv: list[str], log_path: Path, *, env: dict[str, str] | None = None, deadline_s: float | None = None,
            grace_s: float = 5.0, echo: bool = True) -> dict[str, Any]:
    """Run argv in a new session from the repository root; its merged output goes to log_path (and
    the console) as it arrives.  Past deadline_s seconds the session is ended and the exit code is
    124.  Returns the step's record."""
    log_path = Path(log_path)
    log_path.parent.mkdir(parents=True, exist_ok=True)
    started = utc_now()
    t0 = time.monotonic()
    expired = False
    with open(log_path, "wb") as log:
        proc = subprocess.Popen(argv, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, env=env, cwd=str(ROOT),
                                start_new_session=True)
        assert proc.stdout is not None
        fd = proc.stdout.fileno()
        os.set_blocking(fd, False)
        sel = selectors.DefaultSelector()
        sel.register(fd, selectors.EVENT_READ)
        try:
            open_pipe = True
            while open_pipe:
                left = None if deadline_s is None else deadline_s - (time.monotonic() - t0)
                if left is not None and left <= 0:
                    expired = True
                    end_session(proc, grace_s)
                    break
                for _key, _ in sel.select(timeout=left if left is None else min(left, 1.0)):
                    chunk = os.read(fd, 1 << 16)
                    if not chunk:
                        open_pipe = False
                        break
                    log.write(chunk)
                    log.flush()
                    if echo:
                        sys.stdout.write(chunk.decode("utf-8", "replace"))
                        sys.stdout.flush()
            code = proc.wait()
        except BaseException:
            end_session(proc, grace_s)
            raise
        finally:
            sel.close()
            proc.stdout.close()
    return {"command": argv, "log": str(log_path), "started_utc": started,
            "elapsed_seconds": time.monotonic() - t0, "return_code": 124 if expired else code, "timed_out": expired,
            "status": "PASS" if (not expired and code == 0) else "FAIL"}


# ---- artifacts ------------------------------------------------------------------------------------

def count_functional(path: Path) -> tuple[int, int]:
    """(passed, recorded) of a board_matrix summary.json: a list of case records with ``passed``."""
    records = json.loads(Path(path).read_text(encoding="utf-8"))
    if not isinstance(records, list):
        raise ValueError(f"{path}: expected a list of case records")
    return sum(bool(r.get("passed")) for r in records), len(records)


def count_performance(path: Path) -> tuple[int, int]:
    """(passed, recorded) of a bench.py --board-matrix performance.json; a benchmark error in the
    report counts as a case that did not pass."""
    report = json.loads(Path(path).read_text(encoding="utf-8"))
    rows = report.get("results", [])
    passed = sum(bool(r.get("correctness", {}).get("passed")) for r in rows)
    return passed, len(rows) + len(report.get("benchmark_errors", []))


def tally(step: Step, expected: int) -> dict[str, Any]:
    """Pass count of a finished step against the number of cases it was given."""
    if step.artifact is None or step.count is None:
        return {}
    if not step.artifact.is_file():
        return {"artifact": str(step.artifact), "passed": 0, "total": 0, "expected": expected, "all_passed": False}
    passed, total = step.count(step.artifact)
    return {"artifact": str(step.artifact), "passed": passed, "total": total, "expected": expected,
            "all_passed": passed == total == expected}


# ---- case sets ------------------------------------------------------------------------------------

def case_params(path: Path) -> tuple[int, bool]:
    """(seq_len, causal) of a board case file."""
    import numpy as np

    with np.load(path, allow_pickle=False) as d:
        seq_len = int(np.asarray(d["seq_len"]).ravel()[0]) if "seq_len" in d.files else int(d["q_heads"].shape[1])
        causal = bool(np.asarray(d["causal"]).ravel()[0]) if "causal" in d.files else True
    return seq_len, causal


def pick_cases(directory: Path, lengths: list[int] | None, causal_only: bool) -> list[Path]:
    keep = []
    for path in sorted(Path(directory).glob("case_*.npz")):
        seq_len, causal = case_params(path)
        if (not lengths or seq_len in lengths) and (causal or not causal_only):
            keep.append(path)
    return keep


def case_sets_from(specs: list[str]) -> dict[str, Path]:
    """LABEL=DIR specifications -> {label: resolved directory}; labels must be unique."""
    out: dict[str, Path] = {}
    for spec in specs:
        label, sep, directory = spec.partition("=")
        if not sep or not label or not directory:
            raise ValueError(f"a case set is LABEL=DIR, not {spec!r}")
        if label in out:
            raise ValueError(f"case set label {label!r} given twice")
        out[label] = Path(directory).expanduser().resolve()
    return out


# ---- the plan -------------------------------------------------------------------------------------

PROBE_SOURCE = r"""
import json, sys
import numpy as np
from lara_amd import _lib
from lara_amd.attn_driver import AttentionAccelerator
report = {"devices": _lib.device_count(), "library": str(_lib.LIB_PATH)}
with AttentionAccelerator(max_seq_len=64, numerics=sys.argv[1]) as engine:
    zeros = np.zeros((32, 16, 128), np.uint16)
    report["zero_transaction_ok"] = not engine.run_attention(zeros, zeros[:8], zeros[:8], seq_len=16).any()
print(json.dumps(report))
sys.exit(0 if report["devices"] > 0 and report["zero_transaction_ok"] else 1)
"""


def build_plan(args, case_sets: dict[str, Path], out_dir: Path) -> list[Step]:
    py = sys.executable
    filters: list[str] = []
    if args.causal_only:
        filters.append("--causal-only")
    steps = [Step("probe", "", [py, "-c", PROBE_SOURCE, args.numerics])]
    for label, directory in case_sets.items():
        dest = out_dir / "functional" / label
        argv = [py, "-m", "lara_amd.board_matrix", "--cases", str(directory), "--numerics", args.numerics,
                "--output-dir", str(dest), *filters]
        if args.lengths:
            argv += ["--lengths", *map(str, args.lengths)]
        steps.append(Step("functional", label, argv, dest / "summary.json", count_functional,
                          extra={"case_set": label}))
    if not args.skip_performance:
        for threads in args.cpu_threads:
            dest = out_dir / "performance" / f"cpu{threads}"
            argv = [py, str(ROOT / "bench.py"), "--board-matrix", "--numerics", args.numerics, "--board-warmup",
                    str(args.warmup), "--board-repeats", str(args.repeats), "--cpu-threads", str(threads),
                    "--output-dir", str(dest), *filters]
            argv += [f"--case-set={label}={d}" for label, d in case_sets.items()]
            if args.lengths:
                argv += ["--lengths", ",".join(map(str, args.lengths))]
            env = dict(os.environ, LARA_CPU_THREADS=str(threads), OMP_NUM_THREADS=str(threads))
            steps.append(Step("performance", f"cpu{threads}", argv, dest / "performance.json", count_performance,
                              env=env, extra={"cpu_threads": threads}))
    return steps


def provenance(case_files: dict[str, list[Path]], out_dir: Path) -> dict[str, Any]:
    """Copies of the driver sources and the library with their SHA-256 (the board keeps a copy of
    its driver and hashes its bitstream), and the SHA-256 of every selected case file."""
    keep = out_dir / "provenance"
    keep.mkdir(parents=True, exist_ok=True)
    files = []
    for name in TRACKED_SOURCES:
        src = PACKAGE / name
        if src.is_file():
            dst = keep / name
            dst.write_bytes(src.read_bytes())
            files.append({"source": str(src), "copy": str(dst), "sha256": file_sha256(dst)})
    return {"files": files,
            "cases": {label: [{"path": str(p), "sha256": file_sha256(p)} for p in paths]
                      for label, paths in case_files.items()}}


def run_plan(steps: list[Step], ledger: Ledger, log_dir: Path, deadline_s: float,
             expected: dict[str, int]) -> dict[str, Any]:
    """Execute the steps in order (the first failure ends the run), then count the passes each step's
    artifact records against the cases it was given."""
    done: list[Step] = []
    for step in steps:
        print(f"[validation] {step.name}: starting", flush=True)
        result = execute(step.argv, log_dir / f"{step.name.replace(':', '_')}.log", env=step.env,
                         deadline_s=deadline_s)
        result.update(kind=step.kind, **step.extra)
        ledger.add_stage(result)
        print(f"[validation] {step.name}: {'ok' if result['status'] == 'PASS' else 'failed'} "
              f"(exit {result['return_code']}, {result['elapsed_seconds']:.1f} s, log {result['log']})", flush=True)
        if result["status"] != "PASS":
            raise RuntimeError(f"step {step.name} failed" + (" (deadline passed)" if result["timed_out"] else ""))
        done.append(step)
    counts = {"functional": {}, "performance": {}}
    for step in done:
        if step.kind in counts:
            counts[step.kind][step.label] = tally(step, expected[step.name])
    ok = all(c["all_passed"] for group in counts.values() for c in group.values())
    return {"overall_status": "PASS" if ok else "FAIL", **counts}


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--case-set", action="append", default=[], metavar="LABEL=DIR",
                        help="a directory of case_*.npz files (repeatable); default board=tests/golden/board_cases")
    parser.add_argument("--output-dir", default="./gpu_full_results")
    parser.add_argument("--lengths", type=int, nargs="+", help="keep only these seq_len values")
    parser.add_argument("--causal-only", action="store_true")
    parser.add_argument("--numerics", default="kv260", choices=("kv260", "exact"))
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--repeats", type=int, default=5)
    parser.add_argument("--cpu-threads", type=int, nargs="+", default=[1],
                        help="CPU baseline thread counts, one performance step each")
    parser.add_argument("--stage-timeout", type=float, default=1800.0, help="deadline of each step in seconds")
    parser.add_argument("--skip-performance", action="store_true", help="probe and functional steps only")
    args = parser.parse_args(argv)
    if args.warmup < 0 or args.repeats < 1:
        parser.error("--warmup must be >= 0 and --repeats >= 1")
    if min(args.cpu_threads) < 1 or len(set(args.cpu_threads)) != len(args.cpu_threads):
        parser.error("--cpu-threads takes distinct counts >= 1")
    try:
        case_sets = case_sets_from(args.case_set or [f"board={ROOT / 'tests' / 'golden' / 'board_cases'}"])
    except ValueError as exc:
        parser.error(str(exc))
    absent = [str(d) for d in case_sets.values() if not d.is_dir()]
    absent += [str(p) for p in (PACKAGE / "libgqa.so", ROOT / "bench.py") if not p.is_file()]
    if absent:
        raise FileNotFoundError("missing: " + ", ".join(absent))
    case_files = {label: pick_cases(d, args.lengths, args.causal_only) for label, d in case_sets.items()}
    empty = sorted(label for label, files in case_files.items() if not files)
    if empty:
        raise FileNotFoundError(f"the filters select no case file in case set(s) {', '.join(empty)}")

    out_dir = prepare_output_dir(Path(args.output_dir).expanduser().resolve())
    from .benchmark import collect_environment

    configuration = {"case_sets": {k: str(v) for k, v in case_sets.items()}, "lengths": args.lengths,
                     "causal_only": args.causal_only, "numerics": args.numerics, "warmup": args.warmup,
                     "repeats": args.repeats, "cpu_threads": args.cpu_threads, "stage_timeout_s": args.stage_timeout,
                     "skip_performance": args.skip_performance}
    ledger = Ledger(out_dir / "run_manifest.json", {
        "schema": SCHEMA, "status": "RUNNING", "started_utc": utc_now(), "working_directory": str(ROOT),
        "output_directory": str(out_dir), "configuration": configuration, "environment": collect_environment(),
        "provenance": provenance(case_files, out_dir), "stages": []})
    steps = build_plan(args, case_sets, out_dir)
    n_all = sum(len(files) for files in case_files.values())
    expected = {s.name: (len(case_files[s.label]) if s.kind == "functional" else n_all) for s in steps}
    summary_path = out_dir / "consolidated_results.json"
    try:
        summary = run_plan(steps, ledger, out_dir / "logs", args.stage_timeout, expected)
        summary["run_manifest"] = str(ledger.path)
        summary_path.write_text(json.dumps(summary, indent=2) + "\n", encoding="utf-8")
        ledger.record["status"] = summary["overall_status"]
    except KeyboardInterrupt:
        ledger.record.update(status="INTERRUPTED", error="interrupted by the user")
    except (RuntimeError, OSError, ValueError) as exc:  # the ledger keeps why the run stopped
        ledger.record.update(status="FAIL", error=f"{type(exc).__name__}: {exc}")
    finally:
        ledger.record["ended_utc"] = utc_now()
        ledger.flush()
    status = ledger.record["status"]
    print(f"[validation] {status} -- results in {out_dir} (manifest {ledger.path.name}"
          + (f", summary {summary_path.name})" if summary_path.is_file() else ")"), flush=True)
    return 0 if status == "PASS" else 1


if __name__ == "__main__":
    raise SystemExit(main())
