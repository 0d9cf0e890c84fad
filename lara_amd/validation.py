"""Full validation run on one MI355X: the counterpart of the board's ``sw/run_board_full_validation.py``.

Stages, each a child process in its own process group with its output teed to a log
(sw/run_board_full_validation.py:47-113):

1. ``init``: the device probe that replaces the board's ``clear_pynq_cache.py`` report -- the
   library loads, a gfx950 device is visible, and one KV260-contract transaction runs.
2. ``functional/<label>``: ``python -m lara_amd.board_matrix`` over each case set
   (``--case-set LABEL=DIR``, the board's ``case_*.npz`` format), word-for-word against
   ``expected_o`` (:277-297).
3. ``performance/cpu<N>``: ``bench.py --board-matrix`` over the same case sets, once per CPU
   baseline thread count (:299-321).

The run directory must be new or empty (:38-44).  ``run_manifest.json`` is rewritten after
every stage with the configuration, the environment, SHA-256 provenance of the library, the
driver sources and every case file (:146-181), and the stage records; ``consolidated_results.json``
holds the pass counts (:323-350).  Exit status 0 only when every stage and every case passed.

    python -m lara_amd.validation --case-set board=tests/golden/board_cases [--output-dir DIR]
        [--lengths 1 16 32 64 128] [--causal-only] [--numerics kv260|exact] [--cpu-threads 1 4]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import queue
import shutil
import signal
import subprocess
import sys
import threading
import time
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SCHEMA = "lara-mi355x-full-validation-v1"
PROVENANCE_FILES = ("attn_driver.py", "_lib.py", "board_matrix.py", "benchmark.py", "validation.py", "libgqa.so")


def sha256(path: Path) -> str:
    h = hashlib.sha256()
    with Path(path).open("rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def write_json(path: Path, value: Any) -> None:
    tmp = path.with_suffix(path.suffix + ".tmp")
    tmp.write_text(json.dumps(value, indent=2) + "\n", encoding="utf-8")
    tmp.replace(path)


def require_empty_output(path: Path) -> None:
    if path.exists() and any(path.iterdir()):
        raise FileExistsError(f"result directory is not empty: {path}; choose a new --output-dir")
    path.mkdir(parents=True, exist_ok=True)


def _reap(process: subprocess.Popen, grace_s: float) -> None:
    """Stop a stage's whole process group: SIGINT, then SIGTERM, then SIGKILL."""
    for sig in (signal.SIGINT, signal.SIGTERM, signal.SIGKILL):
        if process.poll() is not None:
            return
        try:
            os.killpg(process.pid, sig)
        except ProcessLookupError:
            return
        try:
            process.wait(timeout=grace_s)
            return
        except subprocess.TimeoutExpired:
            continue


def run_stage(command: list[str], log_path: Path, *, env: dict[str, str] | None = None,
              timeout_s: float | None = None, grace_s: float = 5.0) -> dict[str, Any]:
    """Run one stage in a new session, tee its output to ``log_path`` and stdout, and reap its
    process group if the stage overruns ``timeout_s`` or the orchestrator is interrupted."""
    print("RUN:", " ".join(command), flush=True)
    started_utc = datetime.now(timezone.utc).isoformat()
    t0 = time.perf_counter()
    log_path.parent.mkdir(parents=True, exist_ok=True)
    timed_out = False
    with log_path.open("w", encoding="utf-8") as log:
        process = subprocess.Popen(command, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, bufsize=1,
                                   env=env, cwd=str(ROOT), start_new_session=True)
        lines: queue.Queue = queue.Queue()

        def pump() -> None:  # a reader thread, so a silent stage cannot block the deadline check
            assert process.stdout is not None
            for line in process.stdout:
                lines.put(line)
            lines.put(None)

        reader = threading.Thread(target=pump, daemon=True)
        reader.start()
        deadline = None if timeout_s is None else time.monotonic() + timeout_s
        try:
            while True:
                wait = None if deadline is None else deadline - time.monotonic()
                if wait is not None and wait <= 0:
                    timed_out = True
                    _reap(process, grace_s)
                    break
                try:
                    line = lines.get(timeout=wait)
                except queue.Empty:
                    continue
                if line is None:
                    break
                print(line, end="", flush=True)
                log.write(line)
                log.flush()
            return_code = process.wait()
            reader.join(timeout=grace_s)
        except BaseException:
            _reap(process, grace_s)
            raise
    elapsed = time.perf_counter() - t0
    if timed_out:
        return_code = 124
    result = {"command": command, "log": str(log_path), "started_utc": started_utc, "elapsed_seconds": elapsed,
              "return_code": return_code, "timed_out": timed_out,
              "status": "PASS" if return_code == 0 else "FAIL"}
    print(f"STAGE {result['status']}: return_code={return_code} elapsed={elapsed:.3f}s log={log_path}", flush=True)
    return result


def functional_summary(path: Path, expected_total: int) -> dict[str, Any]:
    rows = json.loads(Path(path).read_text(encoding="utf-8"))
    if not isinstance(rows, list):
        raise ValueError(f"functional summary is not a list: {path}")
    passed = sum(r.get("status") == "PASS" for r in rows)
    return {"path": str(path), "passed": passed, "total": len(rows),
            "all_passed": passed == len(rows) == expected_total}


def performance_summary(path: Path, expected_total: int) -> dict[str, Any]:
    report = json.loads(Path(path).read_text(encoding="utf-8"))
    rows = report.get("results", [])
    errors = report.get("benchmark_errors", [])
    passed = sum(bool(r.get("correctness", {}).get("passed")) for r in rows)
    return {"json": str(path), "csv": str(Path(path).with_name("performance.csv")), "passed": passed,
            "total": len(rows), "benchmark_errors": errors,
            "all_passed": passed == len(rows) == expected_total and not errors}


def _case_meta(path: Path) -> tuple[int, bool]:
    import numpy as np
    with np.load(path, allow_pickle=False) as d:
        q = np.asarray(d["q_heads"])
        L = int(np.asarray(d["seq_len"]).reshape(-1)[0]) if "seq_len" in d.files else int(q.shape[1])
        causal = bool(np.asarray(d["causal"]).reshape(-1)[0]) if "causal" in d.files else True
    return L, causal


def select_cases(directory: Path, lengths: list[int] | None, causal_only: bool) -> list[Path]:
    out = []
    for path in sorted(Path(directory).glob("case_*.npz")):
        L, causal = _case_meta(path)
        if (lengths is None or L in lengths) and (causal or not causal_only):
            out.append(path)
    return out


def provenance(case_sets: dict[str, Path], selected: dict[str, list[Path]], out_dir: Path) -> dict[str, Any]:
    """Copies of the driver sources and library with SHA-256 (the board copies its driver and
    hashes its bitstream), plus the hash of every case file."""
    prov = out_dir / "provenance"
    prov.mkdir(parents=True, exist_ok=True)
    files = []
    for name in PROVENANCE_FILES:
        src = PACKAGE / name
        if src.is_file():
            dst = prov / name
            shutil.copy2(src, dst)
            files.append({"source": str(src), "copy": str(dst), "sha256": sha256(dst)})
    cases = {label: [{"path": str(p), "sha256": sha256(p)} for p in selected[label]] for label in case_sets}
    return {"files": files, "cases": cases}


PROBE = r"""
import json, sys
from lara_amd import _lib
from lara_amd.attn_driver import AttentionAccelerator
import numpy as np
info = {"devices": _lib.device_count()}
with AttentionAccelerator(max_seq_len=64, numerics=sys.argv[1]) as acc:
    z = np.zeros((32, 16, 128), np.uint16)
    out = acc.run_attention(z, z[:8], z[:8], seq_len=16)
    info["zero_transaction_ok"] = bool(not out.any())
    info["library"] = str(_lib.LIB_PATH)
print(json.dumps(info))
sys.exit(0 if info["devices"] >= 1 and info["zero_transaction_ok"] else 1)
"""


def parse_case_sets(specs: list[str]) -> dict[str, Path]:
    sets: dict[str, Path] = {}
    for spec in specs:
        label, _, directory = spec.partition("=")
        if not label or not directory:
            raise ValueError(f"--case-set wants LABEL=DIR, got {spec!r}")
        if label in sets:
            raise ValueError(f"duplicate case-set label {label!r}")
        sets[label] = Path(directory).expanduser().resolve()
    return sets


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--case-set", action="append", default=[], metavar="LABEL=DIR",
                        help="directory of case_*.npz files (repeatable); default board=tests/golden/board_cases")
    parser.add_argument("--output-dir", default="./gpu_full_results")
    parser.add_argument("--lengths", type=int, nargs="+", help="only run these seq_len values")
    parser.add_argument("--causal-only", action="store_true")
    parser.add_argument("--numerics", default="kv260", choices=("kv260", "exact"))
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--repeats", type=int, default=5)
    parser.add_argument("--cpu-threads", type=int, nargs="+", default=[1],
                        help="CPU baseline thread counts; '1 4' archives both baselines")
    parser.add_argument("--stage-timeout", type=float, default=1800.0, help="seconds before a stage is stopped")
    parser.add_argument("--skip-performance", action="store_true", help="run the init and functional stages only")
    args = parser.parse_args(argv)
    if args.warmup < 0 or args.repeats < 1:
        parser.error("--warmup must be >= 0 and --repeats must be >= 1")
    if any(t < 1 for t in args.cpu_threads) or len(set(args.cpu_threads)) != len(args.cpu_threads):
        parser.error("--cpu-threads values must be >= 1 and distinct")

    specs = args.case_set or [f"board={ROOT / 'tests' / 'golden' / 'board_cases'}"]
    try:
        case_sets = parse_case_sets(specs)
    except ValueError as exc:
        parser.error(str(exc))
    missing = [str(d) for d in case_sets.values() if not d.is_dir()]
    if not (PACKAGE / "libgqa.so").is_file():
        missing.append(str(PACKAGE / "libgqa.so"))
    bench = ROOT / "bench.py"
    if not args.skip_performance and not bench.is_file():
        missing.append(str(bench))
    if missing:
        raise FileNotFoundError("required inputs are missing: " + ", ".join(missing))
    selected = {label: select_cases(d, args.lengths, args.causal_only) for label, d in case_sets.items()}
    empty = [label for label, paths in selected.items() if not paths]
    if empty:
        raise FileNotFoundError(f"no case_*.npz files match the filters in case set(s): {', '.join(empty)}")

    out_dir = Path(args.output_dir).expanduser().resolve()
    require_empty_output(out_dir)
    manifest_path = out_dir / "run_manifest.json"
    consolidated_path = out_dir / "consolidated_results.json"
    from .benchmark import collect_environment
    manifest: dict[str, Any] = {
        "schema": SCHEMA, "status": "RUNNING", "started_utc": datetime.now(timezone.utc).isoformat(),
        "working_directory": str(ROOT), "output_directory": str(out_dir),
        "configuration": {"case_sets": {k: str(v) for k, v in case_sets.items()},
                          "lengths": args.lengths, "causal_only": args.causal_only, "numerics": args.numerics,
                          "warmup": args.warmup, "repeats": args.repeats, "cpu_threads": args.cpu_threads,
                          "stage_timeout_s": args.stage_timeout, "skip_performance": args.skip_performance},
        "environment": collect_environment(),
        "provenance": provenance(case_sets, selected, out_dir),
        "stages": [],
    }
    write_json(manifest_path, manifest)

    py = sys.executable
    logs = out_dir / "logs"

    def stage(kind: str, command: list[str], log_name: str, env=None, **extra) -> dict[str, Any]:
        rec = run_stage(command, logs / log_name, env=env, timeout_s=args.stage_timeout)
        rec.update({"kind": kind, **extra})
        manifest["stages"].append(rec)
        write_json(manifest_path, manifest)
        return rec

    try:
        if stage("init", [py, "-c", PROBE, args.numerics], "init.log")["return_code"] != 0:
            raise RuntimeError("device probe failed")
        for label, directory in case_sets.items():
            cmd = [py, "-m", "lara_amd.board_matrix", "--cases", str(directory), "--numerics", args.numerics,
                   "--output-dir", str(out_dir / "functional" / label)]
            if args.lengths:
                cmd += ["--lengths", *map(str, args.lengths)]
            if args.causal_only:
                cmd.append("--causal-only")
            if stage("functional", cmd, f"functional_{label}.log", case_set=label)["return_code"] != 0:
                raise RuntimeError(f"functional matrix failed: {label}")
        if not args.skip_performance:
            for threads in args.cpu_threads:
                cmd = [py, str(bench), "--board-matrix", "--numerics", args.numerics,
                       "--board-warmup", str(args.warmup), "--board-repeats", str(args.repeats),
                       "--cpu-threads", str(threads), "--output-dir", str(out_dir / "performance" / f"cpu{threads}")]
                for label, directory in case_sets.items():
                    cmd += ["--case-set", f"{label}={directory}"]
                if args.lengths:
                    cmd += ["--lengths", ",".join(map(str, args.lengths))]
                if args.causal_only:
                    cmd.append("--causal-only")
                env = os.environ.copy()
                env["LARA_CPU_THREADS"] = str(threads)
                env["OMP_NUM_THREADS"] = str(threads)
                if stage("performance", cmd, f"performance_cpu{threads}.log", env=env,
                         cpu_threads=threads)["return_code"] != 0:
                    raise RuntimeError(f"performance matrix failed: CPU threads={threads}")

        functional = {label: functional_summary(out_dir / "functional" / label / "summary.json",
                                                expected_total=len(selected[label])) for label in case_sets}
        total = sum(len(p) for p in selected.values())
        performance = {} if args.skip_performance else {
            f"cpu{t}": performance_summary(out_dir / "performance" / f"cpu{t}" / "performance.json", total)
            for t in args.cpu_threads}
        all_passed = all(x["all_passed"] for x in functional.values()) and \
            all(x["all_passed"] for x in performance.values())
        consolidated = {"overall_status": "PASS" if all_passed else "FAIL", "functional": functional,
                        "performance": performance, "run_manifest": str(manifest_path)}
        write_json(consolidated_path, consolidated)
        manifest["status"] = consolidated["overall_status"]
    except KeyboardInterrupt:
        manifest["status"] = "INTERRUPTED"
        manifest["error"] = "KeyboardInterrupt"
    except Exception as exc:  # the manifest records why the run stopped
        manifest["status"] = "FAIL"
        manifest["error"] = f"{type(exc).__name__}: {exc}"
    finally:
        manifest["ended_utc"] = datetime.now(timezone.utc).isoformat()
        write_json(manifest_path, manifest)

    print(f"FULL VALIDATION STATUS: {manifest['status']}")
    print(f"Result directory: {out_dir}")
    print(f"Run manifest: {manifest_path}")
    if consolidated_path.is_file():
        print(f"Consolidated results: {consolidated_path}")
    return 0 if manifest["status"] == "PASS" else 1


if __name__ == "__main__":
    raise SystemExit(main())
