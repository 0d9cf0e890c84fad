"""Functional case matrix on the GPU: the counterpart of the board's ``sw/board_matrix.py``.

Runs every ``case_*.npz`` of a directory (the board's case format: ``q_heads``, ``k_heads``,
``v_heads``, ``expected_o`` as bf16 words, and optional ``seq_len``, ``causal``,
``q_pos_base``, ``kv_pos_base``; sw/board_matrix.py:117-126) through
``AttentionAccelerator.run_attention`` and compares the output word for word with
``expected_o``.  Cases are sorted by (seq_len, causal) as on the board (:28-33), each one on a
fresh engine (the board reloads its overlay per case, :110-115); the inputs are archived,
and ``summary.json`` / ``manifest.json`` carry SHA-256 provenance (:181-207).

With ``--numerics kv260`` (the default) the engine computes the deployed KV260 arithmetic bit
for bit, so board-verified ``expected_o`` words must match exactly; ``--numerics exact``
reports the first mismatch instead of a pass for any word that differs.

    python -m lara_amd.board_matrix --cases DIR [--output-dir DIR] [--lengths 16 32] [--causal-only]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import shutil
from pathlib import Path

import numpy as np

from .attn_driver import AttentionAccelerator


def _scalar(data, name: str, default: int) -> int:
    return int(np.asarray(data[name]).reshape(-1)[0]) if name in data.files else default


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def _case_key(path: Path):
    with np.load(path, allow_pickle=False) as d:
        q = np.asarray(d["q_heads"])
        return (_scalar(d, "seq_len", int(q.shape[1])), _scalar(d, "causal", 1), path.name)


def run_case(path: Path, out_dir: Path, numerics: str, timeout_ms: int | None) -> dict:
    row: dict = {"case": path.name, "status": "FAIL"}
    with np.load(path, allow_pickle=False) as d:
        q = np.asarray(d["q_heads"], dtype=np.uint16)
        k = np.asarray(d["k_heads"], dtype=np.uint16)
        v = np.asarray(d["v_heads"], dtype=np.uint16)
        expected = np.asarray(d["expected_o"], dtype=np.uint16)
        seq_len = _scalar(d, "seq_len", int(q.shape[1]))
        causal = bool(_scalar(d, "causal", 1))
        qb = _scalar(d, "q_pos_base", 0)
        kb = _scalar(d, "kv_pos_base", 0)
    hq, _, dim = q.shape
    with AttentionAccelerator(n_q_heads=hq, n_kv_heads=k.shape[0], head_dim=dim,
                              max_seq_len=max(seq_len, 512), numerics=numerics) as acc:
        actual = acc.run_attention(q, k, v, seq_len=seq_len, q_pos_base=qb, kv_pos_base=kb, causal=causal,
                                   timeout_ms=timeout_ms)
        np.savez_compressed(out_dir / f"{path.stem}_actual.npz", o_heads=actual)
        acc.save_last_profile(out_dir / f"{path.stem}_profile.json")
        row["perf"] = acc.read_perf()
    row.update(seq_len=seq_len, causal=causal, q_pos_base=qb, kv_pos_base=kb, numerics=numerics)
    mismatch = np.argwhere(actual != expected)
    row["mismatches"] = int(len(mismatch))
    if mismatch.size:
        first = tuple(int(x) for x in mismatch[0])
        row["error"] = (f"bit mismatch at {first}: got=0x{int(actual[first]):04x} "
                        f"expected=0x{int(expected[first]):04x}; mismatches={len(mismatch)}")
    else:
        row["status"] = "PASS"
    return row


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--cases", required=True, help="directory of case_*.npz files")
    parser.add_argument("--output-dir", default="board_matrix_results")
    parser.add_argument("--lengths", type=int, nargs="*", help="only run these seq_len values")
    parser.add_argument("--causal-only", action="store_true")
    parser.add_argument("--numerics", default="kv260", choices=("kv260", "exact"))
    parser.add_argument("--timeout-ms", type=int, default=None)
    args = parser.parse_args(argv)

    case_dir = Path(args.cases)
    out_dir = Path(args.output_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    archive = out_dir / "inputs"
    archive.mkdir(exist_ok=True)
    paths = sorted(case_dir.glob("case_*.npz"), key=_case_key)
    if not paths:
        raise FileNotFoundError(f"no case_*.npz files found in {case_dir}")
    if args.lengths or args.causal_only:
        keep = set(args.lengths) if args.lengths else None
        paths = [p for p in paths if (keep is None or _case_key(p)[0] in keep) and (not args.causal_only or _case_key(p)[1])]
        if not paths:
            raise FileNotFoundError(f"no case_*.npz files in {case_dir} match the requested filters")

    summary = []
    print(f"Selected GPU functional cases: {len(paths)}", flush=True)
    for i, path in enumerate(paths, start=1):
        print(f"[{i}/{len(paths)}] GPU FUNCTIONAL START {path.name}", flush=True)
        shutil.copy2(path, archive / path.name)
        try:
            row = run_case(path, out_dir, args.numerics, args.timeout_ms)
        except Exception as exc:  # keep the summary usable after a failing case
            row = {"case": path.name, "status": "FAIL", "error": str(exc)}
        row["input"] = str(archive / path.name)
        row["input_sha256"] = _sha256(path)
        print(f"[{i}/{len(paths)}] GPU FUNCTIONAL {row['status']} {path.name}"
              + (f": {row['error']}" if "error" in row else ""), flush=True)
        summary.append(row)

    (out_dir / "summary.json").write_text(json.dumps(summary, indent=2) + "\n", encoding="utf-8")
    manifest = {"cases_dir": str(case_dir.resolve()), "results_dir": str(out_dir.resolve()),
                "numerics": args.numerics, "length_filter": sorted(set(args.lengths)) if args.lengths else None,
                "causal_filter": True if args.causal_only else None, "cases": summary}
    (out_dir / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n", encoding="utf-8")
    passed = sum(r["status"] == "PASS" for r in summary)
    print(f"board matrix: {passed}/{len(summary)} PASS", flush=True)
    return 0 if passed == len(summary) else 1


if __name__ == "__main__":
    raise SystemExit(main())
