"""Word-for-word functional matrix of board case files on the GPU engine.

Plays the part of the board's ``sw/board_matrix.py``: every case file of a directory runs as one
``AttentionAccelerator.run_attention`` transaction and its output words are compared with the
words the case file expects.  The case-file format is the board's (``sw/board_matrix.py:117-126``):
an ``.npz`` named ``case_*.npz`` holding ``q_heads`` [H_q, L, D], ``k_heads`` / ``v_heads``
[H_kv, L, D] and ``expected_o`` [H_q, L, D] as bf16 words, plus optional scalars ``seq_len``,
``causal``, ``q_pos_base`` and ``kv_pos_base``.

With ``--numerics kv260`` (default) the engine computes the deployed KV260 arithmetic bit for bit,
so board-verified words must match exactly; ``--numerics exact`` runs the exact kernels and simply
reports the words that differ.  Each case gets a fresh engine (the board reprograms its overlay per
case).  The output directory receives a copy of every input, the engine's output and profile per
case, and two JSON records: ``summary.json`` (one entry per case, ``passed`` true or false) and
``manifest.json`` (the run's settings and the entries with input SHA-256).

    python -m lara_amd.board_matrix --cases DIR [--output-dir DIR] [--lengths 16 32] [--causal-only]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import shutil
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .attn_driver import AttentionAccelerator

CASE_GLOB = "case_*.npz"


@dataclass(frozen=True)
class BoardCase:
    """One case file, its tensors as bf16 words and its transaction parameters."""

    path: Path
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    expected: np.ndarray
    seq_len: int
    causal: bool
    q_pos_base: int
    kv_pos_base: int

    @classmethod
    def load(cls, path: Path) -> "BoardCase":
        with np.load(path, allow_pickle=False) as data:
            def scalar(key: str, default: int) -> int:
                return int(np.asarray(data[key]).ravel()[0]) if key in data.files else default

            q = np.asarray(data["q_heads"], dtype=np.uint16)
            return cls(path=Path(path), q=q, k=np.asarray(data["k_heads"], dtype=np.uint16),
                       v=np.asarray(data["v_heads"], dtype=np.uint16),
                       expected=np.asarray(data["expected_o"], dtype=np.uint16),
                       seq_len=scalar("seq_len", q.shape[1]), causal=bool(scalar("causal", 1)),
                       q_pos_base=scalar("q_pos_base", 0), kv_pos_base=scalar("kv_pos_base", 0))

    @property
    def order(self) -> tuple:
        """Run order: shorter transactions first, causal before non-causal (the board's order)."""
        return (self.seq_len, not self.causal, self.path.name)


def word_difference(actual: np.ndarray, expected: np.ndarray) -> dict | None:
    """None when the words are equal, else the count of differing words and the first of them."""
    if actual.shape != expected.shape:
        return {"count": int(max(actual.size, expected.size)), "shape": [list(actual.shape), list(expected.shape)]}
    where = np.flatnonzero(actual.ravel() != expected.ravel())
    if where.size == 0:
        return None
    first = np.unravel_index(int(where[0]), actual.shape)
    return {"count": int(where.size), "first_index": [int(i) for i in first],
            "gpu_word": f"0x{int(actual[first]):04x}", "expected_word": f"0x{int(expected[first]):04x}"}


def digest(path: Path) -> str:
    h = hashlib.sha256()
    h.update(Path(path).read_bytes())
    return h.hexdigest()


def run_one(case: BoardCase, numerics: str, timeout_ms: int | None, out_dir: Path) -> dict:
    """One transaction on a fresh engine; the record says whether every output word matched."""
    hq, _, dim = case.q.shape
    with AttentionAccelerator(n_q_heads=hq, n_kv_heads=case.k.shape[0], head_dim=dim,
                              max_seq_len=max(case.seq_len, 512), numerics=numerics) as engine:
        out = engine.run_attention(case.q, case.k, case.v, seq_len=case.seq_len, q_pos_base=case.q_pos_base,
                                   kv_pos_base=case.kv_pos_base, causal=case.causal, timeout_ms=timeout_ms)
        stem = case.path.stem
        np.savez_compressed(out_dir / f"{stem}_actual.npz", o_heads=out)
        engine.save_last_profile(out_dir / f"{stem}_profile.json")
        perf = engine.read_perf()
    diff = word_difference(out, case.expected)
    return {"case": case.path.name, "passed": diff is None, "seq_len": case.seq_len, "causal": case.causal,
            "q_pos_base": case.q_pos_base, "kv_pos_base": case.kv_pos_base, "numerics": numerics,
            "difference": diff, "perf": perf}


def select(directory: Path, lengths: list[int] | None, causal_only: bool) -> list[BoardCase]:
    """The directory's case files that pass the filters, in run order."""
    files = sorted(Path(directory).glob(CASE_GLOB))
    if not files:
        raise FileNotFoundError(f"{directory} holds no board case files ({CASE_GLOB})")
    wanted = set(lengths) if lengths else None
    cases = [c for c in map(BoardCase.load, files)
             if (wanted is None or c.seq_len in wanted) and (c.causal or not causal_only)]
    if not cases:
        raise FileNotFoundError(f"the filters leave none of the {len(files)} case files in {directory}")
    return sorted(cases, key=lambda c: c.order)


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--cases", required=True, help=f"directory of {CASE_GLOB} files")
    parser.add_argument("--output-dir", default="board_matrix_results")
    parser.add_argument("--lengths", type=int, nargs="*", help="keep only these seq_len values")
    parser.add_argument("--causal-only", action="store_true")
    parser.add_argument("--numerics", default="kv260", choices=("kv260", "exact"))
    parser.add_argument("--timeout-ms", type=int, default=None)
    args = parser.parse_args(argv)

    case_dir = Path(args.cases)
    out_dir = Path(args.output_dir)
    inputs = out_dir / "inputs"
    inputs.mkdir(parents=True, exist_ok=True)
    cases = select(case_dir, args.lengths, args.causal_only)
    records = []
    for n, case in enumerate(cases, start=1):
        copy = inputs / case.path.name
        shutil.copy2(case.path, copy)
        try:
            rec = run_one(case, args.numerics, args.timeout_ms, out_dir)
        except (RuntimeError, ValueError, TimeoutError) as exc:  # recorded; the matrix goes on
            rec = {"case": case.path.name, "passed": False, "exception": f"{type(exc).__name__}: {exc}"}
        rec.update(input=str(copy), input_sha256=digest(case.path))
        diff = rec.get("difference")
        note = ("ok" if rec["passed"] else rec.get("exception") or
                f"{diff['count']} words differ" + (f", first at {diff['first_index']} (gpu {diff['gpu_word']}, "
                                                   f"expected {diff['expected_word']})" if "first_index" in diff else ""))
        print(f"case {n}/{len(cases)} {case.path.name} (L={case.seq_len}, causal={case.causal}): {note}", flush=True)
        records.append(rec)

    (out_dir / "summary.json").write_text(json.dumps(records, indent=2) + "\n", encoding="utf-8")
    settings = {"cases_dir": str(case_dir.resolve()), "results_dir": str(out_dir.resolve()), "numerics": args.numerics,
                "length_filter": sorted(set(args.lengths)) if args.lengths else None,
                "causal_filter": True if args.causal_only else None}
    (out_dir / "manifest.json").write_text(json.dumps({**settings, "cases": records}, indent=2) + "\n",
                                           encoding="utf-8")
    matched = sum(r["passed"] for r in records)
    print(f"{matched} of {len(records)} board cases match word for word", flush=True)
    return 0 if matched == len(records) else 1


if __name__ == "__main__":
    raise SystemExit(main())
