"""Host logic of the paged K/V cache allocator (lara_amd/csrc/page_table.h) on the CPU.

tests/page_table_check.cpp exercises reservation growth and limits, all-or-nothing failure
when the pool is short, release and reuse, least-recently-used eviction with pinned
sequences, coverage queries, and 20 000 random operations that must keep every page either
free or mapped exactly once.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_page_table_allocator(tmp_path):
    exe = tmp_path / "page_table_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'lara_amd' / 'csrc'}",
                    str(ROOT / "tests" / "page_table_check.cpp"), "-o", str(exe)], check=True, timeout=120)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip() == "ok"
