"""The device pool's block bookkeeping (split, merge, segment recycling
under memory pressure), fuzzed on the CPU: the pool header is compiled with
g++ and sanitizers against a host policy that hands out address ranges of a
bounded device."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_pool_fuzz(tmp_path):
    exe = tmp_path / "pool_fuzz"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", str(HERE / "native" / "pool_fuzz.cpp"),
                    "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.count("ok ") == 2, out.stdout
