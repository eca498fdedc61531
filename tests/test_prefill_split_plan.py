"""The attention split plan shared by the prompt-attention kernel and its
launcher (qwen3-iree_amd/csrc/prefill_split.h), checked by brute force: the
header is compiled with g++ into a small program that enumerates each query
block's cache positions directly."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_split_plan_matches_enumeration(tmp_path):
    exe = tmp_path / "split_plan_check"
    subprocess.run(["g++", "-O1", "-std=c++17", f"-I{REPO / 'qwen3-iree_amd' / 'csrc'}",
                    str(REPO / "tests" / "native" / "split_plan_check.cpp"), "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok")
