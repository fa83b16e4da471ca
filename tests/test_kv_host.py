"""The host prefix registry and block hash (flour_amd/csrc/kv_host.h) checked directly, in C++:
the reference's prefix.rs tests restated on this build's own hash and registry. A simulated hash
collision (same hash, other tokens) must be a miss, which the public cache API cannot provoke
(its 64-bit hashes never collide in a test). Built with g++ from tests/native/kv_host_check.cpp."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_block_hash_and_registry_prefix_rs_64_80(tmp_path):
    exe = tmp_path / "kv_host_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-I", str(ROOT / "flour_amd" / "csrc"),
                    str(ROOT / "tests" / "native" / "kv_host_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
