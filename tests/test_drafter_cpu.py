"""The drafter's round state machine (csrc/drafter.h) on the CPU: compiled with a
host backend whose head records its inputs, checked against the reference's
round semantics (Runner/Qwen4ExpMTPDrafter.swift:162-475): backlog pairing
across observed chunks, the trusted flush, speculative steps and their rollback,
finalize/discard bookkeeping, the depth ceiling and every refused call."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mlxfast-qwen38-125b-a6b-engine_amd", "csrc")


def test_drafter_state_machine_host(tmp_path):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    exe = tmp_path / "drafter_host_test"
    src = os.path.join(ROOT, "tests", "cpp", "drafter_host_test.cpp")
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", CSRC, src, "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert "ok" in r.stdout
