"""hip::Runtime (the C++ runtime surface) through its C++ test program,
tests/cpp/test_hip_runtime.cpp: the reference's Metal-runtime known-answer
tests restated, validation, in-place use, graph mode, batched products.

The GPU test runs the whole program; the CPU test checks that the runtime
reports a missing GPU as an error instead of crashing.
"""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BIN = ROOT / "tests" / "cpp" / "bin" / "test_hip_runtime"


def _run(*args, timeout=180):
    if not BIN.exists():
        raise FileNotFoundError(f"{BIN} is not built: run __graft_entry__.build()")
    proc = subprocess.run([str(BIN), *args], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=timeout)
    print(proc.stdout)
    return proc


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible on this machine")
def test_runtime_reports_missing_device():
    proc = _run("--no-device")
    assert proc.returncode == 0, proc.stdout


@pytest.mark.gpu
def test_hip_runtime_program():
    proc = _run()
    assert proc.returncode == 0, proc.stdout
    assert "all hip::Runtime tests passed" in proc.stdout
