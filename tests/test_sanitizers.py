"""Host AddressSanitizer + UndefinedBehaviorSanitizer runs (CPU only), as
the reference builds its programs by default (CMakeLists.txt:8,18-27).

Built by __graft_entry__.build() with g++ -fsanitize=address,undefined
-fno-sanitize-recover=all (no device code is instrumented):
  - tests/cpp/bin/san/test_archive, test_loader: the checkpoint archive and
    the token dataset / loader on the reference's golden fixtures;
  - tests/cpp/bin/san/test_hip_runtime --no-device: hip::init's error path;
  - oracle/_asan/liboracle.so and oracle/_ref/asan/libref_cpu.so: the
    oracle's known-answer, mathematical and reference-runtime tests re-run
    in a child Python with the sanitizer runtime preloaded.
Any sanitizer report aborts the program, so each check is its exit status
plus the normal expected output.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SAN = ROOT / "tests" / "cpp" / "bin" / "san"
GOLDEN = ROOT / "tests" / "golden"
ORACLE_ASAN = ROOT / "oracle" / "_asan" / "liboracle.so"
REF_ASAN = ROOT / "oracle" / "_ref" / "asan" / "libref_cpu.so"


def _runtime(name: str) -> str:
    return subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True,
                          check=True).stdout.strip()


def _env(**extra) -> dict:
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "halt_on_error=1:abort_on_error=0:detect_leaks=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env.update(extra)
    return env


def _run(exe: Path, *args, env=None) -> subprocess.CompletedProcess:
    if not exe.exists():
        pytest.skip(f"{exe} not built (run __graft_entry__.build())")
    return subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True,
                          env=env or _env(), timeout=300)


def test_archive_under_sanitizers(tmp_path):
    proc = _run(SAN / "test_archive", "dump", GOLDEN / "reference_archive.arc")
    assert proc.returncode == 0, proc.stderr
    assert proc.stdout == (GOLDEN / "reference_archive_dump.txt").read_text()
    out = tmp_path / "ours.arc"
    proc = _run(SAN / "test_archive", "write", out)
    assert proc.returncode == 0, proc.stderr
    proc = _run(SAN / "test_archive", "dump", out)
    assert proc.returncode == 0, proc.stderr


def test_dataset_and_loader_under_sanitizers(tmp_path):
    proc = _run(SAN / "test_loader", GOLDEN / "loader_tokens.tokens", GOLDEN / "loader_text.txt")
    assert proc.returncode == 0, proc.stderr
    assert proc.stdout == (GOLDEN / "loader_reference_output.txt").read_text()
    text = tmp_path / "t.txt"
    text.write_bytes(b"ab\n\ncd\n\n\nef" * 30000)  # several 64 KiB read chunks
    proc = _run(SAN / "test_loader", "--text-to-tokens", text, tmp_path / "t.tokens")
    assert proc.returncode == 0, proc.stderr


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is visible on this machine")
def test_runtime_without_device_under_sanitizers():
    # the HIP runtime library is not instrumented and keeps allocations for
    # the process lifetime: leak checking is for the instrumented code only
    proc = _run(SAN / "test_hip_runtime", "--no-device",
                env=_env(ASAN_OPTIONS="halt_on_error=1:detect_leaks=0"))
    assert proc.returncode == 0, proc.stdout + proc.stderr


def test_oracle_tests_under_sanitizers():
    if not ORACLE_ASAN.exists():
        pytest.skip("oracle/_asan/liboracle.so not built (make -C oracle asan)")
    env = _env(
        LD_PRELOAD=_runtime("libasan.so"),
        # the interpreter itself is not instrumented and leaks by design
        ASAN_OPTIONS="halt_on_error=1:detect_leaks=0:verify_asan_link_order=0",
        TEMPLIT_ORACLE_LIB=str(ORACLE_ASAN),
        TEMPLIT_REF_CPU_LIB=str(REF_ASAN if REF_ASAN.exists() else ROOT / "missing"),
    )
    files = ["tests/test_oracle_kats.py", "tests/test_oracle_math.py",
             "tests/test_oracle_sampler.py"]
    if REF_ASAN.exists():
        files.append("tests/test_oracle_vs_reference.py")
    proc = subprocess.run([sys.executable, "-m", "pytest", *files, "-q", "-x", "-m", "not gpu",
                           "-p", "no:cacheprovider"], cwd=ROOT, capture_output=True, text=True,
                          env=env, timeout=600)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-4000:]
    assert " passed" in proc.stdout


def test_sanitizer_catches_a_planted_overflow():
    # the instrumented oracle writing 64 floats past a 16-float output must
    # be reported, so the passing runs above mean something
    if not ORACLE_ASAN.exists():
        pytest.skip("oracle/_asan/liboracle.so not built (make -C oracle asan)")
    script = (
        "import ctypes, numpy as np\n"
        f"lib = ctypes.CDLL({str(ORACLE_ASAN)!r})\n"
        "x = np.ones(80, np.float32); out = np.empty(16, np.float32)\n"
        "lib.orc_unary(2, x.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p),"
        " ctypes.c_size_t(80))\n"
    )
    env = _env(LD_PRELOAD=_runtime("libasan.so"),
               ASAN_OPTIONS="halt_on_error=1:detect_leaks=0:verify_asan_link_order=0")
    proc = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                          env=env, timeout=120)
    assert proc.returncode != 0
    assert "AddressSanitizer" in proc.stderr and "heap-buffer-overflow" in proc.stderr
