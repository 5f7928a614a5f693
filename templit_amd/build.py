"""Build recipe for the native parts of templit_amd.

Produces, in-tree (so the built files travel with the source tree):
  templit_amd/libtemplit_hip.so     hand-written gfx950 HIP kernels + C-ABI
  templit_amd/libtemplit_runtime.so hip::Runtime / Storage<hip::HIP,T> (host C++
                                    over the C-ABI)
  templit_amd/libtemplit_gpt.so     GPT step program (host C++ over the C-ABI)
  tests/cpp/bin/test_*              C++ tests of the runtime surface

Run:  python -m templit_amd.build   (or __graft_entry__.build()).
Every call recompiles (objects are cached by content hash of the source
and flags, so unchanged files are not rebuilt).
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
INCLUDE = ROOT / "include"
PKG_INCLUDE = PKG / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    # Packed fp32 instructions stay disabled: hipcc -O3 would otherwise form
    # v_pk_{add,mul,fma}_f32 from plain float code, and some of their forms
    # have produced silently wrong results on MI355X.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{PKG_INCLUDE}",
    f"-I{CSRC}",
]

KERNEL_SOURCES = [
    "api.hip",
    "gemm.hip",
    "elementwise.hip",
    "reduce.hip",
    "rowops.hip",
    "embedding.hip",
    "attention.hip",
    "optim.hip",
    "sample.hip",
]

RUNTIME_SOURCES = [
    "hip_context.cpp",
    "runtime.cpp",
    "archive.cpp",
    "dataset.cpp",
    "loader.cpp",
]

GPT_SOURCES = [
    "gpt_program.cpp",
]

HOST_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{PKG_INCLUDE}",
              f"-I{CSRC}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and line.strip()
        and "warning: argument unused" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _digest(paths: list[Path], flags: list[str]) -> str:
    h = hashlib.sha256()
    for p in paths:
        h.update(p.read_bytes())
    h.update(" ".join(flags).encode())
    return h.hexdigest()[:16]


def _headers() -> list[Path]:
    hs = sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))
    hs += sorted(PKG_INCLUDE.rglob("*.h")) + sorted((ROOT / "tests" / "cpp").glob("*.h"))
    return hs


def _compile(src: Path, flags: list[str], compiler: str) -> Path:
    BUILD.mkdir(exist_ok=True)
    key = _digest([src] + _headers(), flags + [compiler])
    obj = BUILD / f"{src.stem}.{key}.o"
    if not obj.exists():
        tmp = obj.with_suffix(".o.tmp")
        _run([compiler, *flags, "-c", str(src), "-o", str(tmp)])
        tmp.replace(obj)
    return obj


def build_kernels(jobs: int = 8) -> Path:
    srcs = [CSRC / s for s in KERNEL_SOURCES if (CSRC / s).exists()]
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, HIP_FLAGS, HIPCC), srcs))
    lib = PKG / "libtemplit_hip.so"
    tmp = PKG / "libtemplit_hip.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), "-L/opt/rocm/lib", "-lrocprofiler-sdk-roctx",
          "-Wl,-rpath,/opt/rocm/lib"])
    tmp.replace(lib)
    return lib


def build_runtime(kernel_lib: Path) -> Path:
    objs = [_compile(CSRC / s, HOST_FLAGS, "g++") for s in RUNTIME_SOURCES]
    lib = PKG / "libtemplit_runtime.so"
    tmp = PKG / "libtemplit_runtime.so.tmp"
    _run(["g++", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          f"-L{PKG}", "-ltemplit_hip", "-Wl,-rpath,$ORIGIN"])
    tmp.replace(lib)
    return lib


def build_gpt(kernel_lib: Path) -> Path | None:
    srcs = [CSRC / s for s in GPT_SOURCES if (CSRC / s).exists()]
    if not srcs:
        return None
    objs = [_compile(s, HOST_FLAGS, "g++") for s in srcs]
    lib = PKG / "libtemplit_gpt.so"
    tmp = PKG / "libtemplit_gpt.so.tmp"
    _run(["g++", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          f"-L{PKG}", "-ltemplit_runtime", "-ltemplit_hip", "-Wl,-rpath,$ORIGIN"])
    tmp.replace(lib)
    return lib


def build_cpp_tests() -> list[Path]:
    tdir = ROOT / "tests" / "cpp"
    bindir = tdir / "bin"
    bindir.mkdir(exist_ok=True)
    out = []
    for src in sorted(tdir.glob("test_*.cpp")):
        exe = bindir / src.stem
        obj = _compile(src, HOST_FLAGS + [f"-I{tdir}"], "g++")
        tmp = exe.with_suffix(".tmp")
        _run(["g++", "-o", str(tmp), str(obj), f"-L{PKG}", "-ltemplit_runtime",
              "-ltemplit_hip", "-Wl,-rpath,$ORIGIN/../../../templit_amd"])
        tmp.replace(exe)
        out.append(exe)
    return out


# Host AddressSanitizer + UndefinedBehaviorSanitizer builds of the C++ test
# programs and the host sources they exercise (archive, dataset, loader, the
# runtime's no-device path), as the reference builds by default
# (CMakeLists.txt:8,18-27). g++ only: no device code is built with them.
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-fno-omit-frame-pointer", "-g"]
SAN_SOURCES = {
    "test_archive": ["archive.cpp"],
    "test_loader": ["dataset.cpp", "loader.cpp"],
    "test_hip_runtime": ["runtime.cpp", "hip_context.cpp", "archive.cpp", "dataset.cpp",
                         "loader.cpp"],
}


def build_sanitized_tests() -> list[Path]:
    tdir = ROOT / "tests" / "cpp"
    bindir = tdir / "bin" / "san"
    bindir.mkdir(parents=True, exist_ok=True)
    flags = HOST_FLAGS + SAN_FLAGS + [f"-I{tdir}"]
    out = []
    for name, sources in SAN_SOURCES.items():
        objs = [_compile(tdir / f"{name}.cpp", flags, "g++")]
        objs += [_compile(CSRC / src, flags, "g++") for src in sources]
        exe = bindir / name
        tmp = exe.with_suffix(".tmp")
        _run(["g++", *SAN_FLAGS, "-o", str(tmp), *map(str, objs), f"-L{PKG}", "-ltemplit_hip",
              "-Wl,-rpath,$ORIGIN/../../../../templit_amd"])
        tmp.replace(exe)
        out.append(exe)
    return out


def clean_stale_objects() -> None:
    if not BUILD.exists():
        return
    by_stem: dict[str, list[Path]] = {}
    for o in BUILD.glob("*.o"):
        by_stem.setdefault(o.name.split(".")[0], []).append(o)
    for objs in by_stem.values():
        objs.sort(key=lambda p: p.stat().st_mtime, reverse=True)
        for stale in objs[3:]:
            stale.unlink(missing_ok=True)


def build_all() -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    lib = build_kernels()
    build_runtime(lib)
    build_gpt(lib)
    build_cpp_tests()
    build_sanitized_tests()
    clean_stale_objects()


if __name__ == "__main__":
    build_all()
    print("built", PKG / "libtemplit_hip.so")
