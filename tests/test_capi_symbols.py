"""The C-ABI libraries load on a CPU-only machine and export every entry
point their headers in include/ declare (no compute calls: no GPU here)."""
import ctypes
import re
from pathlib import Path

import pytest

from templit_amd import native

ROOT = Path(__file__).resolve().parents[1]
DECL = re.compile(r"^[A-Za-z_][\w\s\*]*?\b(tl[hg]_\w+)\s*\(", re.M)


def declared(header: str) -> list[str]:
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(DECL.findall(text)))


def test_kernel_library_exports_every_declared_symbol():
    names = declared("templit_hip.h")
    assert len(names) > 50
    lib = ctypes.CDLL(str(native.HIP_LIB))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_bindings_cover_the_header():
    names = set(declared("templit_hip.h")) - {"tlh_error_string"}
    assert names == set(native.HIP_SIGNATURES), (
        names ^ set(native.HIP_SIGNATURES))
    native.load_hip()  # declares argtypes for every symbol


@pytest.mark.skipif(not (ROOT / "include" / "templit_gpt.h").exists(), reason="no GPT header")
def test_gpt_library_exports_every_declared_symbol():
    names = declared("templit_gpt.h")
    lib = ctypes.CDLL(str(native.GPT_LIB))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
