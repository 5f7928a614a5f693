"""Token dataset and loader parity (host only, no GPU).

The reference's Dataset / Loader (src/model_utils/dataset.cpp:16-102,
loader.cpp:5-43) wrote tests/golden/loader_reference_output.txt on the
fixed checks of tests/cpp/loader_tool_content.h
(tests/golden/make_loader_fixtures.py via oracle/_ref/loader_tool):
splits, batches for three seeds, the whole-split sample, save/load and
every error path. templit_amd's classes must print the same, and the
C-ABI loader must draw the same batches.
"""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from templit_amd.native import NativeError, TokenLoader

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
TOKENS, TEXT = GOLDEN / "loader_tokens.tokens", GOLDEN / "loader_text.txt"
EXPECT = GOLDEN / "loader_reference_output.txt"


def run(tool) -> str:
    return subprocess.run([str(tool), str(TOKENS), str(TEXT)], check=True, capture_output=True,
                          text=True).stdout


def test_classes_match_the_reference():
    assert run(ROOT / "tests" / "cpp" / "bin" / "test_loader") == EXPECT.read_text()
    ref = ROOT / "oracle" / "_ref" / "loader_tool"
    if ref.exists():
        assert run(ref) == EXPECT.read_text()


def fnv(values: np.ndarray) -> int:
    h = 1469598103934665603
    for x in values.tolist():
        h = ((h ^ x) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


@pytest.mark.parametrize("fraction,name", [(0.95, "tokens 0.95"), (0.5, "tokens 0.5")])
def test_c_abi_loader_draws_the_reference_batches(fraction, name):
    lines = EXPECT.read_text().splitlines()
    for seed in (1, 2, 12345):
        loader = TokenLoader(TOKENS, fraction, seed=seed)
        try:
            for i in range(3):
                x, y = loader.batch(4, 16)
                pat = re.compile(rf"^{re.escape(name)} seed {seed} batch {i}: inputs (\w+) "
                                 rf"targets (\w+)")
                m = next(pat.match(l) for l in lines if pat.match(l))
                assert fnv(x) == int(m.group(1), 16) and fnv(y) == int(m.group(2), 16)
                np.testing.assert_array_equal(x.reshape(4, 16)[:, 1:], y.reshape(4, 16)[:, :-1])
        finally:
            loader.close()


def test_c_abi_loader_errors(tmp_path):
    with pytest.raises(NativeError):
        TokenLoader(tmp_path / "missing.tokens")
    with pytest.raises(NativeError):
        TokenLoader(TOKENS, 1.0)
    odd = tmp_path / "odd.tokens"
    odd.write_bytes(b"abcde")
    with pytest.raises(NativeError):
        TokenLoader(odd)
    loader = TokenLoader(TOKENS, 0.95, validation=True)
    try:
        with pytest.raises(NativeError):  # longer than the 128-token validation split
            loader.batch(1, 200)
        x, _ = loader.batch(2, 8)
        assert x.size == 16
    finally:
        loader.close()


def test_text_decoding_across_read_chunks(tmp_path):
    # Dataset::load_text reads in 64 KiB chunks: blank lines that straddle a
    # chunk boundary, a lone newline ending a chunk and runs of three
    # newlines must decode as in one piece. Expected ids: the text split on
    # non-overlapping "\n\n" (left to right), pieces joined by the
    # end-of-sequence id 256, every other byte its own value.
    chunk = 64 * 1024
    text = bytearray(b"x" * (3 * chunk + 100))
    text[chunk - 1:chunk + 1] = b"\n\n"            # a blank line across the boundary
    text[2 * chunk - 1] = ord("\n")                 # a lone newline ending a chunk
    text[2 * chunk + 10:2 * chunk + 13] = b"\n\n\n"  # three newlines
    text[3 * chunk - 2:3 * chunk + 1] = b"\n\n\n"    # three across the boundary
    text[-1:] = b"\n"
    src, out = tmp_path / "t.txt", tmp_path / "t.tokens"
    src.write_bytes(bytes(text))
    subprocess.run([str(ROOT / "tests" / "cpp" / "bin" / "test_loader"), "--text-to-tokens",
                    str(src), str(out)], check=True)
    expect = []
    for i, piece in enumerate(bytes(text).split(b"\n\n")):
        if i:
            expect.append(256)
        expect.extend(piece)
    np.testing.assert_array_equal(np.fromfile(out, np.uint32), np.array(expect, np.uint32))
