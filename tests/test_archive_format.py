"""Checkpoint archive parity (host only, no GPU).

The file layout is pinned by the reference's own Archive
(src/model_utils/archive.cpp:9-92): tests/golden/reference_archive.arc and
its dump were written by it (tests/golden/make_archive_fixtures.py, through
oracle/_ref/archive_tool), and when oracle/_ref/archive_tool is built the
reference also reads what templit_amd writes. The GPT checkpoint order and
shapes are pinned by the reference executor's Compiled::save /
save_optimisers (include/passes/compile.h:259-299) over nn::GPT:
tests/golden/gpt_archive_layout.json.
"""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

from templit_amd.native import GptConfig, NativeError, archive_entry

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
OURS = ROOT / "tests" / "cpp" / "bin" / "test_archive"
REF_TOOL = ROOT / "oracle" / "_ref" / "archive_tool"


def run(*args) -> str:
    return subprocess.run([str(a) for a in args], check=True, capture_output=True,
                          text=True).stdout


def test_reads_the_reference_file():
    expect = (GOLDEN / "reference_archive_dump.txt").read_text()
    assert run(OURS, "dump", GOLDEN / "reference_archive.arc") == expect


def test_writes_the_reference_content(tmp_path):
    path = tmp_path / "ours.arc"
    run(OURS, "write", path)
    expect = (GOLDEN / "reference_archive_dump.txt").read_text()
    assert run(OURS, "dump", path) == expect
    # same entries, so the same number of bytes; entries sorted by name
    assert path.stat().st_size == (GOLDEN / "reference_archive.arc").stat().st_size
    if REF_TOOL.exists():
        assert run(REF_TOOL, "dump", path) == expect


def test_truncated_file_keeps_the_whole_entries(tmp_path):
    data = (GOLDEN / "reference_archive.arc").read_bytes()
    path = tmp_path / "cut.arc"
    path.write_bytes(data[: len(data) - 5])  # the last entry loses its tail
    lines = (GOLDEN / "reference_archive_dump.txt").read_text().splitlines()
    got = run(OURS, "dump", path).splitlines()
    assert len(got) == len(lines) - 1 and set(got) <= set(lines)


def test_gpt_checkpoint_layout_matches_the_reference():
    layout = json.loads((GOLDEN / "gpt_archive_layout.json").read_text())
    c = layout["config"]
    cfg = GptConfig(c["vocab"], c["seq"], c["dim"], c["heads"], c["layers"], 1, c["ffn"])
    for i, entry in enumerate(layout["parameters"]):
        canonical, shape = archive_entry(cfg, i)
        assert shape == tuple(entry["shape"]), i
        if entry["canonical"] >= 0:
            assert canonical == entry["canonical"], i
    with pytest.raises(NativeError):
        archive_entry(cfg, len(layout["parameters"]))
    # every entry is a parameter (size, data) or its AdamW state
    per_tensor = {n.split("/", 2)[2] for n, _ in layout["names"]}
    assert per_tensor == {"size", "data", "momentum1/size", "momentum1/data",
                          "momentum2/size", "momentum2/data", "step"}
