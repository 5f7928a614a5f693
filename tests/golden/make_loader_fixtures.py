"""Writes the dataset / loader fixtures.

  python tests/golden/make_loader_fixtures.py
Writes, next to this script:
  loader_tokens.tokens           3,001 synthetic token ids (uint32, native
                                 order) in [0, 2048) with the end-of-sequence
                                 id 256 every 37-163 tokens
  loader_text.txt                synthetic text with blank lines
  loader_reference_output.txt    the reference's Dataset / Loader
                                 (src/model_utils/dataset.cpp, loader.cpp)
                                 on the fixed checks of
                                 tests/cpp/loader_tool_content.h, through
                                 oracle/_ref/loader_tool (needs the
                                 reference tree: make -C oracle ref)
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
TOOL = HERE.parents[1] / "oracle" / "_ref" / "loader_tool"


def main() -> int:
    rng = np.random.default_rng(2024)
    tokens = rng.integers(0, 2048, 3001, dtype=np.uint32)
    i = 0
    while True:
        i += int(rng.integers(37, 164))
        if i >= tokens.size:
            break
        tokens[i] = 256
    (HERE / "loader_tokens.tokens").write_bytes(tokens.astype("<u4").tobytes())
    words = ["tensor", "kernel", "wave", "tile", "stream", "graph", "block", "lane"]
    paras = []
    for p in range(12):
        lines = [" ".join(words[(p * 7 + k * 3 + j) % len(words)] for j in range(5 + k % 4))
                 for k in range(1 + p % 3)]
        paras.append("\n".join(lines))
    (HERE / "loader_text.txt").write_text("\n\n".join(paras) + "\n")
    if not TOOL.exists():
        print("oracle/_ref/loader_tool is needed for the reference output", file=sys.stderr)
        return 1
    out = subprocess.run([str(TOOL), str(HERE / "loader_tokens.tokens"),
                          str(HERE / "loader_text.txt")], check=True, capture_output=True,
                         text=True).stdout
    (HERE / "loader_reference_output.txt").write_text(out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
