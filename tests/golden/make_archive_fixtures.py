"""Writes the checkpoint-archive fixtures from the reference's own code.

Run in a tree where oracle/_ref is built (make -C oracle ref dropin):
  python tests/golden/make_archive_fixtures.py
Writes, next to this script:
  reference_archive.arc          the fixed test archive written by the
                                 reference's Archive (src/model_utils/
                                 archive.cpp) via oracle/_ref/archive_tool
  reference_archive_dump.txt     its entries (name, size, FNV-1a 64)
  gpt_archive_layout.json        Compiled::save + save_optimisers of the
                                 reference nn::GPT (V 96, T 24, d 64, 2 heads,
                                 4 blocks) after two AdamW steps: per archive
                                 index the shape and the canonical parameter
                                 index, and every entry name with its size
                                 (oracle/_ref/dropin_gpt --archive-layout)
"""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REF = HERE.parents[1] / "oracle" / "_ref"


def main() -> int:
    tool, dropin = REF / "archive_tool", REF / "dropin_gpt"
    if not tool.exists() or not dropin.exists():
        print("oracle/_ref/archive_tool and dropin_gpt are needed", file=sys.stderr)
        return 1
    arc = HERE / "reference_archive.arc"
    subprocess.run([str(tool), "write", str(arc)], check=True)
    dump = subprocess.run([str(tool), "dump", str(arc)], check=True, capture_output=True,
                          text=True).stdout
    (HERE / "reference_archive_dump.txt").write_text(dump)
    out = subprocess.run([str(dropin), "--archive-layout"], check=True, capture_output=True,
                         text=True).stdout
    layout = json.loads(out.split("ARCHIVE LAYOUT", 1)[1])
    (HERE / "gpt_archive_layout.json").write_text(json.dumps(layout, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
