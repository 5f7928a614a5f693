"""Writes the top-k sampler fixture.

  python tests/golden/make_sampler_fixtures.py
Writes, next to this script:
  sampler_reference.json   for each case (vocabulary V, top_k, temperature,
                           mt19937 seed; logits = oracle normal(V, seed
                           LOGIT_SEED + case index) * 2): the tokens the
                           reference's inference::sample_top_k
                           (include/inference.h:14-43) returns on DRAWS calls
                           on one std::mt19937, and the uniform each call's
                           std::discrete_distribution drew (hex doubles), via
                           oracle/_ref/ref_sampler_tool (needs the reference
                           tree: make -C oracle ref)
"""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "tests"))
TOOL = ROOT / "oracle" / "_ref" / "ref_sampler_tool"

LOGIT_SEED = 7000
DRAWS = 200
# (V, top_k, temperature, mt19937 seed); top_k 0 and > V exercise the clamp
CASES = [(2048, 40, 0.6, 1), (2048, 5, 1.0, 2), (2048, 1, 0.6, 3), (2048, 2048, 1.7, 4),
         (2048, 0, 0.9, 5), (300, 3000, 1.3, 6), (97, 12, 0.35, 7), (2048, 64, 2.5, 8)]


def logits_for(index: int, vocab: int):
    import oracle_lib as O
    return O.normal((vocab,), LOGIT_SEED + index, 0.0, 2.0)


def run_reference(index: int, case) -> dict:
    vocab, top_k, temperature, seed = case
    x = logits_for(index, vocab)
    text = "\n".join(float(v).hex() for v in x)
    out = subprocess.run([str(TOOL), str(vocab), str(top_k), repr(temperature), str(seed),
                          str(DRAWS)], input=text, capture_output=True, text=True,
                         check=True).stdout.split()
    return {"vocab": vocab, "top_k": top_k, "temperature": temperature, "seed": seed,
            "tokens": [int(t) for t in out[0::2]], "uniforms": out[1::2]}


def main() -> int:
    if not TOOL.exists():
        print(f"{TOOL} is not built (make -C oracle ref)", file=sys.stderr)
        return 1
    cases = [run_reference(i, c) for i, c in enumerate(CASES)]
    (HERE / "sampler_reference.json").write_text(
        json.dumps({"logit_seed": LOGIT_SEED, "draws": DRAWS, "cases": cases}) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
