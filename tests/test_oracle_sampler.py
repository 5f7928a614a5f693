"""The oracle's top-k sampler (orc_sample_top_k) against the reference's own
inference::sample_top_k (include/inference.h:14-43) and against what the
mathematics fixes (host only, no GPU).

Pins:
  * tests/golden/sampler_reference.json holds the reference's tokens for 200
    calls per case on one std::mt19937, with the uniform each call's
    std::discrete_distribution drew (written through oracle/_ref/
    ref_sampler_tool by tests/golden/make_sampler_fixtures.py); fed the same
    uniforms, the oracle returns the same tokens. When the tool is built the
    same comparison also runs live on fresh seeds;
  * top_k 1 is the lowest-index argmax; top_k 0 and top_k > V clamp;
  * over many SplitMix64 draws the token frequencies follow
    softmax(logits / temperature) restricted to the top k;
  * the EOS re-draw (inference.h:80-84) never returns EOS while draws are
    left, and a row's draws are the stream's next outputs.
"""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = json.loads((ROOT / "tests" / "golden" / "sampler_reference.json").read_text())
TOOL = ROOT / "oracle" / "_ref" / "ref_sampler_tool"


def _oracle_tokens(x, top_k, temperature, uniforms):
    u = np.array([float.fromhex(h) for h in uniforms])
    # one row per call: the same logits row (stride 0), one uniform each
    tokens, draws = O.sample_top_k(x, top_k, temperature, uniforms=u, row_stride=0)
    assert np.all(draws == 1)
    return tokens


@pytest.mark.parametrize("index", range(len(GOLDEN["cases"])))
def test_matches_reference_golden(index):
    c = GOLDEN["cases"][index]
    x = O.normal((c["vocab"],), GOLDEN["logit_seed"] + index, 0.0, 2.0)
    got = _oracle_tokens(x, c["top_k"], c["temperature"], c["uniforms"])
    np.testing.assert_array_equal(got, c["tokens"])


@pytest.mark.skipif(not TOOL.exists(), reason="oracle/_ref/ref_sampler_tool not built")
@pytest.mark.parametrize("vocab,top_k,temperature,seed", [(2048, 40, 0.6, 91), (512, 7, 1.4, 92),
                                                          (2048, 2048, 0.8, 93)])
def test_matches_reference_live(vocab, top_k, temperature, seed):
    x = O.normal((vocab,), 8000 + seed, 0.0, 1.5)
    out = subprocess.run([str(TOOL), str(vocab), str(top_k), repr(temperature), str(seed), "300"],
                         input="\n".join(float(v).hex() for v in x), capture_output=True,
                         text=True, check=True).stdout.split()
    got = _oracle_tokens(x, top_k, temperature, out[1::2])
    np.testing.assert_array_equal(got, [int(t) for t in out[0::2]])


def test_top1_is_lowest_index_argmax_and_clamps():
    x = O.normal((5, 333), 8100, 0.0, 1.0)
    x[2, 10] = x[2, 200] = x[2].max() + 1.0  # a tie: the lower index wins
    for k in (0, 1):
        tokens, _ = O.sample_top_k(x, k, 0.7, seed=3)
        assert list(tokens) == [O.argmax(r) for r in x]
    assert tokens[2] == 10
    a, _ = O.sample_top_k(x, 333, 1.1, seed=4, counter=9)
    b, _ = O.sample_top_k(x, 5000, 1.1, seed=4, counter=9)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("top_k,temperature", [(5, 0.8), (8, 1.0), (3, 2.0)])
def test_frequencies_follow_tempered_softmax(top_k, temperature):
    x = np.array([0.3, 2.0, -1.0, 1.2, 0.9, 1.7, -0.4, 0.0], np.float32)
    n = 40000
    # n calls on the same row: row r uses the stream's output r + 1
    tokens, _ = O.sample_top_k(np.tile(x, (n, 1)), top_k, temperature, seed=77)
    order = np.argsort(-x, kind="stable")[:top_k]
    p = np.exp((x[order] - x[order[0]]) / temperature)
    p /= p.sum()
    freq = np.array([(tokens == t).sum() for t in order]) / n
    assert set(np.unique(tokens)) <= set(order.tolist())
    sigma = np.sqrt(p * (1 - p) / n)
    assert np.all(np.abs(freq - p) <= 5 * sigma + 1e-12), (freq, p)


def test_eos_redraw_and_draw_stream():
    x = np.array([3.0, 2.5, 2.4, -5.0], np.float32)  # EOS = token 0 dominates
    n = 20000
    tokens, draws = O.sample_top_k(np.tile(x, (n, 1)), 3, 1.0, seed=5, eos=0, resample_eos=True,
                                   max_draws=64)
    assert not np.any(tokens == 0)
    p = np.exp(x[:3] - x[0])
    p /= p.sum()
    # draws per row are geometric with success 1 - p(EOS)
    assert abs(draws.mean() - 1 / (1 - p[0])) < 0.05 * (1 / (1 - p[0]))
    # row r's d-th draw is output counter + r*max_draws + d + 1 of the stream:
    # row 1 at counter 0 equals row 0 at counter max_draws
    t1, d1 = O.sample_top_k(np.tile(x, (2, 1)), 3, 1.0, seed=5, eos=0, resample_eos=True,
                            max_draws=64)
    t2, d2 = O.sample_top_k(x, 3, 1.0, seed=5, counter=64, eos=0, resample_eos=True,
                            max_draws=64)
    assert (t1[1], d1[1]) == (t2[0], d2[0])
    # without the re-draw EOS comes back at its probability
    tokens, draws = O.sample_top_k(np.tile(x, (n, 1)), 3, 1.0, seed=6, eos=0)
    assert np.all(draws == 1)
    assert abs((tokens == 0).mean() - p[0]) < 5 * np.sqrt(p[0] * (1 - p[0]) / n)
    # top_k 1 on the EOS argmax: every draw is EOS, the cap ends the loop
    tokens, draws = O.sample_top_k(x, 1, 1.0, seed=7, eos=0, resample_eos=True, max_draws=16)
    assert tokens[0] == 0 and draws[0] == 16
