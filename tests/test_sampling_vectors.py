"""The oracle's temperature sampler against vectors the reference's own sampler wrote.

``tests/golden/sampling_vectors.json`` was produced by
``tests/golden/make_sampling_vectors.py`` from
``backends/diffusion_runtime.py:203-275`` of the reference (``sampling_noise`` and
``_sampled_max_prob_confidence``). It pins the key chaining of the counter hash
(seed, forward, position, token), the 23-bit uniform and the Gumbel transform; the
GPU sampler is then checked against the oracle on the device's own logits
(``tests/test_gpu_ops.py``).
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from oracle import ops as O

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def vectors():
    with open(os.path.join(HERE, "golden", "sampling_vectors.json")) as f:
        return json.load(f)


def _logits(case, i):
    if "logits_bits" in case:
        return np.asarray(case["logits_bits"], dtype=np.uint32).view(np.float32)
    rng = np.random.default_rng(2026 + case["logits_rng"]["case"])
    return (rng.standard_normal((case["rows"], case["vocab"])) * 2.0).astype(np.float32)


def test_noise_matches_reference_bits(vectors):
    for row in vectors["noise"]:
        got = O.sampling_noise(int(row["seed"]), row["step"], row["position"], row["vocab"])
        want = np.asarray(row["bits"], dtype=np.uint32)
        assert got.dtype == np.float32
        assert np.array_equal(got.view(np.uint32), want), (row["seed"], row["step"],
                                                            row["position"])


def test_vectors_separate_the_key_fields(vectors):
    """The fixture can catch a chaining mistake: keys that differ only in which
    field holds a value (step vs position, seed vs step) give different noise."""
    rows = {(r["seed"], r["step"], r["position"]): r["bits"] for r in vectors["noise"]}
    assert rows[("0", 1, 0)] != rows[("0", 0, 1)]
    assert rows[("1", 0, 0)] != rows[("0", 1, 0)]
    assert rows[("0", 0, 0)] != rows[("0", 0, 1)]


def test_sampled_tokens_and_scores_match_reference(vectors):
    for i, case in enumerate(vectors["sampled"]):
        logits = _logits(case, i)
        scores, tokens = O.sampled_max_prob(logits, temperature=case["temperature"],
                                            seed=int(case["seed"]), step=case["step"],
                                            positions=case["positions"])
        assert tokens == case["tokens"], i
        np.testing.assert_allclose(scores, case["scores"], rtol=1e-12, atol=0)
