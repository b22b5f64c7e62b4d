"""Golden fixtures (CPU): the reference's BD3 mask cases and the oracle's
summarised logits on them (``tests/golden/make_golden.py`` wrote both)."""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
sys.path.insert(0, GOLDEN)

import make_golden  # noqa: E402

from oracle import ops as O  # noqa: E402


def _cases():
    with open(os.path.join(GOLDEN, "bd3_mask_cases.json")) as f:
        return json.load(f)["cases"]


def test_reference_cases_are_staircase_cases():
    """Every case: masked positions hold the BD3 mask id, selected rows lie inside
    the canvas, and the staircase allow-relation of the reference's eager
    oracle (key block <= query block, model_coverage/reference.py:158-180)
    equals the d2f_hybrid mask at prompt_len 0, block 32."""
    cases = _cases()
    assert [c["name"] for c in cases] == ["absolute_block_boundary_rows",
                                          "multi_mask_cross_block", "qk_norm_gqa_absolute_blocks"]
    for c in cases:
        ids = c["input_ids"]
        assert all(ids[p] == 151669 for p in c["masked_positions"])
        assert all(0 <= r < len(ids) for r in c["selected_rows"])
        n = len(ids)
        blocks = np.arange(n) // 32
        staircase = blocks[None, :] <= blocks[:, None]
        np.testing.assert_array_equal(O.d2f_visible(np.arange(n), n, prompt_len=0,
                                                    block_size=32), staircase)
    # the cases straddle absolute block boundaries (rows 31 | 32)
    assert {31, 32} <= set(cases[0]["selected_rows"])


def test_oracle_reproduces_its_golden_summaries():
    with open(os.path.join(GOLDEN, "bd3_real_vocab_logits.json")) as f:
        gold = json.load(f)
    g = make_golden.real_vocab_geometry()
    from diffusorrt_amd import synthetic as syn

    model = syn.build_model(g, "q4", seed=gold["seed"])
    for c in _cases():
        got = make_golden.summarise(make_golden.oracle_case_logits(model, "q4", c))
        want = gold["kinds"]["q4"][c["name"]]
        for gr, wr in zip(got, want):
            assert gr["argmax"] == wr["argmax"]
            np.testing.assert_allclose([gr["score"], gr["lse"], gr["max"]],
                                       [wr["score"], wr["lse"], wr["max"]], rtol=1e-5)
            np.testing.assert_allclose(gr["probe"], wr["probe"], rtol=1e-4, atol=1e-5)
