"""A finished block's commit forward merged into the next block's first step.

In a BD3 decode the block before the active one is committed (its K/V written
to the prefix cache) by the forward of the active block's first step: one
64-row forward whose first 32 rows form their own mask segment (they see the
keys up to their block's end, as the separate commit forward does) on the
split-K linears' two row tiles and the four-query-tile decode attention.

At the BD3 (Qwen3-0.6B) layer shapes with a 992-token prompt and three blocks,
every step (the merged forwards eager, captured and replayed) is teacher-forced
against the oracle at the strict bar of the session tests, the commit rows add
up, the native loop reproduces the host loop, and the decode with the commit
kept separate (``DRT_SEPARATE_COMMIT=1``) meets the same bar.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from helpers import compare_proposals, oracle_logits, oracle_weights

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

PROMPT, GEN, BLOCK, STEPS = 992, 96, 32, 24


def _say(*a):
    print("[case]", *a, flush=True)


def _geometry():
    from diffusorrt_amd import synthetic as syn

    return dataclasses.replace(syn.BD3_QWEN3_06B, layer_count=2, vocab_size=4096,
                               mask_token_id=4000, eos_token_id=4001)


def _decode(model, prompt, monkeypatch, separate, native=False):
    from diffusorrt_amd import decode
    from diffusorrt_amd.runtime import Runtime, bd3_session_config

    g = model.geometry
    if separate:
        monkeypatch.setenv("DRT_SEPARATE_COMMIT", "1")
    else:
        monkeypatch.delenv("DRT_SEPARATE_COMMIT", raising=False)
    rt = Runtime(model, max_forward_rows=1024, max_positions=PROMPT + GEN + 64)
    try:
        trace = []
        with rt.session(bd3_session_config(BLOCK, STEPS, PROMPT + GEN)) as s:
            res = decode.generate_device_tokens(
                s, prompt, max_tokens=GEN, mask_token_id=g.mask_token_id,
                eos_token_id=g.eos_token_id, steps=STEPS, block_size=BLOCK, native=native,
                trace=None if native else trace)
            m = s.device_metrics()
        return res, trace, m
    finally:
        monkeypatch.delenv("DRT_SEPARATE_COMMIT", raising=False)
        rt.close()


def _teacher_forced(model, prompt, trace):
    from diffusorrt_amd import synthetic as syn

    geom = model.geometry
    W, cfg = oracle_weights(model), syn.oracle_config(geom, "q4")
    x = list(prompt) + [geom.mask_token_id] * GEN
    problems, ties, worst = [], [], 0.0
    for t in trace:
        ref, kv = oracle_logits(W, cfg, x[:t["window_end"]], mask_kind="d2f_hybrid",
                                mask_geometry=(0, BLOCK), output_rows=t["frontier"],
                                last_layer_output_rows_only=True)
        rep, bad = compare_proposals(t["scores"], t["tokens"], ref, kv_logits=kv,
                                     quota=len(t["chosen"]), gpu_chosen=t["chosen"])
        worst = max(worst, rep["score_rel_max"])
        ties += rep["report"]
        problems += [(t["step"],) + tuple(b) for b in bad]
        for r in t["chosen"]:
            x[t["frontier"][r]] = t["tokens"][r]
    return problems, ties, worst


@pytest.mark.parametrize("separate", [False, True], ids=["merged", "separate"])
def test_bd3_commit_with_next_step(separate, monkeypatch):
    from diffusorrt_amd import synthetic as syn

    geom = _geometry()
    model = syn.build_model(geom, "q4", seed=31)
    prompt = np.random.default_rng(31).integers(0, 3900, PROMPT).tolist()
    _say(f"BD3 layer shapes, {PROMPT}-token prompt, 3 blocks, commit "
         f"{'separate' if separate else 'merged into the next step'}")
    res, trace, m = _decode(model, prompt, monkeypatch, separate)
    assert res.committed_token_count == GEN and res.forward_count == STEPS
    # the prompt, then the two finished blocks before the last
    assert m["rocm_commit_rows"] == PROMPT + 2 * BLOCK
    assert m["rocm_active_rows"] == STEPS * BLOCK
    problems, ties, worst = _teacher_forced(model, prompt, trace)
    _say(f"  score rel max {worst:.2e}; reported: {ties}")
    assert not problems, problems
    if not separate:
        native, _, _ = _decode(model, prompt, monkeypatch, separate, native=True)
        assert native.full_token_ids == res.full_token_ids
