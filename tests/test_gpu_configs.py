"""GPU parity at the defining sizes of the two long workloads.

* BD3 (Qwen3-0.6B layer shapes) over an 8192-token committed prefix: the prefix
  is committed in four 2048-row chunks (large-M kernels and the masked
  long-query attention), then a 32-token block is denoised in 8 steps (the
  graph-replayed decode step, its attention ranges derived from the cache's
  8K capacity), teacher-forced against the oracle; the library's native loop
  must reproduce the host loop's canvas.
* Dream (Qwen2.5-7B layer shapes), the full 512-row canvas of 256 prompt + 256
  masked tokens: window logits of every masked row, then two fixed-quota steps
  (4 rows each) teacher-forced against the oracle.

* Dream's <= 32-row forwards at the 7B layer shapes (its block-threshold decode
  runs them): a 32-row window through the split-K linears at those shapes.

One decoder layer and a 4096-token vocabulary keep the oracle to seconds; every
kernel runs at its real shape. The bar is the one of every session test: strict
(1e-3 tie band, scores within SCORE_REL_TOL) against the oracle with the cached
K/V rounded to fp16, disagreements with the exact oracle reported and
attributed to that storage.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from oracle import forward as F

from helpers import (LOGITS_REL_TOL, compare_proposals, kv_round_f16, oracle_logits,
                     oracle_weights, rel_err_rows)

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _geometry(base):
    return dataclasses.replace(base, layer_count=1, vocab_size=4096, mask_token_id=4000,
                               eos_token_id=4001)


def test_bd3_8k_prefix_chunked_commit_and_block_steps():
    from diffusorrt_amd import decode
    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.runtime import Runtime, bd3_session_config

    PREFIX, GEN, STEPS = 8192, 32, 8
    _say("bd3 8K prefix: 4 x 2048-row commit + 8 steps, real layer shapes")
    geom = _geometry(syn.BD3_QWEN3_06B)
    model = syn.build_model(geom, "q4", seed=4)
    W, cfg = oracle_weights(model), syn.oracle_config(geom, "q4")
    prompt = np.random.default_rng(4).integers(0, 3900, PREFIX).tolist()
    rt = Runtime(model, max_forward_rows=2048, max_positions=PREFIX + GEN + 64)
    try:
        trace = []
        with rt.session(bd3_session_config(32, STEPS, PREFIX + GEN)) as s:
            host = decode.generate_device_tokens(
                s, prompt, max_tokens=GEN, mask_token_id=geom.mask_token_id,
                eos_token_id=geom.eos_token_id, steps=STEPS, block_size=32, trace=trace)
            m = s.device_metrics()
        assert host.forward_count == STEPS and host.committed_token_count == GEN
        # the prefix went through the chunked commit: 8192 rows in 2048-row forwards
        assert m["rocm_commit_rows"] == PREFIX and m["rocm_kv_cache_len"] == PREFIX
        assert all(t["forwarded_rows"] in (32, PREFIX + 32) for t in trace)
        x = prompt + [geom.mask_token_id] * GEN
        problems, ties, worst = [], [], 0.0
        for t in trace:
            ref, kv = oracle_logits(W, cfg, x[:t["window_end"]], mask_kind="d2f_hybrid",
                                    mask_geometry=(0, 32), output_rows=t["frontier"],
                                    last_layer_output_rows_only=True)
            rep, bad = compare_proposals(t["scores"], t["tokens"], ref, kv_logits=kv,
                                         quota=len(t["chosen"]), gpu_chosen=t["chosen"])
            worst = max(worst, rep["score_rel_max"])
            ties += rep["report"]
            problems += [(t["step"],) + tuple(b) for b in bad]
            for r in t["chosen"]:
                x[t["frontier"][r]] = t["tokens"][r]
        _say(f"  score rel max {worst:.2e}; reported: {ties}")
        assert not problems, problems
        with rt.session(bd3_session_config(32, STEPS, PREFIX + GEN)) as s:
            native = decode.generate_device_tokens(
                s, prompt, max_tokens=GEN, mask_token_id=geom.mask_token_id,
                eos_token_id=geom.eos_token_id, steps=STEPS, block_size=32, native=True)
        assert native.full_token_ids == host.full_token_ids
        assert native.forward_count == host.forward_count
    finally:
        rt.close()


def test_dream_512_row_canvas_window_and_fixed_quota_steps():
    from diffusorrt_amd import decode
    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.runtime import Runtime, fixed_quota_session_config

    P_LEN, GEN = 256, 256
    _say("dream 512-row canvas: window + 2 fixed-quota steps, real layer shapes")
    geom = _geometry(syn.DREAM_QWEN25_7B)
    model = syn.build_model(geom, "q4", seed=3)
    W, cfg = oracle_weights(model), syn.oracle_config(geom, "q4")
    prompt = np.random.default_rng(3).integers(0, 3900, P_LEN).tolist()
    x = prompt + [geom.mask_token_id] * GEN
    scope = list(range(P_LEN, P_LEN + GEN))
    rt = Runtime(model, max_forward_rows=512, max_positions=1024)

    def oracle(canvas, frontier):
        return [F.window_logits(W, cfg, canvas, frontier, mask_kind="bidirectional",
                                mask_geometry=None, logits_convention="dream_ar_shift",
                                kv_round=kr, last_layer_output_rows_only=True)
                for kr in (None, kv_round_f16)]

    try:
        with rt.session(fixed_quota_session_config(256, 64, len(x))) as s:
            win = s.execute_window(x, scope)
        assert win.forwarded_rows == len(x)
        ref, kv = oracle(x, scope)
        err, err_kv = rel_err_rows(win.array(), ref), rel_err_rows(win.array(), kv)
        _say(f"  window rel err max={err.max():.2e} (vs fp16-K/V oracle {err_kv.max():.2e})")
        assert err.max() < LOGITS_REL_TOL
        # the canvas's 256 frontier rows, scored on the device, then the policy's
        # first two rounds (quota 4 each) committed through the session
        state = decode.MaskState(x=list(x), prompt_len=P_LEN, mask_token_id=geom.mask_token_id,
                                 eos_token_id=geom.eos_token_id)
        policy = decode.QuotaSchedule(prompt_len=P_LEN, generated=GEN, block_size=256, steps=64,
                                      absolute=False)
        trace = []
        with rt.session(fixed_quota_session_config(256, 64, len(x))) as s:
            s.start_device(state.x, prompt_len=P_LEN, block_size=256,
                           mask_token_id=geom.mask_token_id, exact_kv=False, steps=64)
            decode.run_decode_loop(
                state, commit_policy=policy, iteration_limit=2,
                propose_fn=lambda plan: s.propose_device(plan.frontier, window_end=len(x),
                                                         frozen_prefix=P_LEN),
                commit_device_fn=s.commit_device, trace=trace)
        assert [len(t["chosen"]) for t in trace] == [4, 4]
        xx = list(x)
        problems, ties, worst = [], [], 0.0
        for t in trace:
            ref, kv = oracle(xx, t["frontier"])
            rep, bad = compare_proposals(t["scores"], t["tokens"], ref, kv_logits=kv,
                                         quota=len(t["chosen"]), gpu_chosen=t["chosen"])
            worst = max(worst, rep["score_rel_max"])
            ties += rep["report"]
            problems += [(t["step"],) + tuple(b) for b in bad]
            for r in t["chosen"]:
                xx[t["frontier"][r]] = t["tokens"][r]
        _say(f"  steps score rel max {worst:.2e}; reported: {ties}")
        assert not problems, problems
        assert state.x == xx
    finally:
        rt.close()


@pytest.mark.parametrize("rows", [32, 48])
def test_dream_7b_shapes_window(rows):
    """A one-layer Dream window at the 7B layer shapes. 32 rows run the
    weight-streaming linears; 48 rows (two 32-row tiles) run the split-K linears
    with the pre-scaled norm inputs at K = 3584 (eight 64-k units per q|k|v
    work-group)."""
    from diffusorrt_amd import synthetic as syn
    from diffusorrt_amd.runtime import Runtime, fixed_quota_session_config

    _say(f"dream 7B shapes, {rows}-row window")
    geom = _geometry(syn.DREAM_QWEN25_7B)
    model = syn.build_model(geom, "q4", seed=5)
    W, cfg = oracle_weights(model), syn.oracle_config(geom, "q4")
    x = np.random.default_rng(5).integers(0, 3900, rows - 8).tolist() + [geom.mask_token_id] * 8
    scope = list(range(rows - 8, rows))
    rt = Runtime(model, max_forward_rows=64, max_positions=256)
    try:
        with rt.session(fixed_quota_session_config(8, 8, len(x))) as s:
            win = s.execute_window(x, scope)
        assert win.forwarded_rows == len(x)
        ref, kv = [F.window_logits(W, cfg, x, scope, mask_kind="bidirectional",
                                   mask_geometry=None, logits_convention="dream_ar_shift",
                                   kv_round=kr) for kr in (None, kv_round_f16)]
        got = win.array()
        err, err_kv = rel_err_rows(got, ref), rel_err_rows(got, kv)
        _say(f"  window rel err max={err.max():.2e} (vs fp16-K/V oracle {err_kv.max():.2e})")
        assert err.max() < LOGITS_REL_TOL
        assert err_kv.max() < 2e-3  # every operand but the K/V cache carries ~22 bits
    finally:
        rt.close()
