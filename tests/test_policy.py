"""Decode control plane (CPU only): the oracle's literal loops against closed
forms, and the product's host policies (``diffusorrt_amd.decode``) against the
oracle on random canvases."""
from __future__ import annotations

import math

import numpy as np
import pytest

from diffusorrt_amd import decode as D
from oracle import ops as O
from oracle import policy as P

MASK, EOS = 99, 98


def _bd3_plans(prompt_len, gen, steps, bs=32):
    x = [1] * prompt_len + [MASK] * gen
    state, out = {}, []
    sched = math.ceil(gen / bs)
    spb = math.ceil(steps / sched)
    for step in range(P.block_count(prompt_len, gen, bs, 0) * spb):
        kind, frontier, wend, quota = P.bd3_schedule_step(x, prompt_len, MASK, EOS, bs, steps,
                                                          step, state)
        if kind == "stop":
            break
        out.append((step, kind, frontier, wend, quota))
        if kind == "go":
            for p in frontier[:quota]:
                x[p] = 7
    return out, x


def test_bd3_schedule_config1_closed_form():
    """Prompt 64, 128 tokens, steps 32: 4 blocks x 8 rounds x 4 tokens, window = block end."""
    plans, x = _bd3_plans(64, 128, 32)
    assert len(plans) == 32
    for step, kind, frontier, wend, quota in plans:
        b = step // 8
        assert kind == "go" and quota == 4
        assert wend == 96 + 32 * b
        assert all(64 + 32 * b <= p < 96 + 32 * b for p in frontier)
        assert len(frontier) == 32 - 4 * (step % 8)
    assert MASK not in x


def test_bd3_schedule_uneven_quota_and_absolute_blocks():
    """divmod(masked, steps_per_block): remainder rounds get one more token; blocks
    are absolute (origin 0), so a prompt of 40 leaves a first block of 24."""
    plans, _ = _bd3_plans(64, 64, 5)   # 2 blocks, spb = 3: quotas 11, 11, 10
    assert [q for *_, q in plans[:3]] == [11, 11, 10]
    with pytest.raises(ValueError):
        _bd3_plans(40, 64, 4)
    assert P.block_span(40, 64, 32, 0, 0) == (40, 64)
    assert P.block_span(40, 64, 32, 0, 2) == (96, 104)
    assert P.block_count(40, 64, 32, 0) == 3


def test_bd3_eos_stops_only_at_block_boundary():
    x = [1] * 32 + [MASK] * 64
    state = {}
    k, *_ = P.bd3_schedule_step(x, 32, MASK, EOS, 32, 8, 0, state)
    assert k == "go"
    x[40] = EOS  # EOS committed inside block 0
    for step in (1, 2, 3):
        k, *_ = P.bd3_schedule_step(x, 32, MASK, EOS, 32, 8, step, state)
        assert k == "go"
    k, *_ = P.bd3_schedule_step(x, 32, MASK, EOS, 32, 8, 4, state)  # next block boundary
    assert k == "stop"


def test_fixed_quota_dream_config():
    """256 prompt + 256 masks, block >= 256, steps 64: one block, 64 rounds x 4, no window."""
    x = [1] * 256 + [MASK] * 256
    state = {}
    n = 0
    for step in range(64):
        kind, frontier, wend, quota = P.fixed_quota_schedule_step(x, 256, MASK, 256, 64, step,
                                                                  state)
        assert kind == "go" and quota == 4 and wend is None
        assert len(frontier) == 256 - 4 * step
        for p in frontier[:4]:
            x[p] = 5
        n += 4
    assert n == 256
    assert P.fixed_quota_schedule_step(x, 256, MASK, 256, 64, 64, state)[0] == "stop"


def test_finalize_cases():
    assert P.finalize([1, 2, 3, EOS, 4], 1, MASK, EOS) == {
        "visible_token_ids": [2, 3], "hit_eos": True, "remaining_mask_count": 0,
        "finish_reason": "stop"}
    assert P.finalize([1, 2, MASK, 3], 1, MASK, EOS) == {
        "visible_token_ids": [2], "hit_eos": False, "remaining_mask_count": 1,
        "finish_reason": "length"}
    assert P.finalize([1, 2, 3], 1, MASK, EOS)["finish_reason"] == "length"


def _fake_logits(vocab):
    """Deterministic frontier logits from the canvas (a stand-in model)."""
    def fn(x, frontier, _wend):
        rows = []
        for p in frontier:
            rng = np.random.default_rng(hash((tuple(x), p)) & 0xFFFFFFFF)
            rows.append(rng.standard_normal(vocab).astype(np.float32) * 3)
        return np.stack(rows)
    return fn


@pytest.mark.parametrize("strategy,prompt_len,gen,bs,steps", [
    ("bd3_fixed_quota", 32, 96, 32, 12),
    ("bd3_fixed_quota", 64, 70, 32, 7),
    ("fixed_quota", 20, 48, 16, 9),
    ("fixed_quota", 16, 40, 64, 10),
])
def test_product_loop_matches_oracle_loop(strategy, prompt_len, gen, bs, steps):
    vocab = 120
    fn = _fake_logits(vocab)
    prompt = list(np.random.default_rng(prompt_len).integers(0, 90, prompt_len))
    trace_o = []
    ref = P.run_fixed_quota_decode(prompt, max_tokens=gen, mask_id=MASK, eos_id=EOS,
                                   block_size=bs, steps=steps, strategy=strategy,
                                   frontier_logits_fn=fn, trace=trace_o)
    state = D.MaskState(x=[*prompt, *([MASK] * gen)], prompt_len=prompt_len,
                        mask_token_id=MASK, eos_token_id=EOS)
    pol = D.QuotaSchedule(prompt_len=prompt_len, generated=gen, block_size=bs, steps=steps,
                          absolute=strategy == "bd3_fixed_quota")

    def propose(plan):
        scores, toks = O.raw_max_prob(fn(list(state.x), plan.frontier, plan.window_end))
        return scores, toks, len(plan.frontier)

    trace_p = []
    fwd, committed, _ = D.run_decode_loop(state, commit_policy=pol,
                                          iteration_limit=pol.iteration_limit,
                                          propose_fn=propose, commit_device_fn=lambda p, t: None,
                                          trace=trace_p)
    assert state.x == ref["x"]
    assert fwd == ref["forward_count"] and committed == ref["committed_token_count"]
    assert [t["chosen"] for t in trace_p] == [t["chosen"] for t in trace_o]
    assert [t["window_end"] for t in trace_p] == [t["window_end"] for t in trace_o]
    assert state.finalize() == {k: ref[k] for k in
                                ("visible_token_ids", "hit_eos", "remaining_mask_count",
                                 "finish_reason")}


def test_product_bd3_eos_boundary_matches_oracle():
    """A stand-in model that emits EOS early: both loops stop at the same boundary."""
    vocab = 120

    def fn(x, frontier, _wend):
        out = np.zeros((len(frontier), vocab), np.float32)
        for r, p in enumerate(frontier):
            out[r, EOS if p == 40 else (p % 50)] = 5.0 + (p % 7) * 0.1
        return out

    ref = P.run_fixed_quota_decode([3] * 32, max_tokens=96, mask_id=MASK, eos_id=EOS,
                                   block_size=32, steps=24, strategy="bd3_fixed_quota",
                                   frontier_logits_fn=fn)
    state = D.MaskState(x=[3] * 32 + [MASK] * 96, prompt_len=32, mask_token_id=MASK,
                        eos_token_id=EOS)
    pol = D.QuotaSchedule(prompt_len=32, generated=96, block_size=32, steps=24, absolute=True)

    def propose(plan):
        s, t = O.raw_max_prob(fn(list(state.x), plan.frontier, plan.window_end))
        return s, t, 32

    D.run_decode_loop(state, commit_policy=pol, iteration_limit=pol.iteration_limit,
                      propose_fn=propose, commit_device_fn=lambda p, t: None)
    assert state.x == ref["x"]
    assert ref["hit_eos"] and MASK in ref["x"]   # stopped with later blocks still masked


def test_block_spans_match_the_oracle_grid():
    """block_spans against the oracle's block_span / block_count on absolute and
    prompt-relative grids, aligned and ragged."""
    for start, length, bs, origin in [(40, 64, 32, 0), (64, 128, 32, 0), (0, 5, 2, 0),
                                      (17, 33, 8, 17), (256, 256, 256, 256), (9, 0, 4, 0),
                                      (5, 40, 64, 0)]:
        spans = D.block_spans(start, length, bs, origin)
        assert len(spans) == P.block_count(start, length, bs, origin)
        assert spans == [P.block_span(start, length, bs, origin, i) for i in range(len(spans))]
    assert D.round_quotas(32, 8) == [4] * 8
    assert D.round_quotas(32, 3) == [11, 11, 10]
    assert D.round_quotas(2, 4) == [1, 1, 0, 0]


def test_product_policy_validation():
    with pytest.raises(ValueError):
        D.block_spans(-1, 4, 2)
    with pytest.raises(ValueError):
        D.block_spans(4, 4, 2, 5)
    with pytest.raises(ValueError):
        D.QuotaSchedule(prompt_len=0, generated=1, block_size=0, steps=1, absolute=True)
    with pytest.raises(ValueError):  # a misaligned BD3 prompt
        st = D.MaskState(x=[1] * 40 + [MASK] * 64, prompt_len=40, mask_token_id=MASK,
                         eos_token_id=EOS)
        D.QuotaSchedule(prompt_len=40, generated=64, block_size=32, steps=4,
                        absolute=True).plan(state=st, step=0)
    with pytest.raises(D.GenerationCancelled):
        state = D.MaskState(x=[1, MASK], prompt_len=1, mask_token_id=MASK, eos_token_id=EOS)
        pol = D.QuotaSchedule(prompt_len=1, generated=1, block_size=1, steps=1, absolute=False)
        D.run_decode_loop(state, commit_policy=pol, iteration_limit=1,
                          propose_fn=lambda p: ([1.0], [5], 1),
                          commit_device_fn=lambda p, t: None, cancelled=lambda: True)


def test_topk_matches_oracle_and_numpy_quicksort():
    rng = np.random.default_rng(3)
    for _ in range(50):
        s = rng.random(rng.integers(1, 40))
        k = int(rng.integers(0, len(s) + 1))
        assert D.topk_count_choices(s, k) == O.topk_count_choices(s, k)


def test_topk_exact_ties_lowest_index_first():
    """Exactly equal scores go lowest index first (the native loop and the
    device-side choice take the same order), and a tie never outranks a higher
    score; the choices always form a valid top-k of the scores."""
    assert D.topk_count_choices([0.5, 0.7, 0.5, 0.7, 0.5], 3) == [1, 3, 0]
    assert D.topk_count_choices([0.25] * 32, 4) == [0, 1, 2, 3]
    rng = np.random.default_rng(4)
    for _ in range(200):
        s = rng.integers(0, 4, int(rng.integers(1, 40))) / 4.0  # many exact ties
        k = int(rng.integers(0, len(s) + 1))
        got = D.topk_count_choices(s, k)
        ref = sorted(range(len(s)), key=lambda i: (-s[i], i))[:k]
        assert got == ref
        # the same multiset of scores as numpy's (any) quicksort order takes
        assert sorted(s[got]) == sorted(s[O.topk_count_choices(s, k)])


def test_topk_nan_scores_rank_last():
    """A NaN score ranks below every number, NaN rows among themselves in index
    order: numpy's stable argsort of -score puts NaN last, and the native loop
    (``std::isnan`` -> -inf) and the device-side choice (``block_commit_kernel``)
    rank it as -inf, which probabilities in [0, 1] never reach."""
    nan = float("nan")
    s = [0.3, nan, 0.7, nan, 0.1]
    assert D.topk_count_choices(s, 5) == [2, 0, 4, 1, 3]
    assert D.topk_count_choices(s, 2) == [2, 0]
    assert D.topk_count_choices([nan, nan, 0.0], 2) == [2, 0]
    as_neg_inf = [-math.inf if v != v else v for v in s]
    assert D.topk_count_choices(as_neg_inf, 5) == D.topk_count_choices(s, 5)


def test_threshold_choices_closed_forms():
    for pick in (D.threshold_choices, P.threshold_pick):
        assert pick([0.95, 0.5, 0.91], 0.9) == [0, 2]
        assert pick([0.9, 0.5], 0.9) == [0]            # at the threshold counts
        assert pick([0.2, 0.7, 0.7], 0.9) == [1]        # floor of one: the first maximum
        assert pick([0.3], 0.9) == [0]


def test_excluded_max_prob_drops_the_mask_column():
    logits = np.array([[0.0, 5.0, 1.0, 1.0], [2.0, 0.0, 0.0, 0.0]], dtype=np.float32)
    scores, toks = P.excluded_max_prob(logits, mask_id=1)
    # row 0: MASK (column 1) would win; without it columns 2, 3 tie -> first
    assert toks == [2, 0]
    e = np.exp(np.array([0.0, 1.0, 1.0]) - 1.0)
    assert scores[0] == pytest.approx(e.max() / e.sum(), rel=1e-12)
    # an out-of-vocabulary sentinel needs no exclusion
    s2, t2 = P.excluded_max_prob(logits, mask_id=99)
    assert t2 == [1, 0]


def test_block_threshold_walk_closed_form():
    """Blocks of 8 over 20 generated positions: [0, 8), [8, 16), [16, 20); each
    step commits the rows at or above 0.9 (here: rows whose position is odd)
    or the first most confident one; committed blocks are skipped."""
    prompt, gen, bs = [1, 2, 3], 20, 8

    def fn(x, frontier, wend):
        out = np.full((len(frontier), 120), -4.0, dtype=np.float32)
        for r, p in enumerate(frontier):
            out[r, 7] = 12.0 if p % 2 else 1.0 + 0.01 * r
        return out

    trace = []
    ref = P.run_block_threshold_decode(prompt, max_tokens=gen, mask_id=MASK, eos_id=EOS,
                                       block_size=bs, steps=100, threshold=0.9,
                                       frontier_logits_fn=fn, trace=trace)
    assert [t["window_end"] for t in trace][:2] == [11, 11]
    assert trace[0]["frontier"] == list(range(3, 11))
    assert [trace[0]["frontier"][r] for r in trace[0]["chosen"]] == [3, 5, 7, 9]
    # then the even positions one per step, highest 0.01*r bonus first (the last row)
    assert [trace[1]["frontier"][r] for r in trace[1]["chosen"]] == [10]
    assert ref["x"][3:] == [7] * gen and ref["committed_token_count"] == gen
    # per block: 1 step for the odd rows + one per even row: 1+4, 1+4, 1+2
    assert ref["forward_count"] == 5 + 5 + 3


@pytest.mark.parametrize("prompt_len,gen,bs,steps,thr", [(5, 24, 8, 60, 0.9),
                                                         (16, 33, 8, 40, 0.02),
                                                         (8, 16, 4, 6, 0.5)])
def test_product_block_threshold_matches_oracle(prompt_len, gen, bs, steps, thr):
    vocab = 120
    fn = _fake_logits(vocab)
    prompt = list(np.random.default_rng(prompt_len).integers(0, 90, prompt_len))
    trace_o = []
    ref = P.run_block_threshold_decode(prompt, max_tokens=gen, mask_id=MASK, eos_id=EOS,
                                       block_size=bs, steps=steps, threshold=thr,
                                       frontier_logits_fn=fn, trace=trace_o)
    state = D.MaskState(x=[*prompt, *([MASK] * gen)], prompt_len=prompt_len,
                        mask_token_id=MASK, eos_token_id=EOS)
    pol = D.BlockThresholdCommit(confidence_threshold=thr, block_size=bs, requested_steps=steps)

    def propose(plan):
        frozen = prompt_len + (min(plan.frontier) - prompt_len) // bs * bs
        wend = min(len(state.x), frozen + bs)
        scores, toks = P.excluded_max_prob(fn(list(state.x), plan.frontier, wend), MASK)
        return scores, toks, len(plan.frontier)

    trace_p = []
    fwd, committed, _ = D.run_decode_loop(state, commit_policy=pol,
                                          iteration_limit=pol.iteration_limit,
                                          propose_fn=propose, commit_device_fn=lambda p, t: None,
                                          trace=trace_p)
    assert state.x == ref["x"]
    assert fwd == ref["forward_count"] and committed == ref["committed_token_count"]
    assert [t["chosen"] for t in trace_p] == [t["chosen"] for t in trace_o]
    assert MASK not in [t for tr in trace_p for t in tr["tokens"]]
