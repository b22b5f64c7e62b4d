"""The request surface on the CPU: decode-plan admission, steps floor, seed
policy, the chunked reply loop, over a fake device session."""
from __future__ import annotations

import threading

import pytest

from diffusorrt_amd import engine as E
from diffusorrt_amd.decode import DecodeResult

from helpers import tiny_dream_geometry, tiny_geometry


class FakeSession:
    """Scores every frontier row; proposes token ``(7 * position) % 97 + 1`` except
    ``eos_at`` positions, which propose the end token."""

    def __init__(self, rt, config):
        self.rt, self.config = rt, config

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        pass

    def start_device(self, tokens, **kw):
        self.rt.starts.append((list(tokens), dict(kw), dict(self.config)))

    def propose_device(self, frontier, *, window_end, frozen_prefix):
        toks = [self.rt.eos if p in self.rt.eos_at else (7 * p) % 97 + 1 for p in frontier]
        scores = [1.0 / (1 + p) for p in frontier]
        return scores, toks, len(frontier)

    def commit_device(self, positions, tokens):
        pass


class FakeRuntime:
    def __init__(self, eos, eos_at=()):
        self.eos, self.eos_at, self.starts, self.closed = eos, set(eos_at), [], False

    def session(self, config):
        return FakeSession(self, config)

    def close(self):
        self.closed = True


class _Model:
    def __init__(self, g, kind="q4"):
        self.geometry, self.weight_kind = g, kind


def _engine(g, eos_at=(), **kw):
    rt = FakeRuntime(g.eos_token_id, eos_at)
    eng = E.RocmEngine(_Model(g), runtime_factory=lambda *a, **k: rt, **kw)
    return eng, rt


def test_backend_id_and_policies():
    assert E.RocmEngine.backend_id == "rocm"
    bd3 = E.admit_decode_plan("qwen3_bd3lm")
    assert (bd3.decode_strategy, bd3.block_size, bd3.steps, bd3.attention_mask_kind,
            bd3.requires_prompt_block_alignment) == ("bd3_fixed_quota", 32, 128, "d2f_hybrid", True)
    mdlm = E.admit_decode_plan("qwen3_mdlm")
    assert (mdlm.decode_strategy, mdlm.block_size, mdlm.steps, mdlm.whole_canvas) == \
        ("fixed_quota", 64, 256, True)
    ragged = E.admit_decode_plan("qwen3_bd3lm", policy="fixed_quota_ragged_v1")
    assert not ragged.requires_prompt_block_alignment
    bt = E.admit_decode_plan("qwen2_dream")  # Dream's own block-threshold policy
    assert (bt.decode_strategy, bt.block_size, bt.steps, bt.confidence_threshold,
            bt.attention_mask_kind, bt.whole_canvas) == ("block_threshold", 8, 512, 0.9,
                                                         "d2f_hybrid", False)
    assert E.request_steps(bt, 2000) == 512
    dream = E.admit_decode_plan("qwen2_dream", decode_strategy="fixed_quota", block_size=256,
                                steps=64)
    assert (dream.decode_strategy, dream.block_size, dream.steps) == ("fixed_quota", 256, 64)
    with pytest.raises(E.PlanNotAdmitted):
        E.admit_decode_plan("qwen3_mdlm", decode_strategy="entropy_budget")
    # the BD3 contract's package keys, when present, must agree
    good = {"mlx_diffusion_decode_strategy": "bd3_fixed_quota", "mlx_diffusion_block_size": 32,
            "bd3_requires_prompt_block_alignment": True}
    E.admit_decode_plan("qwen3_bd3lm", good)
    for key, bad in (("mlx_diffusion_block_size", 64),
                     ("mlx_diffusion_decode_strategy", "fixed_quota"),
                     ("bd3_requires_prompt_block_alignment", False)):
        with pytest.raises(ValueError, match=key):
            E.admit_decode_plan("qwen3_bd3lm", dict(good, **{key: bad}))


def test_steps_floor():
    bd3 = E.admit_decode_plan("qwen3_bd3lm")
    assert E.request_steps(bd3, 32) == 128       # the plan's steps
    assert E.request_steps(bd3, 200) == 224      # 7 blocks x 32
    assert E.request_steps(E.admit_decode_plan("qwen3_mdlm"), 300) == 320


def test_request_validation():
    for bad in (dict(max_tokens=0), dict(max_tokens=True), dict(temperature=-1.0),
                dict(temperature=float("nan")), dict(seed=-1), dict(seed=1 << 64),
                dict(seed=1.5)):
        args = dict(max_tokens=4, temperature=0.0, seed=None)
        args.update(bad)
        with pytest.raises(ValueError):
            E.validate_request(**args)


def test_bd3_generate_greedy_and_seeded():
    g = tiny_geometry()
    eng, rt = _engine(g)
    res = eng.generate_ids(list(range(64)), max_tokens=64)
    assert res.backend == "rocm" and res.seed is None and res.decodes == 1
    assert len(res.token_ids) == 64 and res.finish_reason == "length"
    assert res.steps == 128 and res.forward_count == 64  # 2 blocks x 32 quota-1 steps... floor
    tokens, kw, cfg = rt.starts[0]
    assert kw["temperature"] == 0.0 and kw["seed"] == 0 and kw["steps"] == 128
    assert cfg["block_size"] == 32 and cfg["max_tokens"] == 128
    # a sampled request without a seed draws one and reports it
    res2 = eng.generate_ids(list(range(64)), max_tokens=32, temperature=0.7)
    assert isinstance(res2.seed, int) and 0 <= res2.seed < 1 << 32
    assert rt.starts[-1][1]["seed"] == res2.seed and rt.starts[-1][1]["temperature"] == 0.7
    res3 = eng.generate_ids(list(range(64)), max_tokens=32, temperature=0.7, seed=5)
    assert res3.seed == 5
    # BD3 requires block-aligned prompts
    with pytest.raises(ValueError):
        eng.generate_ids(list(range(63)), max_tokens=32)


def test_block_causal_without_limit_decodes_once():
    g = tiny_geometry(max_position_embeddings=4096)
    eng, rt = _engine(g, eos_at={64 + 40})
    res = eng.generate_ids(list(range(64)), max_tokens=None)
    assert res.decodes == 1 and res.budget == E.AUTO_REPLY_LIMIT_TOKENS
    assert res.hit_eos and res.finish_reason == "stop"
    # the reply ends before the end token (MaskState.finalize truncates there)
    assert len(res.token_ids) == 40 and g.eos_token_id not in res.token_ids


def test_whole_canvas_without_limit_decodes_in_chunks():
    g = tiny_dream_geometry(max_position_embeddings=64 + 300)
    eng, rt = _engine(g, plan_overrides={"decode_strategy": "fixed_quota", "block_size": 256,
                                         "steps": 64})
    with pytest.raises(ValueError):  # block_threshold (Dream's default) is greedy
        _engine(g)[0].generate_ids(list(range(64)), max_tokens=8, temperature=0.5)
    res = eng.generate_ids(list(range(64)), max_tokens=None)
    # limit = 364 - 64 = 300: chunks of 128, 128, 44, each joining the next prompt
    assert res.decodes == 3 and [len(c.visible_generated_token_ids) for c in res.chunks] == \
        [128, 128, 44]
    assert len(res.token_ids) == 300 and res.budget == 44
    assert [len(t) for t, _, _ in rt.starts] == [64 + 128, 64 + 128 + 128, 64 + 256 + 44]
    assert rt.starts[1][0][:64 + 128] == list(range(64)) + res.token_ids[:128]
    # an end token inside a chunk ends the reply
    eng2, _ = _engine(g, eos_at={64 + 128 + 10},
                      plan_overrides={"decode_strategy": "fixed_quota", "block_size": 256,
                                      "steps": 64})
    res2 = eng2.generate_ids(list(range(64)), max_tokens=None)
    assert res2.decodes == 2 and res2.hit_eos


def test_sequence_limit_and_serialized_callers():
    g = tiny_geometry(max_position_embeddings=128)
    eng, rt = _engine(g)
    with pytest.raises(ValueError, match="sequence limit"):
        eng.generate_ids(list(range(64)), max_tokens=96)
    out = []

    def worker():
        out.append(eng.generate_ids(list(range(32)), max_tokens=32).token_ids)

    threads = [threading.Thread(target=worker) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(out) == 4 and all(o == out[0] for o in out)
    eng.close()
    assert rt.closed


def test_decode_until_end_with_limit_is_one_decode():
    calls = []

    def once(prompt, budget):
        calls.append((len(prompt), budget))
        return DecodeResult(visible_generated_token_ids=[1] * budget, iteration_count=1,
                            forward_count=1, committed_token_count=budget, hit_eos=False,
                            remaining_mask_count=0, finish_reason="length",
                            decode_loop_kind="x")

    chunks, budget = E.decode_until_end(once, [0] * 10, max_tokens=500, sequence_limit=4096,
                                        whole_canvas=True)
    assert len(chunks) == 1 and budget == 500 and calls == [(10, 500)]
