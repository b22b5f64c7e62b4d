"""The ``rocm`` backend's request surface: backend id, decode-plan admission, a
``RuntimeHandle.generate``-like call over token ids, the chunked reply loop and
request validation.

Reference (``python/src/edllm/``):
  * ``backend_ids.py:14-20`` -- the closed backend-id set; ``rocm`` is this
    package's id (``BACKEND_ID``);
  * ``model_definitions.py:260-273, 347-375, 454-459`` -- the decode policy of
    each runtime architecture (``DECODE_POLICIES``);
  * ``model.py:1222-1300`` (``RuntimeHandle.generate``) and ``model.py:922-1087``
    (``_generate_cuda_native``): strategy admission, greedy requests carry no
    seed, a sampled request without one draws 32 random bits;
  * ``model.py:2180-2250`` (``_decode_until_end``): with no ``max_tokens`` a
    block-causal model decodes once with the automatic budget, a whole-canvas
    model in chunks of 128 positions, each chunk's output joining the prompt of
    the next, until an end token, a hole, 1024 tokens or the sequence limit;
  * ``model.py:2252-2266`` (``_fixed_quota_request_steps``): never fewer steps
    than one per token of each block;
  * ``engine.py:143-157`` -- one request at a time per engine.

Token ids in, token ids out: tokenization and chat templates stay with the
caller.
"""
from __future__ import annotations

import math
import secrets
import threading
import time
from dataclasses import dataclass, field
from typing import Callable

from . import BACKEND_ID
from .abi import AttentionMaskKind, CommitPolicy, DecodeStrategy
from .decode import DecodeResult, generate_device_tokens

AUTO_REPLY_CHUNK_TOKENS = 128
AUTO_REPLY_LIMIT_TOKENS = 1024


@dataclass(frozen=True)
class DecodePlan:
    """The decode semantics a package runs with (``DecodeContract`` /
    ``DecodePolicy.defaults`` of ``model_definitions.py:240-345``)."""

    key: str
    decode_strategy: str
    attention_mask_kind: str
    block_size: int
    steps: int
    requires_prompt_block_alignment: bool = False
    confidence_threshold: float = 0.9

    @property
    def whole_canvas(self) -> bool:
        """Attends over its whole canvas (masked diffusion), not block-causally."""
        return self.attention_mask_kind == "bidirectional"


DECODE_POLICIES = {
    "bidirectional_fixed_quota_v1": DecodePlan("bidirectional_fixed_quota_v1", "fixed_quota",
                                               "bidirectional", 64, 256),
    "bd3_fixed_quota_v1": DecodePlan("bd3_fixed_quota_v1", "bd3_fixed_quota", "d2f_hybrid", 32,
                                     128, True),
    "fixed_quota_ragged_v1": DecodePlan("fixed_quota_ragged_v1", "bd3_fixed_quota", "d2f_hybrid",
                                        32, 128, False),
    # Dream's policy: 8-token prompt-relative blocks, threshold 0.9, over the
    # exact K/V of the prompt and the frozen blocks; the step budget is the
    # device route's default (backends/device_runtime.py:186-197)
    "block_threshold_v1": DecodePlan("block_threshold_v1", "block_threshold", "d2f_hybrid", 8,
                                     512, False, 0.9),
}
ARCHITECTURE_POLICY = {"qwen2_dream": "block_threshold_v1",
                       "qwen3_mdlm": "bidirectional_fixed_quota_v1",
                       "qwen3_bd3lm": "bd3_fixed_quota_v1"}


class PlanNotAdmitted(NotImplementedError):
    """The request's decode plan is not one this backend runs."""


def admit_decode_plan(architecture: str, model_config: dict | None = None, *,
                      policy: str | None = None, **overrides) -> DecodePlan:
    """The decode plan of a package: its architecture's policy (or ``policy``),
    with the BD3 contract's package keys checked (``model_definitions.py:303-331``)
    and explicit ``decode_strategy`` / ``block_size`` / ``steps`` /
    ``confidence_threshold`` overrides (the benchmark configurations run Dream
    with a fixed quota)."""
    key = policy or ARCHITECTURE_POLICY.get(architecture)
    if key is None:
        raise PlanNotAdmitted(f"no decode policy for architecture {architecture!r}")
    base = DECODE_POLICIES.get(key)
    if base is None:
        raise ValueError(f"unknown decode policy {key!r}")
    cfg = model_config or {}
    if base.decode_strategy == "bd3_fixed_quota" and \
            "mlx_diffusion_decode_strategy" in cfg:
        if cfg.get("mlx_diffusion_decode_strategy") != base.decode_strategy:
            raise ValueError(f"decode policy {key!r} requires "
                             f"mlx_diffusion_decode_strategy={base.decode_strategy!r}")
        if cfg.get("mlx_diffusion_block_size") != base.block_size:
            raise ValueError(f"decode policy {key!r} requires "
                             f"mlx_diffusion_block_size={base.block_size}")
        if cfg.get("bd3_requires_prompt_block_alignment") is not \
                base.requires_prompt_block_alignment:
            raise ValueError(f"decode policy {key!r} requires bd3_requires_prompt_block_alignment="
                             f"{base.requires_prompt_block_alignment!r}")
    strategy = overrides.get("decode_strategy", base.decode_strategy)
    if strategy not in ("fixed_quota", "bd3_fixed_quota", "block_threshold"):
        raise PlanNotAdmitted(f"decode_strategy {strategy!r}: the rocm backend runs "
                              "block_threshold, fixed_quota and bd3_fixed_quota")
    mask = "bidirectional" if strategy == "fixed_quota" else "d2f_hybrid"
    same = strategy == base.decode_strategy
    block = int(overrides.get("block_size", base.block_size if same else 64))
    steps = int(overrides.get("steps", base.steps if same else 256))
    align = bool(overrides.get("requires_prompt_block_alignment",
                               base.requires_prompt_block_alignment if same else False))
    tau = float(overrides.get("confidence_threshold", base.confidence_threshold))
    if block < 1 or steps < 1:
        raise ValueError("block_size and steps must be positive")
    if not 0.0 <= tau <= 1.0:
        raise ValueError("confidence_threshold must lie in [0, 1]")
    return DecodePlan(key, strategy, mask, block, steps, align, tau)


def request_steps(plan: DecodePlan, max_tokens: int) -> int:
    """``model.py:2252-2266``: at least one step per token of each block for the
    fixed-quota policies; the plan's own steps otherwise."""
    if plan.decode_strategy == "block_threshold":
        return plan.steps
    blocks = (max_tokens + plan.block_size - 1) // plan.block_size
    return max(plan.steps, blocks * plan.block_size)


def validate_request(*, max_tokens, temperature, seed) -> None:
    """``validate_generation_length`` / ``validate_request_sampling``."""
    if max_tokens is not None and (isinstance(max_tokens, bool) or not isinstance(max_tokens, int)
                                   or max_tokens < 1):
        raise ValueError("max_tokens must be a positive integer or None")
    if isinstance(temperature, bool) or not isinstance(temperature, (int, float)) or \
            not math.isfinite(temperature) or temperature < 0:
        raise ValueError("temperature must be a finite number >= 0")
    if seed is not None and (isinstance(seed, bool) or not isinstance(seed, int)
                             or not 0 <= seed < 1 << 64):
        raise ValueError("seed must be an integer in [0, 2**64) or None")


@dataclass
class GenerateResult:
    """What a request returns (the token part of the reference's ``GenerateResult``)."""

    token_ids: list
    finish_reason: str
    hit_eos: bool
    forward_count: int
    committed_token_count: int
    iteration_count: int
    remaining_mask_count: int
    decodes: int
    budget: int
    steps: int
    seed: int | None
    backend: str = BACKEND_ID
    decode_loop_kind: str = ""
    elapsed_s: float = 0.0
    chunks: list = field(default_factory=list)


def decode_until_end(decode_once: Callable[[list, int], DecodeResult], prompt_ids: list, *,
                     max_tokens: int | None, sequence_limit: int | None,
                     whole_canvas: bool) -> tuple:
    """``model.py:2186-2250``. Returns ``(results, budget of the last decode)``:
    one result, or one per chunk for a whole-canvas model without a limit."""
    if max_tokens is not None:
        return [decode_once(prompt_ids, max_tokens)], max_tokens
    limit = AUTO_REPLY_LIMIT_TOKENS
    if isinstance(sequence_limit, int) and sequence_limit > 0:
        limit = min(limit, sequence_limit - len(prompt_ids))
    limit = max(1, limit)
    if not whole_canvas:
        return [decode_once(prompt_ids, limit)], limit
    budget = min(AUTO_REPLY_CHUNK_TOKENS, limit)
    chunks = [decode_once(prompt_ids, budget)]
    written = list(chunks[-1].visible_generated_token_ids)
    while (chunks[-1].finish_reason == "length" and chunks[-1].remaining_mask_count == 0
           and len(chunks[-1].visible_generated_token_ids) == budget and len(written) < limit):
        budget = min(AUTO_REPLY_CHUNK_TOKENS, limit - len(written))
        chunks.append(decode_once(prompt_ids + written, budget))
        written.extend(chunks[-1].visible_generated_token_ids)
    return chunks, budget


class RocmEngine:
    """A runtime plus its admitted decode plan; ``generate_ids`` serves one request
    at a time (a lock, as the reference's ``Engine`` serializes callers)."""

    backend_id = BACKEND_ID

    def __init__(self, model, *, precision: str = "q4", device_ordinal: int = 0,
                 policy: str | None = None, plan_overrides: dict | None = None,
                 eos_token_id: int | None = None, mask_token_id: int | None = None,
                 runtime_factory=None, **runtime_kw):
        """``model``: a package directory or a prepared model object.
        ``precision``: ``"q4"`` (4-bit g64 linears, quantized at load for a
        package) or ``"bf16"``. ``runtime_factory(model, engine_config, device_ordinal,
        **runtime_kw)`` replaces the device runtime (host-logic tests)."""
        if precision not in ("q4", "bf16"):
            raise ValueError("precision must be 'q4' or 'bf16'")
        import os

        from .package import read_package, resolve_architecture

        if isinstance(model, (str, os.PathLike)):
            manifest, _spec, geometry = read_package(model)
            cfg = manifest.get("model_config") or {}
            arch = resolve_architecture(cfg.get("architecture"))
        else:
            geometry, cfg = model.geometry, {}
            arch = ("qwen2_dream" if geometry.logits_convention == "dream_ar_shift"
                    else "qwen3_bd3lm")
            if getattr(model, "weight_kind", precision) != precision:
                raise ValueError(f"the model's weights are {model.weight_kind}, "
                                 f"not precision={precision!r}")
        self.geometry = geometry
        self.plan = admit_decode_plan(arch, cfg, policy=policy, **(plan_overrides or {}))
        self.eos_token_id = geometry.eos_token_id if eos_token_id is None else int(eos_token_id)
        self.mask_token_id = geometry.mask_token_id if mask_token_id is None else int(mask_token_id)
        engine_config = {"linear_quant_bits": 4, "linear_quant_group_size": 64} \
            if precision == "q4" else {}
        if runtime_factory is None:
            from .runtime import Runtime

            self.runtime = Runtime(model, engine_config=engine_config,
                                   device_ordinal=device_ordinal, **runtime_kw)
        else:
            self.runtime = runtime_factory(model, engine_config, device_ordinal, **runtime_kw)
        self.sequence_limit = int(runtime_kw.get("max_positions")
                                  or geometry.max_position_embeddings)
        self._lock = threading.Lock()

    def _session_config(self, max_total: int, steps: int) -> dict:
        p = self.plan
        strategy = {"bd3_fixed_quota": DecodeStrategy.BD3_FIXED_QUOTA,
                    "fixed_quota": DecodeStrategy.FIXED_QUOTA,
                    "block_threshold": DecodeStrategy.BLOCK_THRESHOLD}[p.decode_strategy]
        commit = CommitPolicy.THRESHOLD if p.decode_strategy == "block_threshold" \
            else CommitPolicy.FIXED_QUOTA
        mask = AttentionMaskKind.D2F_HYBRID if p.attention_mask_kind == "d2f_hybrid" \
            else AttentionMaskKind.BIDIRECTIONAL
        return {"decode_strategy": int(strategy), "commit_policy": int(commit),
                "attention_mask_kind": int(mask), "block_size": p.block_size, "steps": steps,
                "max_tokens": max_total}

    def generate_ids(self, prompt_ids: list, *, max_tokens: int | None = 32,
                     temperature: float = 0.0, seed: int | None = None,
                     cancelled: Callable[[], bool] | None = None,
                     trace: list | None = None) -> GenerateResult:
        validate_request(max_tokens=max_tokens, temperature=temperature, seed=seed)
        if temperature != 0 and self.plan.decode_strategy == "block_threshold":
            raise ValueError("this model decodes with block_threshold, which is greedy; "
                             "temperature sampling belongs to the fixed-quota policies")
        prompt_ids = [int(t) for t in prompt_ids]
        if not prompt_ids:
            raise ValueError("a request needs a non-empty prompt")
        if temperature == 0:
            seed = None  # greedy: nothing to key
        elif seed is None:
            seed = secrets.randbits(32)
        started = time.perf_counter()
        steps_used = []

        def decode_once(prompt: list, budget: int) -> DecodeResult:
            if len(prompt) + budget > self.sequence_limit:
                raise ValueError(f"prompt ({len(prompt)}) + max_tokens ({budget}) exceeds the "
                                 f"sequence limit {self.sequence_limit}")
            steps = request_steps(self.plan, budget)
            steps_used.append(steps)
            with self.runtime.session(self._session_config(len(prompt) + budget, steps)) as s:
                return generate_device_tokens(
                    s, prompt, max_tokens=budget, mask_token_id=self.mask_token_id,
                    eos_token_id=self.eos_token_id, steps=steps, block_size=self.plan.block_size,
                    decode_strategy=self.plan.decode_strategy,
                    requires_prompt_block_alignment=self.plan.requires_prompt_block_alignment,
                    temperature=float(temperature), seed=0 if seed is None else int(seed),
                    confidence_threshold=self.plan.confidence_threshold,
                    cancelled=cancelled, trace=trace)

        with self._lock:
            chunks, budget = decode_until_end(decode_once, prompt_ids, max_tokens=max_tokens,
                                              sequence_limit=self.sequence_limit,
                                              whole_canvas=self.plan.whole_canvas)
        last = chunks[-1]
        tokens = [t for c in chunks for t in c.visible_generated_token_ids]
        return GenerateResult(
            token_ids=tokens, finish_reason=last.finish_reason, hit_eos=last.hit_eos,
            forward_count=sum(c.forward_count for c in chunks),
            committed_token_count=sum(c.committed_token_count for c in chunks),
            iteration_count=sum(c.iteration_count for c in chunks),
            remaining_mask_count=last.remaining_mask_count, decodes=len(chunks), budget=budget,
            steps=steps_used[-1], seed=seed, decode_loop_kind=last.decode_loop_kind,
            elapsed_s=time.perf_counter() - started, chunks=chunks)

    def close(self) -> None:
        self.runtime.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
