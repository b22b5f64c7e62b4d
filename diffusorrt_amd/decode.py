"""Host control plane of the denoise loop for the strategies the device session
runs: the two fixed-quota policies and Dream's block threshold.

Behaviour follows the reference's ``backends/diffusion_runtime.py`` (the masked
canvas :387-558, block threshold :1023-1098, block grid :1099-1141, fixed
quota :1145-1196, BD3 fixed quota :1200-1346, the decode loop :1829-1991);
the two fixed-quota policies are one precomputed schedule here
(``QuotaSchedule``), the shape the library's native loop also takes;
``backends/decode_session.py`` (``DecodeRequest.prepare`` :113-210) and
``backends/device_runtime.py`` (``_run_device_state`` :108-183,
``generate_device_tokens`` :186-274), limited to what the device route needs:
the device session scores each frontier row and the shared commit policy here
picks the rows (``argsort(-score)[:quota]``, or every row at or above the
confidence threshold) and commits them.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable

import numpy as np


class GenerationCancelled(RuntimeError):
    """Raised at a step boundary when the caller's cancellation check fires."""


# --------------------------------------------------------------------------- state


@dataclass
class MaskState:
    """The masked canvas: prompt + generated region (``diffusion_runtime.py:387-558``)."""

    x: list
    prompt_len: int
    mask_token_id: int
    eos_token_id: int

    def masked_positions(self) -> list:
        return [p for p in range(self.prompt_len, len(self.x)) if self.x[p] == self.mask_token_id]

    def all_fillable_positions(self) -> list:
        return list(range(self.prompt_len, len(self.x)))

    def commit(self, *, position: int, token_id: int) -> None:
        self.x[position] = token_id

    def finalize(self) -> dict:
        gen = self.x[self.prompt_len:]
        if self.eos_token_id in gen:
            first = gen.index(self.eos_token_id)
            answer, hit_eos, reason = gen[:first], True, "stop"
        else:
            answer, hit_eos, reason = gen, False, "length"
        remaining = answer.count(self.mask_token_id)
        if remaining:
            reason = "length"
            visible = answer[:answer.index(self.mask_token_id)]
        else:
            visible = answer
        return {"visible_token_ids": list(visible), "hit_eos": hit_eos,
                "remaining_mask_count": remaining, "finish_reason": reason}


@dataclass
class StepPlan:
    frontier: list
    window_end: int | None = None
    skip: bool = False
    stop: bool = False


def topk_count_choices(scores, transfer_count: int) -> list:
    """Top ``transfer_count`` rows by descending score: ``argsort(-score)[:k]``
    (``diffusion_runtime.py:290-299``).

    Rows with exactly equal scores go lowest index first (a stable sort). The
    reference's default-quicksort ``np.argsort`` leaves their order to the sort
    implementation (an introsort, handed to SIMD sorts by numpy 2.x where the
    CPU has them), so no single order matches it everywhere; this one is what
    the native loop and the device-side choice use too, so every loop of this
    build commits the same rows."""
    chosen = np.argsort(-np.asarray(scores, dtype=np.float64), kind="stable")[:transfer_count]
    return [int(i) for i in chosen]


def threshold_choices(scores, threshold: float) -> list:
    """Rows at or above ``threshold``; the single most confident row when none
    clears it (``diffusion_runtime.py:302-314``)."""
    conf = np.asarray(scores, dtype=np.float64)
    chosen = np.flatnonzero(conf >= float(threshold))
    if chosen.size == 0:
        return [int(np.argmax(conf))]
    return [int(i) for i in chosen]


# --------------------------------------------------------------------------- policies


@dataclass
class BlockThresholdCommit:
    """Block-sequential threshold commit (``diffusion_runtime.py:1023-1098``): the
    frontier is the current left-to-right block of ``block_size`` fillable
    positions still masked; the pointer moves past fully committed blocks; STOP
    when none remain. ``select`` commits every row at or above the threshold
    (floor of one). The step budget is the request's ``steps``
    (``:1854-1857``)."""

    confidence_threshold: float
    block_size: int
    requested_steps: int
    name: str = field(default="block_threshold", init=False)
    _block_index: int = field(default=0, init=False)

    def __post_init__(self):
        if self.block_size <= 0 or self.requested_steps <= 0:
            raise ValueError("block_threshold requires positive block_size and steps")
        if not 0.0 <= float(self.confidence_threshold) <= 1.0:
            raise ValueError("confidence_threshold must lie in [0, 1]")

    @property
    def iteration_limit(self) -> int:
        return self.requested_steps

    def plan(self, *, state: MaskState, step: int) -> StepPlan:
        fillable = state.all_fillable_positions()
        while self._block_index < len(fillable):
            block = fillable[self._block_index:self._block_index + self.block_size]
            masked = [p for p in block if state.x[p] == state.mask_token_id]
            if masked:
                return StepPlan(frontier=masked)
            self._block_index += self.block_size
        return StepPlan(frontier=[], stop=True)

    def select(self, *, scores, step: int) -> list:
        return threshold_choices(scores, self.confidence_threshold)



def block_spans(start: int, length: int, block_size: int, origin: int = 0) -> list:
    """Cut the interval ``[start, start + length)`` at the multiples of
    ``block_size`` counted from ``origin``; returns the ``(lo, hi)`` pieces in
    order. ``origin = 0`` gives BD3's absolute blocks, ``origin = start`` the
    prompt-relative blocks of the full-canvas policy (the block geometry of
    ``backends/diffusion_runtime.py:1099-1141``)."""
    for label, v, least in (("start", start, 0), ("length", length, 0), ("origin", origin, 0),
                            ("block_size", block_size, 1)):
        if isinstance(v, bool) or not isinstance(v, int) or v < least:
            raise ValueError(f"block grid: {label} must be an int >= {least}, got {v!r}")
    if origin > start:
        raise ValueError(f"block grid: origin {origin} lies after the interval start {start}")
    spans, lo, end = [], start, start + length
    while lo < end:
        hi = min(end, origin + ((lo - origin) // block_size + 1) * block_size)
        spans.append((lo, hi))
        lo = hi
    return spans


def round_quotas(masked: int, rounds: int) -> list:
    """Rows committed by each of a block's ``rounds`` rounds: ``masked`` spread
    evenly, the remainder going to the earliest rounds (the divmod rule of
    ``diffusion_runtime.py:1145-1196, 1320-1330``)."""
    base, extra = divmod(masked, rounds)
    return [base + 1] * extra + [base] * (rounds - extra)


class QuotaSchedule:
    """The two fixed-quota policies as one precomputed schedule.

    The generated region is cut into block spans (``block_spans``); every span
    gets ``rounds`` steps, ``rounds = ceil(steps / ceil(generated / block))``,
    so the step budget is ``len(spans) * rounds``. When step ``k`` enters span
    ``k // rounds`` the span's masked rows fix that span's per-round quotas
    (``round_quotas``); step ``k`` proposes the span's still-masked rows and
    commits the ``quota[k % rounds]`` most confident ones (``argsort(-score)``);
    a step with no masked row or a zero quota is skipped.

    ``absolute=True`` is BD3 (``diffusion_runtime.py:1200-1346,
    2223-2264``): blocks on the absolute grid, the proposal's window ends at the
    span's end, an end token ends the decode at a block boundary, and so does a
    canvas with no mask left. ``absolute=False`` is the full-canvas policy
    (``:1145-1196, 2199-2219``): prompt-relative blocks, no window, no early
    stop."""

    def __init__(self, *, prompt_len: int, generated: int, block_size: int, steps: int,
                 absolute: bool, requires_prompt_block_alignment: bool = True):
        for label, v, least in (("block_size", block_size, 1), ("steps", steps, 1),
                                ("generated", generated, 0), ("prompt_len", prompt_len, 0)):
            if isinstance(v, bool) or not isinstance(v, int) or v < least:
                raise ValueError(f"fixed-quota schedule: {label} must be an int >= {least}")
        self.prompt_len = prompt_len
        self.generated = generated
        self.block_size = block_size
        self.absolute = absolute
        self.aligned = requires_prompt_block_alignment
        self.spans = block_spans(prompt_len, generated, block_size,
                                 0 if absolute else prompt_len)
        sched_blocks = -(-generated // block_size)
        self.rounds = -(-steps // sched_blocks) if self.spans else 0
        self.name = "bd3_fixed_quota" if absolute else "fixed_quota"
        self._span = -1       # span whose quotas are in _quotas
        self._quotas: list = []
        self._quota = 0       # quota of the step last planned

    @property
    def iteration_limit(self) -> int:
        return len(self.spans) * self.rounds

    def plan(self, *, state: MaskState, step: int) -> StepPlan:
        if self.absolute and (state.prompt_len, len(state.x) - state.prompt_len) != (
                self.prompt_len, self.generated):
            raise ValueError("the canvas no longer matches the schedule's generated region")
        if step >= self.iteration_limit:
            return StepPlan(frontier=[], stop=True)
        if self.absolute and self.aligned and self.prompt_len % self.block_size:
            raise ValueError(f"prompt of {self.prompt_len} tokens is not aligned to "
                             f"{self.block_size}-token blocks")
        span, rnd = divmod(step, self.rounds)
        if self.absolute:
            region = state.x[self.prompt_len:]
            if (rnd == 0 and state.eos_token_id in region) or state.mask_token_id not in region:
                return StepPlan(frontier=[], stop=True)
        lo, hi = self.spans[span]
        frontier = [p for p in range(lo, hi) if state.x[p] == state.mask_token_id]
        if span != self._span:
            self._span, self._quotas = span, round_quotas(len(frontier), self.rounds)
        self._quota = self._quotas[rnd]
        if not frontier or self._quota == 0:
            return StepPlan(frontier=[], skip=True)
        return StepPlan(frontier=frontier, window_end=hi if self.absolute else None)

    def select(self, *, scores, step: int) -> list:
        return topk_count_choices(scores, self._quota)


# --------------------------------------------------------------------------- loop


@dataclass
class DecodeResult:
    """Mirrors ``DiffusionIterationResult`` (``diffusion_runtime.py:566-600``)."""

    visible_generated_token_ids: list
    iteration_count: int
    forward_count: int
    committed_token_count: int
    hit_eos: bool
    remaining_mask_count: int
    finish_reason: str
    decode_loop_kind: str
    entropy_used: bool = False
    committed_per_forward: float = 0.0
    full_token_ids: list = field(default_factory=list)


def run_decode_loop(state: MaskState, *, commit_policy, iteration_limit: int, propose_fn,
                    commit_device_fn, cancelled: Callable[[], bool] | None = None,
                    trace: list | None = None) -> tuple:
    """forward -> score -> select -> commit, propose branch (``:1829-1991``).

    ``propose_fn(plan) -> (scores, token_ids, forwarded_rows)`` runs on the device;
    the commit policy selects rows on the host; ``commit_device_fn(positions,
    tokens)`` updates the device canvas before the host mirror."""
    if type(iteration_limit) is not int or iteration_limit < 0:
        raise ValueError("iteration_limit must be a nonnegative integer")
    forwards = committed = iterations = 0
    for step in range(iteration_limit):
        if cancelled is not None and cancelled():
            raise GenerationCancelled("generation cancelled")
        plan = commit_policy.plan(state=state, step=step)
        if plan.stop:
            break
        if plan.skip:
            continue
        frontier = list(plan.frontier)
        scores, token_ids, forwarded = propose_fn(plan)
        if len(scores) != len(frontier) or len(token_ids) != len(frontier):
            raise ValueError("device proposal does not match the policy frontier")
        forwards += 1
        chosen = commit_policy.select(scores=scores, step=step)
        if trace is not None:
            trace.append({"step": step, "frontier": frontier, "window_end": plan.window_end,
                          "scores": [float(s) for s in scores], "tokens": list(token_ids),
                          "chosen": list(chosen), "forwarded_rows": int(forwarded)})
        if chosen:
            commit_device_fn([frontier[r] for r in chosen], [int(token_ids[r]) for r in chosen])
        for r in chosen:
            state.commit(position=frontier[r], token_id=int(token_ids[r]))
        committed += len(chosen)
        iterations += 1
    return forwards, committed, iterations


_DEVICE_STRATEGIES = ("bd3_fixed_quota", "fixed_quota", "block_threshold")


def _count(name: str, value, least: int) -> None:
    if type(value) is not int or value < least:  # bools are refused too
        raise ValueError(f"{name} must be an integer >= {least}")


def _check_request(strategy: str, *, max_tokens, steps, block_size, memory_budget_bytes,
                   temperature, prompt, mask_token_id) -> None:
    """The device route's request rules (``backends/device_runtime.py:80-92,
    186-247``), checked before the session is touched."""
    if strategy not in _DEVICE_STRATEGIES:
        raise ValueError(f"decode strategy {strategy!r} has no rocm device session "
                         f"(available: {', '.join(_DEVICE_STRATEGIES)})")
    _count("max_tokens", max_tokens, 0)
    _count("steps", steps, 1)
    _count("block_size", block_size, 1)
    _count("memory_budget_bytes", memory_budget_bytes, 0)
    if not (math.isfinite(temperature) and temperature >= 0):
        raise ValueError("temperature must be a finite number >= 0")
    if strategy == "block_threshold" and temperature != 0:
        raise ValueError("block_threshold scores greedily: temperature must be 0")
    if len(prompt) == 0:
        raise ValueError("a device decode needs at least one prompt token")
    if strategy == "bd3_fixed_quota" and mask_token_id in prompt:
        raise ValueError("a bd3_fixed_quota prompt on the device may not contain the mask token")


def generate_device_tokens(session, prompt_token_ids: list, *, max_tokens: int,
                           mask_token_id: int, eos_token_id: int, steps: int, block_size: int,
                           decode_strategy: str = "bd3_fixed_quota",
                           requires_prompt_block_alignment: bool = True,
                           temperature: float = 0.0, seed: int = 0,
                           memory_budget_bytes: int = 0, confidence_threshold: float = 0.9,
                           native: bool = True,
                           cancelled: Callable[[], bool] | None = None,
                           trace: list | None = None) -> DecodeResult:
    """Run a policy with scoring on the device (``backends/device_runtime.py:108-274``).
    ``block_threshold`` scores without the MASK column (the session leaves it out
    of the softmax and argmax) and decodes greedily over the exact K/V of the
    prompt and the frozen blocks. With ``native`` (and no trace or cancellation
    hook) ``bd3_fixed_quota`` runs the same loop inside the library
    (``drt_session_bd3_decode``)."""
    _check_request(decode_strategy, max_tokens=max_tokens, steps=steps, block_size=block_size,
                   memory_budget_bytes=memory_budget_bytes, temperature=temperature,
                   prompt=prompt_token_ids, mask_token_id=mask_token_id)
    prompt_len = len(prompt_token_ids)
    state = MaskState(x=[*prompt_token_ids, *([mask_token_id] * max_tokens)],
                      prompt_len=prompt_len, mask_token_id=mask_token_id,
                      eos_token_id=eos_token_id)
    exact_kv = False
    if decode_strategy == "block_threshold":
        # D2F over the exact prompt + frozen-block K/V: blocks count from the
        # prompt, each proposal forwards the active block (and the Dream shift's
        # feeder row) over the cached prefix (backends/device_runtime.py:108-183)
        policy = BlockThresholdCommit(confidence_threshold=confidence_threshold,
                                      block_size=block_size, requested_steps=steps)
        origin = prompt_len
        exact_kv = True
        loop_kind = "rocm_dream_block_threshold"
    else:
        bd3 = decode_strategy == "bd3_fixed_quota"
        policy = QuotaSchedule(prompt_len=prompt_len, generated=max_tokens,
                               block_size=block_size, steps=steps, absolute=bd3,
                               requires_prompt_block_alignment=requires_prompt_block_alignment)
        origin = 0 if bd3 else prompt_len
        loop_kind = "rocm_qwen3_bd3_fixed_quota" if bd3 else "rocm_bidirectional_fixed_quota"
    session.start_device(state.x, prompt_len=origin, block_size=block_size,
                         mask_token_id=mask_token_id, exact_kv=exact_kv, steps=steps,
                         memory_budget_bytes=memory_budget_bytes,
                         temperature=float(temperature), seed=int(seed))

    def propose(plan):
        # rows before the active block's grid start are frozen (served from the
        # cache on a d2f session); the full canvas freezes only its prompt
        if decode_strategy == "fixed_quota":
            return session.propose_device(plan.frontier, window_end=len(state.x),
                                          frozen_prefix=state.prompt_len)
        frozen = origin + (min(plan.frontier) - origin) // block_size * block_size
        window_end = plan.window_end or min(len(state.x), frozen + block_size)
        return session.propose_device(plan.frontier, window_end=window_end,
                                      frozen_prefix=frozen)

    if (native and decode_strategy == "bd3_fixed_quota" and trace is None and cancelled is None
            and hasattr(session, "bd3_decode")):
        # the same loop run inside the library: no return to Python between steps
        forwards, committed, _done = session.bd3_decode(
            prompt_len=prompt_len, max_tokens=max_tokens, steps=steps, eos_token_id=eos_token_id,
            requires_prompt_block_alignment=requires_prompt_block_alignment,
            max_forwards=policy.iteration_limit)
        iterations = forwards
        state.x = session.canvas()
    else:
        forwards, committed, iterations = run_decode_loop(
            state, commit_policy=policy, iteration_limit=policy.iteration_limit,
            propose_fn=propose, commit_device_fn=session.commit_device, cancelled=cancelled,
            trace=trace)
    fin = state.finalize()
    return DecodeResult(
        visible_generated_token_ids=fin["visible_token_ids"], iteration_count=iterations,
        forward_count=forwards, committed_token_count=committed, hit_eos=fin["hit_eos"],
        remaining_mask_count=fin["remaining_mask_count"], finish_reason=fin["finish_reason"],
        decode_loop_kind=loop_kind,
        committed_per_forward=(committed / forwards) if forwards else 0.0,
        full_token_ids=list(state.x))
