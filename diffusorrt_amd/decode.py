"""Host control plane of the denoise loop for the strategies the device session
runs: the two fixed-quota policies and Dream's block threshold.

Mirrors the reference's ``backends/diffusion_runtime.py`` (``MaskState``
:387-558, ``BlockThresholdCommit`` :1023-1098, ``BlockLayout`` :1099-1141,
``FixedQuotaCommit`` :1145-1196, ``BD3FixedQuotaCommit`` :1200-1346,
``run_decode_loop`` :1829-1991),
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


@dataclass(frozen=True)
class BlockLayout:
    """A generated interval on a fixed block grid (``diffusion_runtime.py:1099-1141``).
    ``origin=0`` gives BD3's absolute blocks."""

    start: int
    length: int
    block_size: int
    origin: int = 0

    def __post_init__(self):
        for name in ("start", "length", "origin"):
            v = getattr(self, name)
            if type(v) is not int or v < 0:
                raise ValueError(f"block layout {name} must be a nonnegative integer")
        if type(self.block_size) is not int or self.block_size <= 0:
            raise ValueError("block layout block_size must be a positive integer")
        if self.origin > self.start:
            raise ValueError("block layout origin must not exceed start")

    @property
    def count(self) -> int:
        if self.length == 0:
            return 0
        first = (self.start - self.origin) // self.block_size
        last = (self.start + self.length - 1 - self.origin) // self.block_size
        return last - first + 1

    def span(self, index: int) -> tuple:
        if not 0 <= index < self.count:
            raise IndexError(f"block index {index} outside layout with {self.count} blocks")
        first = (self.start - self.origin) // self.block_size
        grid = self.origin + (first + index) * self.block_size
        return max(self.start, grid), min(self.start + self.length, grid + self.block_size)

    @property
    def mask_geometry(self) -> dict:
        return {"prompt_len": self.origin, "block_size": self.block_size}


@dataclass
class StepPlan:
    frontier: list
    window_end: int | None = None
    skip: bool = False
    stop: bool = False


def topk_count_choices(scores, transfer_count: int) -> list:
    """Top ``transfer_count`` rows by descending score: ``argsort(-score)[:k]``
    (``diffusion_runtime.py:290-299``)."""
    chosen = np.argsort(-np.asarray(scores, dtype=np.float64))[:transfer_count]
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



@dataclass
class FixedQuotaCommit:
    """Prompt-relative logical blocks, full bidirectional canvas
    (``diffusion_runtime.py:1145-1196``)."""

    block_size: int
    requested_steps: int
    generated_token_count: int
    name: str = field(default="fixed_quota", init=False)
    _active_block: int | None = field(default=None, init=False)
    _quota: int = field(default=0, init=False)
    _base: int = field(default=0, init=False)
    _remainder: int = field(default=0, init=False)

    def __post_init__(self):
        if self.block_size <= 0 or self.requested_steps <= 0:
            raise ValueError("fixed quota requires positive block_size and steps")

    @property
    def block_count(self) -> int:
        return (self.generated_token_count + self.block_size - 1) // self.block_size

    @property
    def steps_per_block(self) -> int:
        if not self.block_count:
            return 0
        return (self.requested_steps + self.block_count - 1) // self.block_count

    @property
    def iteration_limit(self) -> int:
        return self.block_count * self.steps_per_block

    def plan(self, *, state: MaskState, step: int) -> StepPlan:
        if step >= self.iteration_limit:
            return StepPlan(frontier=[], stop=True)
        block = step // self.steps_per_block
        start = block * self.block_size
        positions = state.all_fillable_positions()[start:start + self.block_size]
        frontier = [p for p in positions if state.x[p] == state.mask_token_id]
        if block != self._active_block:
            self._active_block = block
            self._base, self._remainder = divmod(len(frontier), self.steps_per_block)
        self._quota = self._base + int(step % self.steps_per_block < self._remainder)
        return StepPlan(frontier=frontier, skip=not frontier or self._quota == 0)

    def select(self, *, scores, step: int) -> list:
        return topk_count_choices(scores, self._quota)


@dataclass
class BD3FixedQuotaCommit:
    """BD3LM absolute blocks + fixed per-round transfer (``diffusion_runtime.py:1200-1346``)."""

    block_size: int
    requested_steps: int
    generated_token_count: int
    block_layout: BlockLayout
    requires_prompt_block_alignment: bool = True
    name: str = field(default="bd3_fixed_quota", init=False)
    _active_block_id: int | None = field(default=None, init=False)
    _round: int = field(default=0, init=False)
    _base: int = field(default=0, init=False)
    _remainder: int = field(default=0, init=False)

    def __post_init__(self):
        if type(self.block_size) is not int or self.block_size <= 0:
            raise ValueError("block_size must be a positive integer")
        if type(self.requested_steps) is not int or self.requested_steps <= 0:
            raise ValueError("requested_steps must be a positive integer")

    @property
    def steps_per_block(self) -> int:
        if self.block_layout.count == 0:
            return 0
        sched = (self.block_layout.length + self.block_size - 1) // self.block_size
        return (self.requested_steps + sched - 1) // sched

    @property
    def iteration_limit(self) -> int:
        return self.block_layout.count * self.steps_per_block

    def plan(self, *, state: MaskState, step: int) -> StepPlan:
        x, prompt_len = state.x, state.prompt_len
        if len(x) - prompt_len != self.generated_token_count:
            raise ValueError("BD3LM generated-token count changed during decode")
        if (self.block_layout.start, self.block_layout.length) != (prompt_len,
                                                                   self.generated_token_count):
            raise ValueError("BD3LM block layout does not cover the generated region")
        if step >= self.iteration_limit:
            return StepPlan(frontier=[], stop=True)
        if self.requires_prompt_block_alignment and prompt_len % self.block_size:
            raise ValueError("BD3LM Candidate prompt length must be a multiple of block_size")
        spb = self.steps_per_block
        generated = x[prompt_len:]
        # EOS ends the decode only at a block boundary (:1305-1309).
        if step % spb == 0 and state.eos_token_id in generated:
            return StepPlan(frontier=[], stop=True)
        mask = state.mask_token_id
        if mask not in generated:  # no masked position left
            return StepPlan(frontier=[], stop=True)
        block_id = step // spb
        # the block's span lies inside the generated region (the layout covers
        # exactly [prompt_len, len(x)), checked above), so its masked positions
        # are the masked positions of the canvas that fall in the span
        start, end = self.block_layout.span(block_id)
        frontier = [p for p in range(start, end) if x[p] == mask]
        if self._active_block_id != block_id:
            self._active_block_id = block_id
            self._base, self._remainder = divmod(len(frontier), spb)
        self._round = step % spb
        if not frontier or self._base + int(self._round < self._remainder) == 0:
            return StepPlan(frontier=[], skip=True)
        return StepPlan(frontier=frontier, window_end=end)

    def select(self, *, scores, step: int) -> list:
        return topk_count_choices(scores, self._base + int(self._round < self._remainder))


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
    if decode_strategy not in {"fixed_quota", "bd3_fixed_quota", "block_threshold"}:
        raise ValueError("the rocm device session runs block_threshold, fixed_quota and "
                         f"bd3_fixed_quota, not {decode_strategy!r}")
    if decode_strategy == "block_threshold" and temperature != 0:
        raise ValueError("block_threshold decodes greedily; temperature must be 0")
    for name, value, minimum in (("max_tokens", max_tokens, 0), ("steps", steps, 1),
                                 ("block_size", block_size, 1),
                                 ("memory_budget_bytes", memory_budget_bytes, 0)):
        if isinstance(value, bool) or not isinstance(value, int) or value < minimum:
            raise ValueError(f"{name} must be an integer >= {minimum}")
    if not math.isfinite(temperature) or temperature < 0:
        raise ValueError("temperature must be finite and >= 0")
    if not prompt_token_ids:
        raise ValueError("device generation requires a non-empty prompt")
    if decode_strategy == "bd3_fixed_quota" and mask_token_id in prompt_token_ids:
        raise ValueError("device bd3_fixed_quota cannot carry MASK in its prompt")
    prompt_len = len(prompt_token_ids)
    state = MaskState(x=[*prompt_token_ids, *([mask_token_id] * max_tokens)],
                      prompt_len=prompt_len, mask_token_id=mask_token_id,
                      eos_token_id=eos_token_id)
    exact_kv = False
    if decode_strategy == "block_threshold":
        # D2F over the exact prompt + frozen-block K/V: blocks count from the
        # prompt, each proposal forwards the active block (and the Dream shift's
        # feeder row) over the cached prefix (backends/device_runtime.py:108-183)
        layout = None
        policy = BlockThresholdCommit(confidence_threshold=confidence_threshold,
                                      block_size=block_size, requested_steps=steps)
        origin = prompt_len
        exact_kv = True
        loop_kind = "rocm_dream_block_threshold"
    elif decode_strategy == "bd3_fixed_quota":
        layout = BlockLayout(start=prompt_len, length=max_tokens, block_size=block_size, origin=0)
        policy = BD3FixedQuotaCommit(block_size=block_size, requested_steps=steps,
                                     generated_token_count=max_tokens, block_layout=layout,
                                     requires_prompt_block_alignment=requires_prompt_block_alignment)
        origin = 0
        loop_kind = "rocm_qwen3_bd3_fixed_quota"
    else:
        layout = None
        policy = FixedQuotaCommit(block_size=block_size, requested_steps=steps,
                                  generated_token_count=max_tokens)
        origin = prompt_len
        loop_kind = "rocm_bidirectional_fixed_quota"
    session.start_device(state.x, prompt_len=origin, block_size=block_size,
                         mask_token_id=mask_token_id, exact_kv=exact_kv, steps=steps,
                         memory_budget_bytes=memory_budget_bytes,
                         temperature=float(temperature), seed=int(seed))

    def propose(plan):
        if decode_strategy == "block_threshold":
            block = (min(plan.frontier) - origin) // block_size
            frozen = origin + block * block_size
            return session.propose_device(plan.frontier,
                                          window_end=min(len(state.x), frozen + block_size),
                                          frozen_prefix=frozen)
        if layout is None:
            return session.propose_device(plan.frontier, window_end=len(state.x),
                                          frozen_prefix=state.prompt_len)
        block = (min(plan.frontier) - origin) // block_size
        frozen = origin + block * block_size
        return session.propose_device(plan.frontier, window_end=plan.window_end,
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
