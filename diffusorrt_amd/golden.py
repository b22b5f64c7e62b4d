"""Golden vectors and cross-backend replay for the denoise loop.

A vector records what one implementation produced for one request: the
control plane (the schedule, integer logic: bit-exact at every tier), a digest
and shape of the first forward's frontier logits (bit-exact within one backend),
and the committed tokens (the cross-backend promise). Format, tiers and replay
follow the reference's ``abi/golden.py:38-136`` and ``abi/parity.py:1-100``
(``python/src/edllm/``); vectors written by either side load on the other.

``RocmCandidate`` drives this backend's device session on a vector's request.
The control plane it reports is the schedule only -- per forward the quota, the
frontier size and the window end, plus the step arithmetic and the totals -- the
facts that do not depend on which rows scored highest, so two backends agree on
it whenever their tokens agree.
"""
from __future__ import annotations

import hashlib
import json
import pathlib
from dataclasses import dataclass
from enum import IntEnum

import numpy as np


class ParityTier(IntEnum):
    CONTROL_PLANE = 0        # bit-exact integer logic
    SAME_BACKEND_TENSOR = 1  # bit-exact logits digest
    CROSS_BACKEND = 2        # committed-token equality (logits within tolerance)


@dataclass(frozen=True)
class ParityResult:
    tier: int
    passed: bool
    detail: str


def digest(array) -> str:
    """sha256 of the little-endian C-order bytes (``abi/parity.py:31-36``)."""
    a = np.ascontiguousarray(array)
    if a.dtype.byteorder == ">":
        a = a.astype(a.dtype.newbyteorder("<"))
    return hashlib.sha256(a.tobytes()).hexdigest()


def _result(tier: int, problem: str | None, ok: str) -> ParityResult:
    return ParityResult(tier, problem is None, ok if problem is None else problem)


def compare_control_plane(a: dict, b: dict) -> ParityResult:
    """Bit-exact: the result names the first key, in sorted order, that one side
    lacks or whose values differ."""
    missing = object()
    for key in sorted(set(a) | set(b)):
        va, vb = a.get(key, missing), b.get(key, missing)
        if va is missing or vb is missing:
            return _result(ParityTier.CONTROL_PLANE, f"{key}: present on one side only", "")
        if va != vb:
            return _result(ParityTier.CONTROL_PLANE, f"{key}: {va!r} != {vb!r}", "")
    return _result(ParityTier.CONTROL_PLANE, None, "identical")


def compare_tensor_tolerant(a, b, *, rtol: float, atol: float) -> ParityResult:
    """Elementwise |a - b| <= atol + rtol * |b|; a failure reports how many
    elements miss the bound and the largest difference."""
    x = np.asarray(a, dtype=np.float64)
    y = np.asarray(b, dtype=np.float64)
    if x.shape != y.shape:
        return _result(ParityTier.CROSS_BACKEND, f"shape {x.shape} != {y.shape}", "")
    miss = ~np.isclose(x, y, rtol=rtol, atol=atol)
    if not miss.any():
        return _result(ParityTier.CROSS_BACKEND, None, "within tolerance")
    worst = float(np.max(np.abs(x - y)))
    return _result(ParityTier.CROSS_BACKEND,
                   f"{int(miss.sum())} elements beyond rtol={rtol} atol={atol} "
                   f"(max abs diff {worst:.3e})", "")


def compare_tokens(a, b) -> ParityResult:
    """Committed-token equality, the promise that holds across backends; a
    failure names the first index where the two sequences part."""
    x, y = np.asarray(a), np.asarray(b)
    if x.shape != y.shape:
        return _result(ParityTier.CROSS_BACKEND, f"token shape {x.shape} != {y.shape}", "")
    where = np.flatnonzero(x.ravel() != y.ravel())
    if where.size == 0:
        return _result(ParityTier.CROSS_BACKEND, None, "tokens identical")
    i = int(where[0])
    return _result(ParityTier.CROSS_BACKEND,
                   f"tokens differ from index {i} on ({x.flat[i]} != {y.flat[i]}; "
                   f"{where.size} positions in all)", "")


def _jsonable(v):
    if isinstance(v, tuple):
        return [_jsonable(x) for x in v]
    if isinstance(v, list):
        return [_jsonable(x) for x in v]
    if isinstance(v, dict):
        return {str(k): _jsonable(x) for k, x in v.items()}
    return v


def _tupleize(v):
    if isinstance(v, list):
        return tuple(_tupleize(x) for x in v)
    if isinstance(v, dict):
        return {int(k) if str(k).lstrip("-").isdigit() else k: _tupleize(x) for k, x in v.items()}
    return v


@dataclass(frozen=True)
class GoldenVector:
    label: str
    source: str            # e.g. "numpy_reference", "mlx_local", "rocm"
    model_identity: str    # package / model name + weights digest
    request_dict: dict
    control_plane: dict
    logits_digest: str
    logits_shape: tuple
    committed_tokens: tuple

    def to_dict(self) -> dict:
        return {"label": self.label, "source": self.source,
                "model_identity": self.model_identity, "request": self.request_dict,
                "control_plane": {k: _jsonable(v) for k, v in self.control_plane.items()},
                "logits_digest": self.logits_digest, "logits_shape": list(self.logits_shape),
                "committed_tokens": list(self.committed_tokens)}

    @classmethod
    def from_dict(cls, d: dict) -> "GoldenVector":
        return cls(label=d["label"], source=d["source"], model_identity=d["model_identity"],
                   request_dict=d["request"],
                   control_plane={k: _tupleize(v) for k, v in d["control_plane"].items()},
                   logits_digest=d["logits_digest"],
                   logits_shape=tuple(int(x) for x in d["logits_shape"]),
                   committed_tokens=tuple(int(t) for t in d["committed_tokens"]))


@dataclass(frozen=True)
class ReplayOutcome:
    label: str
    passed: bool
    detail: str


def record_vector(*, label: str, source: str, model_identity: str, request_dict: dict,
                  control_plane: dict, logits, committed_tokens) -> GoldenVector:
    shape = tuple(int(d) for d in np.shape(logits))
    return GoldenVector(label=label, source=source, model_identity=model_identity,
                        request_dict=dict(request_dict), control_plane=dict(control_plane),
                        logits_digest=digest(logits),
                        logits_shape=(shape[0], shape[1] if len(shape) > 1 else 0),
                        committed_tokens=tuple(int(t) for t in committed_tokens))


def write_corpus(vectors, directory) -> None:
    path = pathlib.Path(directory)
    path.mkdir(parents=True, exist_ok=True)
    for v in vectors:
        (path / (v.label.replace("/", "__") + ".json")).write_text(
            json.dumps(v.to_dict(), indent=2, sort_keys=True) + "\n")


def load_corpus(directory) -> list:
    path = pathlib.Path(directory)
    if not path.is_dir():
        return []
    return [GoldenVector.from_dict(json.loads(f.read_text()))
            for f in sorted(path.glob("*.json"))]


def replay(vectors, candidate, *, tier: ParityTier) -> list:
    """``candidate(vector) -> (control_plane, logits or None, tokens)``; the control
    plane is compared at every tier, the logits digest from tier 1 up when the
    candidate returns logits, then the committed tokens."""
    out = []
    for v in vectors:
        control, logits, tokens = candidate(v)
        r = compare_control_plane(v.control_plane, control)
        if not r.passed:
            out.append(ReplayOutcome(v.label, False, r.detail))
            continue
        if tier >= ParityTier.SAME_BACKEND_TENSOR and logits is not None:
            if digest(logits) != v.logits_digest:
                out.append(ReplayOutcome(v.label, False,
                                         f"logits digest differs (tier {ParityTier(tier).name})"))
                continue
        t = compare_tokens(list(v.committed_tokens), list(tokens))
        out.append(ReplayOutcome(v.label, t.passed, "ok" if t.passed else t.detail))
    return out


def model_weights_digest(weights: dict) -> str:
    """sha256 over the sorted weight names and their bytes (a q4 bundle's words,
    scales and biases in that order): the weights part of a model identity."""
    import torch

    h = hashlib.sha256()
    for name in sorted(weights):
        value = weights[name]
        parts = ((value.w_q, value.scales, value.biases) if hasattr(value, "w_q") else (value,))
        h.update(name.encode())
        for t in parts:
            t = t.detach().cpu().contiguous()
            h.update(str(tuple(t.shape)).encode() + str(t.dtype).encode())
            h.update(t.view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


# ----------------------------------------------------------------- the schedule


def schedule_control_plane(request: dict, steps_trace: list, result: dict) -> dict:
    """The score-independent control plane of one decode: the request's step
    arithmetic, and per forward its quota, frontier size and window end (-1 when
    the strategy has none), plus the totals and how the decode ended."""
    strategy = request["decode_strategy"]
    block = int(request["block_size"])
    steps = int(request["steps"])
    n_blocks = (int(request["max_tokens"]) + block - 1) // block
    spb = (steps + n_blocks - 1) // n_blocks if n_blocks else 0
    return {
        "decode_strategy": strategy,
        "steps_per_block": spb,
        "iteration_limit": n_blocks * spb,
        "forward_count": len(steps_trace),
        "quotas": tuple(int(t["quota"]) for t in steps_trace),
        "frontier_sizes": tuple(len(t["frontier"]) for t in steps_trace),
        "window_ends": tuple(-1 if t["window_end"] is None or strategy == "fixed_quota"
                             else int(t["window_end"]) for t in steps_trace),
        "committed_token_count": int(result["committed_token_count"]),
        "finish_reason": str(result["finish_reason"]),
        "hit_eos": bool(result["hit_eos"]),
    }


class RocmCandidate:
    """Replays vectors on a ``Runtime``: runs each request through the device
    session and the fixed-quota loop; with ``with_logits`` also returns the first
    forward's frontier logits (``execute_window`` on the initial canvas)."""

    def __init__(self, runtime, *, with_logits: bool = False):
        self.runtime = runtime
        self.with_logits = with_logits

    def __call__(self, vector: GoldenVector):
        from .decode import generate_device_tokens
        from .runtime import bd3_session_config, fixed_quota_session_config

        rq = vector.request_dict
        prompt = [int(t) for t in rq["prompt_ids"]]
        max_tokens, block, steps = int(rq["max_tokens"]), int(rq["block_size"]), int(rq["steps"])
        strategy = rq["decode_strategy"]
        total = len(prompt) + max_tokens
        make = bd3_session_config if strategy == "bd3_fixed_quota" else fixed_quota_session_config
        trace = []
        with self.runtime.session(make(block, steps, total)) as s:
            res = generate_device_tokens(
                s, prompt, max_tokens=max_tokens, mask_token_id=int(rq["mask_token_id"]),
                eos_token_id=int(rq["eos_token_id"]), steps=steps, block_size=block,
                decode_strategy=strategy,
                requires_prompt_block_alignment=bool(rq.get("requires_prompt_block_alignment",
                                                            True)),
                temperature=float(rq.get("temperature", 0.0)), seed=int(rq.get("seed", 0)),
                trace=trace)
        for t in trace:
            t["quota"] = len(t["chosen"])
        control = schedule_control_plane(rq, trace, {
            "committed_token_count": res.committed_token_count,
            "finish_reason": res.finish_reason, "hit_eos": res.hit_eos})
        logits = None
        if self.with_logits and trace:
            first = trace[0]
            canvas = prompt + [int(rq["mask_token_id"])] * max_tokens
            wend = first["window_end"] if strategy == "bd3_fixed_quota" else len(canvas)
            with self.runtime.session(make(block, steps, total)) as s:
                geo = (0, block) if strategy == "bd3_fixed_quota" else None
                logits = s.execute_window(canvas[:wend], first["frontier"],
                                          mask_geometry=geo).array()
        return control, logits, res.full_token_ids[len(prompt):]
