"""Decode-loop control plane restated as plain loops (oracle; test-only).

Restates, for the two fixed-quota strategies on this path:
  * ``MaskState`` masked scan / commit / finalize
    (``backends/diffusion_runtime.py:387-558``),
  * ``BlockLayout`` (``:1099-1141``),
  * ``FixedQuotaCommit`` (``:1145-1196``) and ``BD3FixedQuotaCommit``
    (``:1200-1346``),
  * ``run_decode_loop`` forward -> score -> select -> commit (``:1829-1991``)
    with ``exclude_mask_token=False`` (``:2199-2264``),
  * and Dream's block-threshold policy: the block walk of
    ``_block_frontier_plan`` (``:1023-1052``), the threshold choice with its
    floor of one (``:302-314``) and the MASK column left out of the scoring
    (``exclude_mask_token=True``, ``:256-282, 1955-1958``),
  * ``DecodeRequest.prepare`` canvas + BD3 absolute layout
    (``backends/decode_session.py:113-160``).

Deliberately written as the most literal loops (no shared code with the
product's control plane) so that tests can cross-check the two.
"""
from __future__ import annotations

from . import ops


def block_span(start, length, block_size, origin, index):
    """``BlockLayout.span``: the index-th grid block clipped to the interval."""
    first = (start - origin) // block_size
    grid_start = origin + (first + index) * block_size
    return max(start, grid_start), min(start + length, grid_start + block_size)


def block_count(start, length, block_size, origin):
    if length == 0:
        return 0
    first = (start - origin) // block_size
    last = (start + length - 1 - origin) // block_size
    return last - first + 1


def finalize(x, prompt_len, mask_id, eos_id):
    """``MaskState.finalize`` (``diffusion_runtime.py:526-558``)."""
    gen = list(x[prompt_len:])
    if eos_id in gen:
        answer = gen[:gen.index(eos_id)]
        hit_eos, reason = True, "stop"
    else:
        answer, hit_eos, reason = gen, False, "length"
    remaining = answer.count(mask_id)
    if remaining:
        reason = "length"
        visible = answer[:answer.index(mask_id)]
    else:
        visible = answer
    return {"visible_token_ids": visible, "hit_eos": hit_eos,
            "remaining_mask_count": remaining, "finish_reason": reason}


def bd3_schedule_step(x, prompt_len, mask_id, eos_id, block_size, steps, step, state):
    """One ``BD3FixedQuotaCommit.plan`` call. ``state`` carries the active block
    id and its (base, remainder). Returns ``("stop"|"skip"|"go", frontier,
    window_end, quota)``."""
    gen_len = len(x) - prompt_len
    blocks = block_count(prompt_len, gen_len, block_size, 0)
    sched_blocks = (gen_len + block_size - 1) // block_size
    spb = (steps + sched_blocks - 1) // sched_blocks if blocks else 0
    if step >= blocks * spb:
        return "stop", [], None, 0
    if prompt_len % block_size:
        raise ValueError("BD3LM Candidate prompt length must be a multiple of block_size")
    if step % spb == 0 and eos_id in x[prompt_len:]:
        return "stop", [], None, 0
    masked = [p for p in range(prompt_len, len(x)) if x[p] == mask_id]
    if not masked:
        return "stop", [], None, 0
    bid = step // spb
    bstart, bend = block_span(prompt_len, gen_len, block_size, 0, bid)
    frontier = [p for p in masked if bstart <= p < bend]
    if state.get("block") != bid:
        state["block"] = bid
        state["base"], state["rem"] = divmod(len(frontier), spb)
    rnd = step % spb
    quota = state["base"] + (1 if rnd < state["rem"] else 0)
    if not frontier or quota == 0:
        return "skip", [], None, 0
    return "go", frontier, bend, quota


def fixed_quota_schedule_step(x, prompt_len, mask_id, block_size, steps, step, state):
    """One ``FixedQuotaCommit.plan`` call (prompt-relative logical blocks, no
    window end: the whole canvas is forwarded)."""
    fillable = list(range(prompt_len, len(x)))
    nblocks = (len(fillable) + block_size - 1) // block_size
    spb = (steps + nblocks - 1) // nblocks if nblocks else 0
    if step >= nblocks * spb:
        return "stop", [], None, 0
    block = step // spb
    positions = fillable[block * block_size: block * block_size + block_size]
    frontier = [p for p in positions if x[p] == mask_id]
    if state.get("block") != block:
        state["block"] = block
        state["base"], state["rem"] = divmod(len(frontier), spb)
    quota = state["base"] + (1 if step % spb < state["rem"] else 0)
    if not frontier or quota == 0:
        return "skip", [], None, 0
    return "go", frontier, None, quota


def run_fixed_quota_decode(prompt_ids, *, max_tokens, mask_id, eos_id, block_size, steps,
                           strategy, frontier_logits_fn, trace=None):
    """Drive a whole decode: ``frontier_logits_fn(x, frontier, window_end)``
    returns fp32 frontier logits (convention already applied). Greedy scoring is
    the float64 max-prob (``diffusion_runtime.py:179-192``) and the commit is
    ``argsort(-conf)[:quota]``; the MASK column is kept (``exclude_mask_token``
    is False for both strategies, ``:2215-2219, :2257-2264``)."""
    x = list(prompt_ids) + [mask_id] * max_tokens
    prompt_len = len(prompt_ids)
    gen_len = max_tokens
    if strategy == "bd3_fixed_quota":
        blocks = block_count(prompt_len, gen_len, block_size, 0)
        sched = (gen_len + block_size - 1) // block_size
        spb = (steps + sched - 1) // sched if blocks else 0
        limit = blocks * spb
    else:
        nblocks = (gen_len + block_size - 1) // block_size
        spb = (steps + nblocks - 1) // nblocks if nblocks else 0
        limit = nblocks * spb
    state = {}
    forwards = 0
    committed = 0
    for step in range(limit):
        if strategy == "bd3_fixed_quota":
            kind, frontier, wend, quota = bd3_schedule_step(
                x, prompt_len, mask_id, eos_id, block_size, steps, step, state)
        else:
            kind, frontier, wend, quota = fixed_quota_schedule_step(
                x, prompt_len, mask_id, block_size, steps, step, state)
        if kind == "stop":
            break
        if kind == "skip":
            continue
        logits = frontier_logits_fn(list(x), list(frontier), wend)
        forwards += 1
        scores, tokens = ops.raw_max_prob(logits)
        chosen = ops.topk_count_choices(scores, quota)
        if trace is not None:
            trace.append({"step": step, "frontier": list(frontier), "window_end": wend,
                          "scores": [float(s) for s in scores], "tokens": list(tokens),
                          "chosen": list(chosen), "quota": quota})
        for r in chosen:
            x[frontier[r]] = int(tokens[r])
        committed += len(chosen)
    out = finalize(x, prompt_len, mask_id, eos_id)
    out.update({"x": x, "forward_count": forwards, "committed_token_count": committed})
    return out


def excluded_max_prob(logits, mask_id):
    """``_exclude_mask_token`` then the float64 max-prob (``diffusion_runtime.py:
    256-282, 179-192``): the MASK column becomes -inf before softmax and argmax."""
    import numpy as np

    values = np.array(logits, dtype=np.float32, copy=True)
    if 0 <= int(mask_id) < values.shape[1]:
        values[:, int(mask_id)] = -np.inf
    return ops.raw_max_prob(values)


def threshold_pick(scores, threshold):
    """Every row with ``score >= threshold``, else the first most confident row."""
    picked = [i for i, s in enumerate(scores) if float(s) >= float(threshold)]
    if picked:
        return picked
    best = 0
    for i, s in enumerate(scores):
        if float(s) > float(scores[best]):
            best = i
    return [best]


def run_block_threshold_decode(prompt_ids, *, max_tokens, mask_id, eos_id, block_size, steps,
                               threshold, frontier_logits_fn, trace=None):
    """Drive Dream's block-threshold decode. ``frontier_logits_fn(x, frontier,
    window_end)`` returns the frontier's fp32 logits (convention applied) for the
    canvas forwarded up to ``window_end`` = the end of the active block (rows past
    it are dead: the d2f mask hides them from the active rows)."""
    x = list(prompt_ids) + [mask_id] * max_tokens
    prompt_len = len(prompt_ids)
    block_index = 0
    forwards = committed = 0
    for step in range(steps):
        frontier = []
        while block_index < max_tokens:
            lo = prompt_len + block_index
            hi = min(lo + block_size, len(x))
            frontier = [p for p in range(lo, hi) if x[p] == mask_id]
            if frontier:
                break
            block_index += block_size
        if not frontier:
            break
        window_end = min(len(x), prompt_len + block_index + block_size)
        logits = frontier_logits_fn(list(x), list(frontier), window_end)
        forwards += 1
        scores, tokens = excluded_max_prob(logits, mask_id)
        chosen = threshold_pick(scores, threshold)
        if trace is not None:
            trace.append({"step": step, "frontier": list(frontier), "window_end": window_end,
                          "scores": [float(s) for s in scores], "tokens": list(tokens),
                          "chosen": list(chosen), "quota": len(chosen)})
        for r in chosen:
            x[frontier[r]] = int(tokens[r])
        committed += len(chosen)
    out = finalize(x, prompt_len, mask_id, eos_id)
    out.update({"x": x, "forward_count": forwards, "committed_token_count": committed})
    return out
