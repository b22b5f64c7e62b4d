"""Writes the golden-vector corpus under tests/golden/vectors/ (run from the
repository root): the oracle's decodes of small seeded models, in the golden
vector format (``source = "numpy_reference"``).

Each vector's request is a fixed-quota decode of a tiny model (the test helpers'
BD3-layout and Dream-layout geometries, q4 weights from a fixed seed). Its
model identity names the model and the sha256 of its weights, so a replay can
prove it rebuilt the same model. Prompts are drawn from a seed and the first
seed whose oracle trajectory is robust is used: every committed token leads its
row by more than 1e-3 in probability, the last chosen row of each step
outscores the first unchosen one by more than 1e-3 (relative), and the same
decode with every operand the device stores in fp16 rounded to fp16 commits
exactly the same tokens at the same positions.

Usage: python tests/golden/make_vectors.py
"""
from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402

from diffusorrt_amd import golden as G  # noqa: E402
from diffusorrt_amd import synthetic as syn  # noqa: E402
from helpers import oracle_weights, tiny_dream_geometry, tiny_geometry  # noqa: E402
from oracle import forward as F  # noqa: E402
from oracle import ops as O  # noqa: E402
from oracle import policy as P  # noqa: E402

CLEAR = 1e-3
OUT = os.path.join(HERE, "vectors")

CASES = [
    # label, geometry, weight seed, strategy, prompt len, max tokens, steps, block, eos override.
    # The Dream case commits its whole canvas in one step: under the bidirectional
    # mask every MASK row sees the same context and differs only by position, so
    # the rows' scores nearly tie and a quota boundary between them is not robust.
    ("bd3__tiny-q4__one-block", "bd3", 10, "bd3_fixed_quota", 64, 32, 4, 32, None),
    ("bd3__tiny-q4__two-blocks", "bd3", 11, "bd3_fixed_quota", 32, 64, 8, 32, None),
    ("bd3__tiny-q4__eos-stop", "bd3", 10, "bd3_fixed_quota", 64, 64, 8, 32, "first"),
    ("dream__tiny-q4__fixed-quota-32", "dream", 12, "fixed_quota", 48, 32, 1, 256, None),
]


def r16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def _geometry(kind):
    return tiny_geometry() if kind == "bd3" else tiny_dream_geometry()


def identity(kind, seed, model) -> str:
    g = model.geometry
    return f"synthetic:{g.name}:q4:seed{seed}:{G.model_weights_digest(model.weights)}"


def oracle_decode(W, cfg, g, strategy, prompt, max_tokens, steps, block, eos, rnd=None):
    def logits_fn(x, frontier, wend):
        if strategy == "bd3_fixed_quota":
            return F.forward_full(W, cfg, x[:wend], mask_kind="d2f_hybrid",
                                  mask_geometry=(0, block), output_rows=frontier,
                                  operand_round=rnd)
        return F.window_logits(W, cfg, x, frontier, mask_kind="bidirectional",
                               mask_geometry=None, logits_convention=g.logits_convention,
                               operand_round=rnd)

    trace = []
    out = P.run_fixed_quota_decode(prompt, max_tokens=max_tokens, mask_id=g.mask_token_id,
                                   eos_id=eos, block_size=block, steps=steps,
                                   strategy=strategy, frontier_logits_fn=logits_fn, trace=trace)
    return out, trace, logits_fn


def clear_of_ties(trace, logits_fn, x0):
    """Every decision of the trajectory has a margin above CLEAR."""
    x = list(x0)
    for t in trace:
        logits = np.asarray(logits_fn(list(x), t["frontier"], t["window_end"]), dtype=np.float64)
        p = np.exp(logits - logits.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        top2 = np.sort(p, axis=1)[:, -2:]
        for r in t["chosen"]:
            if (top2[r, 1] - top2[r, 0]) / top2[r, 1] <= CLEAR:
                return False
        scores = np.asarray(t["scores"])
        order = np.argsort(-scores, kind="stable")
        k = len(t["chosen"])
        if k < len(order):
            a, b = scores[order[k - 1]], scores[order[k]]
            if (a - b) / a <= CLEAR:
                return False
        for r in t["chosen"]:
            x[t["frontier"][r]] = t["tokens"][r]
    return True


def main():
    vectors = []
    for label, kind, wseed, strategy, plen, max_tokens, steps, block, eos_mode in CASES:
        g = _geometry(kind)
        model = syn.build_model(g, "q4", wseed)
        W, cfg = oracle_weights(model), syn.oracle_config(g, "q4")
        for pseed in range(100, 200):
            prompt = np.random.default_rng(pseed).integers(0, 900, plen).tolist()
            eos = g.eos_token_id
            if eos_mode == "first":
                # end token = a token the model commits in the first generated block,
                # so the decode stops at that block's boundary
                out, _, _ = oracle_decode(W, cfg, g, strategy, prompt, max_tokens, steps,
                                          block, eos)
                eos = int(out["x"][plen + 5])
            out, trace, logits_fn = oracle_decode(W, cfg, g, strategy, prompt, max_tokens,
                                                  steps, block, eos)
            x0 = prompt + [g.mask_token_id] * max_tokens
            if not clear_of_ties(trace, logits_fn, x0):
                continue
            out16, _, _ = oracle_decode(W, cfg, g, strategy, prompt, max_tokens, steps, block,
                                        eos, rnd=r16)
            if out16["x"] == out["x"]:
                break
        else:
            raise SystemExit(f"{label}: no tie-free prompt seed")
        request = {"prompt_ids": prompt, "prompt_seed": pseed, "max_tokens": max_tokens,
                   "decode_strategy": strategy, "block_size": block, "steps": steps,
                   "mask_token_id": g.mask_token_id, "eos_token_id": eos, "temperature": 0.0,
                   "seed": 0, "requires_prompt_block_alignment": True}
        control = G.schedule_control_plane(request, trace, out)
        first = trace[0]
        logits = np.asarray(logits_fn(x0, first["frontier"], first["window_end"]),
                            dtype=np.float32)
        vectors.append(G.record_vector(
            label=label, source="numpy_reference", model_identity=identity(kind, wseed, model),
            request_dict=request, control_plane=control, logits=logits,
            committed_tokens=out["x"][plen:]))
        print(f"{label}: prompt seed {pseed}, {control['forward_count']} forwards, "
              f"{control['finish_reason']}", flush=True)
    G.write_corpus(vectors, OUT)


if __name__ == "__main__":
    main()
