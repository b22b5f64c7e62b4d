"""Writes the golden fixtures under tests/golden/ (run from the repository root).

1. ``bd3_mask_cases.json``: the reference's own BD3 parity cases (input ids,
   masked positions, selected rows across absolute block boundaries), copied as
   data from ``python/src/edllm/model_coverage/data/cases/qwen3_06b_bd3lm_v0_1.json``
   of the reference; the reference ships no expected logits for them.
2. ``bd3_real_vocab_logits.json``: for each case, the oracle's logits of the
   selected rows (staircase mask, block 32, absolute blocks) on a small seeded
   model with the real BD3 vocabulary, summarised per row (float64 max-prob
   score, first argmax, second-largest logit, log-sum-exp, row sum / sum of squares, and the logits
   at fixed probe ids; for q4 also the score, argmax and top two logits of the same rows with
   the cached K/V rounded to fp16). The GPU tests compare the device path with these.

Usage: python tests/golden/make_golden.py [--reference-root PATH]
"""
from __future__ import annotations

import argparse
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from diffusorrt_amd import synthetic as syn  # noqa: E402
from oracle import forward as F  # noqa: E402
from oracle import ops as O  # noqa: E402

CASES_REL = "python/src/edllm/model_coverage/data/cases/qwen3_06b_bd3lm_v0_1.json"
PROBE_IDS = [0, 1, 1000, 151643, 151645, 151669, 151935]
SEED = 21


def real_vocab_geometry() -> syn.ModelGeometry:
    """Two BD3-shaped layers (qk-norm, GQA 2:1, head_dim 128) with the real
    Qwen3 BD3 vocabulary and special ids."""
    return syn.ModelGeometry(
        name="tiny-bd3-real-vocab", layer_count=2, hidden_size=256, num_heads=4,
        num_kv_heads=2, head_dim=128, intermediate_size=512, vocab_size=151936,
        rms_norm_eps=1e-6, rope_theta=1e6, qk_norm=True, qkv_bias=False,
        logits_convention="raw", mask_token_id=151669, eos_token_id=151645,
        tie_word_embeddings=True, max_position_embeddings=4096)


def summarise(logits: np.ndarray) -> list:
    scores, tokens = O.raw_max_prob(logits)
    out = []
    for r in range(logits.shape[0]):
        row = logits[r].astype(np.float64)
        m = row.max()
        second = float(np.partition(row, -2)[-2])
        out.append({"score": float(scores[r]), "argmax": int(tokens[r]), "second": second,
                    "lse": float(m + np.log(np.exp(row - m).sum())),
                    "sum": float(row.sum()), "sumsq": float((row * row).sum()),
                    "max": float(m), "probe": [float(row[i]) for i in PROBE_IDS]})
    return out


def kv_round_f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def oracle_case_logits(model, kind: str, case: dict, kv_round=None) -> np.ndarray:
    weights = {}
    for k, v in syn.to_oracle_weights(model).items():
        weights[k] = O.Q4Weight(*v) if isinstance(v, tuple) else v
    cfg = syn.oracle_config(model.geometry, kind)
    return F.forward_full(weights, cfg, case["input_ids"], mask_kind="d2f_hybrid",
                          mask_geometry=(0, 32), output_rows=case["selected_rows"],
                          kv_round=kv_round)


def add_kv_summary(rows: list, logits: np.ndarray) -> list:
    """The same rows with the cached K/V rounded to fp16 (the device cache's
    storage type): score, argmax, top two logits."""
    scores, tokens = O.raw_max_prob(logits)
    for r, row in enumerate(rows):
        lr = logits[r].astype(np.float64)
        row.update(kv_score=float(scores[r]), kv_argmax=int(tokens[r]), kv_max=float(lr.max()),
                   kv_second=float(np.partition(lr, -2)[-2]))
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference-root", default="/root/reference")
    args = ap.parse_args()
    src = os.path.join(args.reference_root, CASES_REL)
    with open(src) as f:
        ref = json.load(f)
    cases = [{k: c[k] for k in ("name", "input_ids", "masked_positions", "selected_rows")}
             for c in ref["cases"]]
    with open(os.path.join(HERE, "bd3_mask_cases.json"), "w") as f:
        json.dump({"source": "reference " + CASES_REL, "candidate_key": ref["candidate_key"],
                   "cases": cases}, f, indent=1)
    g = real_vocab_geometry()
    out = {"seed": SEED, "geometry": g.name, "probe_ids": PROBE_IDS, "mask": "staircase block 32",
           "kinds": {}}
    for kind in ("q4", "bf16"):
        model = syn.build_model(g, kind, seed=SEED)
        out["kinds"][kind] = {}
        for c in cases:
            rows = summarise(oracle_case_logits(model, kind, c))
            if kind == "q4":
                rows = add_kv_summary(rows, oracle_case_logits(model, kind, c, kv_round_f16))
            out["kinds"][kind][c["name"]] = rows
    with open(os.path.join(HERE, "bd3_real_vocab_logits.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", len(cases), "cases")


if __name__ == "__main__":
    main()
