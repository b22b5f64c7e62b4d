"""The golden-vector corpus (tests/golden/vectors/, written by
tests/golden/make_vectors.py from the oracle): format round trip, model
identity, and replay of the oracle itself at the same-backend tier."""
from __future__ import annotations

import importlib.util
import os

import pytest

from diffusorrt_amd import golden as G
from diffusorrt_amd import synthetic as syn

from helpers import oracle_weights, tiny_dream_geometry, tiny_geometry

HERE = os.path.dirname(os.path.abspath(__file__))
CORPUS = os.path.join(HERE, "golden", "vectors")


def _make_vectors_module():
    spec = importlib.util.spec_from_file_location(
        "make_vectors", os.path.join(HERE, "golden", "make_vectors.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def model_for(vector):
    """Rebuild the vector's synthetic model and prove it is the same one."""
    _, name, kind, seed, wdigest = vector.model_identity.split(":")
    g = {"tiny-bd3": tiny_geometry, "tiny-dream": tiny_dream_geometry}[name]()
    model = syn.build_model(g, kind, int(seed.removeprefix("seed")))
    assert G.model_weights_digest(model.weights) == wdigest, vector.label
    return model


def oracle_candidate(vector):
    mv = _make_vectors_module()
    model = model_for(vector)
    g = model.geometry
    W, cfg = oracle_weights(model), syn.oracle_config(g, "q4")
    rq = vector.request_dict
    out, trace, logits_fn = mv.oracle_decode(
        W, cfg, g, rq["decode_strategy"], rq["prompt_ids"], rq["max_tokens"], rq["steps"],
        rq["block_size"], rq["eos_token_id"])
    x0 = list(rq["prompt_ids"]) + [rq["mask_token_id"]] * rq["max_tokens"]
    first = trace[0]
    import numpy as np

    logits = np.asarray(logits_fn(x0, first["frontier"], first["window_end"]), np.float32)
    return G.schedule_control_plane(rq, trace, out), logits, out["x"][len(rq["prompt_ids"]):]


def test_corpus_loads_and_round_trips():
    vectors = G.load_corpus(CORPUS)
    assert len(vectors) == 4
    for v in vectors:
        again = G.GoldenVector.from_dict(v.to_dict())
        assert again == v
        assert v.source == "numpy_reference" and len(v.logits_digest) == 64
        cp = v.control_plane
        assert cp["forward_count"] == len(cp["quotas"]) == len(cp["frontier_sizes"])
        assert sum(cp["quotas"]) == cp["committed_token_count"]
        model_for(v)
    eos = [v for v in vectors if v.label.endswith("eos-stop")][0]
    # the end token is committed in the first block and the decode stops at its boundary
    assert eos.control_plane["hit_eos"] and eos.control_plane["forward_count"] == 4


def test_oracle_replays_its_own_corpus_bit_exact():
    vectors = G.load_corpus(CORPUS)
    outcomes = G.replay(vectors, oracle_candidate, tier=G.ParityTier.SAME_BACKEND_TENSOR)
    assert all(o.passed for o in outcomes), outcomes


def test_replay_names_what_differs():
    v = G.load_corpus(CORPUS)[0]

    def wrong_schedule(vector):
        cp, logits, toks = oracle_candidate(vector)
        cp = dict(cp, quotas=tuple(q + 1 for q in cp["quotas"]))
        return cp, logits, toks

    def wrong_token(vector):
        cp, logits, toks = oracle_candidate(vector)
        toks = list(toks)
        toks[3] += 1
        return cp, None, toks

    def wrong_logits(vector):
        cp, logits, toks = oracle_candidate(vector)
        logits = logits.copy()
        logits[0, 0] += 1e-6
        return cp, logits, toks

    (o,) = G.replay([v], wrong_schedule, tier=G.ParityTier.CONTROL_PLANE)
    assert not o.passed and o.detail.startswith("quotas")
    (o,) = G.replay([v], wrong_token, tier=G.ParityTier.CROSS_BACKEND)
    assert not o.passed and "index 3" in o.detail
    (o,) = G.replay([v], wrong_logits, tier=G.ParityTier.SAME_BACKEND_TENSOR)
    assert not o.passed and "digest" in o.detail
