"""The oracle's golden-vector corpus replayed on the device session: the
schedule bit-exact and the committed tokens equal (the cross-backend tier), and
the first forward's frontier logits within the logits bar."""
from __future__ import annotations

import pytest

from diffusorrt_amd import golden as G

from helpers import LOGITS_REL_TOL, rel_err_rows
from test_golden_vectors import CORPUS, model_for, oracle_candidate

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def test_rocm_replays_the_oracle_corpus():
    from diffusorrt_amd.runtime import Runtime

    vectors = G.load_corpus(CORPUS)
    assert len(vectors) == 4
    for v in vectors:
        print("[case] replay", v.label, flush=True)
        rt = Runtime(model_for(v), max_forward_rows=512, max_positions=1024)
        (outcome,) = G.replay([v], G.RocmCandidate(rt), tier=G.ParityTier.CROSS_BACKEND)
        assert outcome.passed, outcome
        control, logits, tokens = G.RocmCandidate(rt, with_logits=True)(v)
        _, ref, _ = oracle_candidate(v)
        err = rel_err_rows(logits, ref)
        print(f"[case]   first-forward logits rel err max={err.max():.2e}", flush=True)
        assert logits.shape == v.logits_shape and err.max() < LOGITS_REL_TOL
        rt.close()
