"""Failure handling of the device path, forced from the host so that every
kernel still runs to completion:

* the split-K linears' XCD placement: a wrong XCD count (``DRT_N_XCC``) makes
  the kernels' own placement check fire; the forward finishes and the host
  raises, and the GPU is then fine for a new runtime;
* the fenced split-K exchange (``DRT_SPLITK_FENCED=1``, what a runtime falls
  back to when its placement probe fails) gives bit-identical results;
* the fp16 range of the activations: a first-layer norm weight that pushes the
  normalized activation past 65504 raises the range error, one that keeps it
  near 4e4 (checked on the CPU) does not.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import ops as O

from helpers import tiny_geometry

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


def _propose(model, env=None):
    from diffusorrt_amd.runtime import Runtime, bd3_session_config

    env = env or {}
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        rt = Runtime(model, max_forward_rows=256, max_positions=512)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    g = model.geometry
    x = list(range(64)) + [g.mask_token_id] * 32
    try:
        with rt.session(bd3_session_config(32, 8, len(x))) as s:
            s.start_device(x, prompt_len=0, block_size=32, mask_token_id=g.mask_token_id,
                           exact_kv=False, steps=8)
            return s.propose_device(list(range(64, 96)), window_end=96, frozen_prefix=64)
    finally:
        rt.close()


def test_wrong_xcd_count_raises_and_the_gpu_stays_usable():
    from diffusorrt_amd import synthetic as syn

    _say("placement error path: DRT_N_XCC=4 on an 8-XCD part")
    model = syn.build_model(tiny_geometry(), "q4", seed=51)
    with pytest.raises(RuntimeError, match="unexpected XCD"):
        _propose(model, {"DRT_N_XCC": "4"})
    scores, tokens, _ = _propose(model)  # a fresh runtime on the same GPU works
    assert np.isfinite(scores).all() and len(tokens) == 32


def test_fenced_split_k_exchange_is_bit_identical():
    from diffusorrt_amd import synthetic as syn

    _say("fenced split-K exchange")
    model = syn.build_model(tiny_geometry(), "q4", seed=52)
    s0, t0, f0 = _propose(model)
    s1, t1, f1 = _propose(model, {"DRT_SPLITK_FENCED": "1"})
    assert (t1, f1) == (t0, f0)
    assert np.array_equal(np.asarray(s1), np.asarray(s0))


def test_fp16_range_flag():
    from diffusorrt_amd import synthetic as syn

    g = tiny_geometry(layer_count=1)
    ids = list(range(64)) + [g.mask_token_id] * 32

    def with_norm_weight(w):
        model = syn.build_model(g, "q4", seed=53)
        model.weights["model.layers.0.input_layernorm.weight"] = torch.full(
            (g.hidden_size,), w, dtype=torch.bfloat16)
        emb = model.weights["model.embed_tokens.weight"].float().numpy()[ids]
        ones = np.ones(g.hidden_size, np.float32)
        peak = np.abs(O.rms_norm(emb, ones, g.rms_norm_eps)).max() * float(
            torch.tensor(w, dtype=torch.bfloat16).float())
        return model, peak

    near, peak = with_norm_weight(1.0e4)
    _say(f"fp16 range: first-layer activation peak {peak:.3g} (in range)")
    assert 2e4 < peak < 6e4  # the CPU check: near, but inside the fp16 range
    scores, _, _ = _propose(near)
    assert np.isfinite(scores).all()
    over, peak = with_norm_weight(1.0e5)
    _say(f"fp16 range: first-layer activation peak {peak:.3g} (beyond 65504)")
    assert peak > 65504
    with pytest.raises(RuntimeError, match="fp16 range"):
        _propose(over)
