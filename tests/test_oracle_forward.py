"""Pins the oracle's full-context forward (CPU only).

Checks: a second implementation of the decoder written with torch's CPU
kernels (rms_norm, scaled_dot_product_attention with a boolean mask, silu) and
its own q4 dequantisation; the BD3 staircase invariants (rows never see later
blocks, so a longer canvas leaves earlier rows unchanged); the Dream logits
shift; the bf16 choreography against torch's bf16 matmul.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from diffusorrt_amd import synthetic as syn
from oracle import forward as F
from oracle import ops as O
from helpers import oracle_weights, tiny_dream_geometry, tiny_geometry


def _torch_q4_dense(w_q, scales, biases):
    words = torch.from_numpy(np.asarray(w_q, dtype=np.uint32).astype(np.int64))
    shifts = torch.arange(8, dtype=torch.int64) * 4
    q = ((words[:, :, None] >> shifts) & 15).reshape(words.shape[0], -1).to(torch.float64)
    s = torch.from_numpy(np.asarray(scales, np.float32)).to(torch.float64)
    b = torch.from_numpy(np.asarray(biases, np.float32)).to(torch.float64)
    s = s.repeat_interleave(64, dim=1)
    b = b.repeat_interleave(64, dim=1)
    return (s * q + b).to(torch.float32)


def _torch_forward(model, g, ids, visible, kind):
    """Independent decoder forward with torch CPU ops (fp32; bf16 matmuls for bf16)."""
    raw = syn.to_oracle_weights(model)

    def W(key):
        v = raw[key]
        return _torch_q4_dense(*v) if isinstance(v, tuple) else torch.from_numpy(np.asarray(v))

    def lin(x, key, bias_key=None):
        w = W(key)
        if kind == "bf16":
            y = (x.bfloat16() @ w.bfloat16().T).float()
        else:
            y = x @ w.T
        if bias_key is not None and bias_key in raw:
            y = y + torch.from_numpy(np.asarray(raw[bias_key], np.float32))
        return y

    s = len(ids)
    hd, hq, hkv = g.head_dim, g.num_heads, g.num_kv_heads
    h = torch.from_numpy(np.asarray(raw["model.embed_tokens.weight"], np.float32))[ids]
    pos = torch.arange(s, dtype=torch.float64)
    inv = 1.0 / (g.rope_theta ** (torch.arange(0, hd // 2, dtype=torch.float64) / (hd // 2)))
    ang = pos[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1).float()[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1).float()[:, None, :]

    def rope(x):
        x1, x2 = x[..., : hd // 2], x[..., hd // 2:]
        return x * cos + torch.cat([-x2, x1], -1) * sin

    mask = None if visible is None else torch.from_numpy(visible)
    for i in range(g.layer_count):
        p = f"model.layers.{i}."
        n = torch.nn.functional.rms_norm(h, (g.hidden_size,), W(p + "input_layernorm.weight"),
                                         eps=g.rms_norm_eps)
        q = lin(n, p + "self_attn.q_proj.weight", p + "self_attn.q_proj.bias").view(s, hq, hd)
        k = lin(n, p + "self_attn.k_proj.weight", p + "self_attn.k_proj.bias").view(s, hkv, hd)
        v = lin(n, p + "self_attn.v_proj.weight", p + "self_attn.v_proj.bias").view(s, hkv, hd)
        if g.qk_norm:
            q = torch.nn.functional.rms_norm(q, (hd,), W(p + "self_attn.q_norm.weight"),
                                             eps=g.rms_norm_eps)
            k = torch.nn.functional.rms_norm(k, (hd,), W(p + "self_attn.k_norm.weight"),
                                             eps=g.rms_norm_eps)
        q, k = rope(q), rope(k)
        rep = hq // hkv
        kk = k.repeat_interleave(rep, dim=1).transpose(0, 1)
        vv = v.repeat_interleave(rep, dim=1).transpose(0, 1)
        a = torch.nn.functional.scaled_dot_product_attention(q.transpose(0, 1), kk, vv,
                                                             attn_mask=mask)
        h = h + lin(a.transpose(0, 1).reshape(s, hq * hd), p + "self_attn.o_proj.weight")
        n2 = torch.nn.functional.rms_norm(h, (g.hidden_size,),
                                          W(p + "post_attention_layernorm.weight"),
                                          eps=g.rms_norm_eps)
        act = torch.nn.functional.silu(lin(n2, p + "mlp.gate_proj.weight")) * \
            lin(n2, p + "mlp.up_proj.weight")
        h = h + lin(act, p + "mlp.down_proj.weight")
    hn = torch.nn.functional.rms_norm(h, (g.hidden_size,), W("model.norm.weight"),
                                      eps=g.rms_norm_eps)
    return lin(hn, "lm_head.weight").numpy()


@pytest.mark.parametrize("kind,tol", [("q4", 2e-4), ("bf16", 3e-2)])
def test_forward_matches_independent_torch_decoder(kind, tol):
    g = tiny_geometry()
    model = syn.build_model(g, kind, seed=11)
    ids = syn.prompt_ids(11, 70, high=1000)
    cfg = syn.oracle_config(g, kind)
    got = F.forward_full(oracle_weights(model), cfg, ids, mask_kind="d2f_hybrid",
                         mask_geometry=(0, 32))
    vis = O.d2f_visible(np.arange(70), 70, prompt_len=0, block_size=32)
    ref = _torch_forward(model, g, ids, vis, kind)
    err = np.abs(got - ref).max(axis=-1) / np.abs(ref).max(axis=-1)
    assert err.max() < tol, err.max()


def test_dream_forward_matches_independent_torch_decoder():
    g = tiny_dream_geometry()
    model = syn.build_model(g, "q4", seed=12)
    ids = syn.prompt_ids(12, 48, high=1000)
    got = F.forward_full(oracle_weights(model), syn.oracle_config(g, "q4"), ids,
                         mask_kind="bidirectional")
    ref = _torch_forward(model, g, ids, None, "q4")
    err = np.abs(got - ref).max(axis=-1) / np.abs(ref).max(axis=-1)
    assert err.max() < 2e-4, err.max()


def test_staircase_rows_never_see_later_blocks():
    g = tiny_geometry()
    model = syn.build_model(g, "q4", seed=13)
    W = oracle_weights(model)
    cfg = syn.oracle_config(g, "q4")
    ids = syn.prompt_ids(13, 96, high=1000)
    base = F.forward_full(W, cfg, ids, mask_kind="d2f_hybrid", mask_geometry=(0, 32))
    # change every token of the last block: rows of blocks 0 and 1 are untouched
    ids2 = list(ids[:64]) + [g.mask_token_id] * 32
    alt = F.forward_full(W, cfg, ids2, mask_kind="d2f_hybrid", mask_geometry=(0, 32))
    np.testing.assert_array_equal(base[:64], alt[:64])
    assert not np.allclose(base[64:], alt[64:])
    # a shorter canvas ending at a block boundary gives the same rows
    short = F.forward_full(W, cfg, ids[:64], mask_kind="d2f_hybrid", mask_geometry=(0, 32))
    np.testing.assert_allclose(short, base[:64], rtol=1e-5, atol=1e-5)
    # inside a block attention is bidirectional: a later in-block token matters
    ids3 = list(ids)
    ids3[70] = (ids3[70] + 1) % 1000
    alt3 = F.forward_full(W, cfg, ids3, mask_kind="d2f_hybrid", mask_geometry=(0, 32))
    assert not np.allclose(base[64], alt3[64])


def test_window_logits_dream_shift_reads_previous_row():
    g = tiny_dream_geometry()
    model = syn.build_model(g, "q4", seed=14)
    W = oracle_weights(model)
    cfg = syn.oracle_config(g, "q4")
    ids = syn.prompt_ids(14, 40, high=1000)
    full = F.forward_full(W, cfg, ids, mask_kind="bidirectional")
    scope = [0, 1, 5, 39]
    win = F.window_logits(W, cfg, ids, scope, mask_kind="bidirectional", mask_geometry=None,
                          logits_convention="dream_ar_shift")
    np.testing.assert_allclose(win, full[[0, 0, 4, 38]], rtol=1e-6, atol=1e-6)
    raw = F.window_logits(W, cfg, ids, scope, mask_kind="bidirectional", mask_geometry=None,
                          logits_convention="raw")
    np.testing.assert_allclose(raw, full[scope], rtol=1e-6, atol=1e-6)


def test_kv_hook_sees_roped_keys():
    """The K/V a cache would store are post-norm, post-RoPE keys and raw values."""
    g = tiny_geometry(layer_count=1)
    model = syn.build_model(g, "q4", seed=15)
    W = oracle_weights(model)
    cfg = syn.oracle_config(g, "q4")
    ids = syn.prompt_ids(15, 8, high=1000)
    seen = {}
    F.forward_full(W, cfg, ids, mask_kind="d2f_hybrid", mask_geometry=(0, 32),
                   kv_hook=lambda i, k, v: seen.update(k=k, v=v))
    # position 0 has an identity rotation; the per-head key norm gives unit RMS
    k0 = seen["k"][0].astype(np.float64)
    np.testing.assert_allclose(np.sqrt((k0 ** 2).mean(axis=-1)), 1.0, rtol=1e-4)
    assert seen["v"].shape == (8, g.num_kv_heads, g.head_dim)


@pytest.mark.parametrize("seed", [21, 22])
def test_operand_precision_sites(seed):
    """Per-site attribution of the device path's operand precision at the BD3
    layer shapes (2 layers, all 128 rows of a 96-token prompt + one masked
    block), measured as the largest shift of the margins between the top token
    and the next seven:
      * fp16 rounding of every operand site (the linears' inputs, Q, K/V and the
        LM head's input) shifts them by more than the 1e-3 tie bar: a device
        path with plain fp16 operands could not meet it;
      * the fp16 hi + lo pairs the device carries for those sites (x as fp16(x)
        + fp16(x - fp16(x))) shift them by < 2e-5, far inside the bar;
      * fp16 storage of the cached K/V alone, the one site that stays, shifts
        them by < 2e-3 but > 1e-4: the GPU tests hold the device to the 1e-3
        bar against the oracle run with that rounding (``kv_round``) and
        attribute the remaining disagreements with the exact oracle to it."""
    import dataclasses

    from helpers import NEAR_TIE_REL, kv_round_f16

    geom = dataclasses.replace(syn.BD3_QWEN3_06B, layer_count=2, vocab_size=4096,
                               mask_token_id=4000, eos_token_id=4001)
    model = syn.build_model(geom, "q4", seed)
    W, cfg = oracle_weights(model), syn.oracle_config(geom, "q4")
    x = np.random.default_rng(5).integers(0, 3900, 96).tolist() + [4000] * 32

    def r16(a):
        return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)

    def hilo(a):
        a = np.asarray(a, np.float32)
        hi = a.astype(np.float16).astype(np.float32)
        return hi + (a - hi).astype(np.float16).astype(np.float32)

    def run(**kw):
        return F.forward_full(W, cfg, x, mask_kind="d2f_hybrid", mask_geometry=(0, 32),
                              **kw).astype(np.float64)

    ref = run()
    order = np.argsort(-ref, axis=-1)[:, :8]
    rows = np.arange(ref.shape[0])
    top = order[:, 0]

    def shift(got):
        return max(np.abs((got[rows, order[:, j]] - got[rows, top]) -
                          (ref[rows, order[:, j]] - ref[rows, top])).max() for j in range(1, 8))

    all_f16 = shift(run(operand_round=r16))
    pairs = shift(run(operand_round=hilo, kv_round=lambda a: a))
    kv_only = shift(run(kv_round=kv_round_f16))
    assert all_f16 > NEAR_TIE_REL, all_f16
    assert 0 < pairs < 2e-5, pairs
    assert 1e-4 < kv_only < 2e-3, kv_only
    # a planted coarser cache (bf16 storage) is not what the bar is measured on
    bf16_kv = shift(run(kv_round=lambda a: O.bf16_round(np.asarray(a, np.float32))))
    assert bf16_kv > 2 * kv_only


@pytest.mark.parametrize("kind,mask", [("q4", "d2f_hybrid"), ("bf16", "bidirectional")])
def test_last_layer_output_rows_shortcut(kind, mask):
    """The long-canvas shortcut (the last layer computes only the LM rows) gives
    the full forward's logits for those rows, in the requested order."""
    g = tiny_geometry(layer_count=2)
    model = syn.build_model(g, kind, seed=31)
    W, cfg = oracle_weights(model), syn.oracle_config(g, kind)
    ids = syn.prompt_ids(31, 70, high=1000)
    rows = [69, 3, 40, 3]
    geom = (0, 32) if mask == "d2f_hybrid" else None
    full = F.forward_full(W, cfg, ids, mask_kind=mask, mask_geometry=geom, output_rows=rows)
    fast = F.forward_full(W, cfg, ids, mask_kind=mask, mask_geometry=geom, output_rows=rows,
                          last_layer_output_rows_only=True)
    np.testing.assert_allclose(fast, full, rtol=1e-5, atol=1e-5)
