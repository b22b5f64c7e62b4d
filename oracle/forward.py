"""Full-context transformer forward, restated on the CPU (oracle; test-only).

Restates the full-context branch of ``_forward_full_logits_from_weights``
(``backends/mlx_forward.py:235-636``) with ``_transformer_layer_forward``
(``:1164-1309``), ``_project_kv_rows`` (``:1312-1361``), ``_embedding_rows``
(``:1538-1557``) and ``_rope_tables`` (``:1566-1595``). Every visible row is
recomputed every call, as the reference does each denoise step; the LM head runs
only on ``output_rows`` (``:578-601``).

``weights`` is a dict keyed by the reference's package weight names
(``model.layers.{i}.self_attn.q_proj.weight`` ...). A linear weight is either a
float32 array holding bf16 values (``weight_kind="bf16"``) or an
:class:`oracle.ops.Q4Weight` (``weight_kind="q4"``).
"""
from __future__ import annotations

import numpy as np

from . import ops


def _lin(weights, key, x, kind):
    w = weights[key + ".weight"]
    b = weights.get(key + ".bias")
    return ops.linear(x, w, b, weight_kind=kind)


def _keep(x):
    return x


def layer_forward(weights, cfg, i, hidden, cos, sin, visible, kv_hook=None, operand_round=None,
                  kv_round=None, query_rows=None):
    """One decoder layer over all rows of ``hidden`` (fp32 ``[S, d]``).

    ``h += o(attn(rope(qnorm(q(n))), rope(knorm(k(n))), v(n)))`` with
    ``n = rmsnorm(h)``, then ``h += down(swiglu(gate(n2), up(n2)))`` with
    ``n2 = rmsnorm(h)`` (``mlx_forward.py:1164-1309``; op order fixed by
    ``graph/ir.py:106``).

    ``operand_round`` (a precision model, not reference semantics) is applied to
    every tensor that a lower-precision device path stores in its operand type:
    the linears' inputs (n, attention output, n2, swiglu output), Q, and the
    cached K/V. ``kv_round`` (also a precision model) rounds only the K and V
    that a prefix cache stores (e.g. to fp16): the reference computation with
    the cache's storage type. ``None`` for both is the reference computation.

    ``query_rows`` (optional, sorted row indices): only these rows' outputs are
    computed and returned; the K/V still come from every row. Row outputs are
    independent, so this gives the same values for those rows as a full layer
    (up to float32 summation order in the row-subset matmuls).
    """
    rnd = operand_round or _keep
    kv_rnd = kv_round or rnd
    kind = cfg["weight_kind"]
    eps = cfg["eps"]
    hq, hkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    p = f"model.layers.{i}."
    s = hidden.shape[0]
    n = rnd(ops.rms_norm(hidden, weights[p + "input_layernorm.weight"], eps))
    qr = slice(None) if query_rows is None else np.asarray(query_rows, dtype=np.int64)
    q = _lin(weights, p + "self_attn.q_proj", n[qr], kind).reshape(-1, hq, hd)
    if cfg["qk_norm"]:
        q = ops.rms_norm(q, weights[p + "self_attn.q_norm.weight"], eps)
    q = rnd(ops.apply_split_half_rope(q, cos[qr], sin[qr]))
    k = _lin(weights, p + "self_attn.k_proj", n, kind).reshape(s, hkv, hd)
    v = kv_rnd(_lin(weights, p + "self_attn.v_proj", n, kind).reshape(s, hkv, hd))
    if cfg["qk_norm"]:
        k = ops.rms_norm(k, weights[p + "self_attn.k_norm.weight"], eps)
    k = kv_rnd(ops.apply_split_half_rope(k, cos, sin))
    if kv_hook is not None:
        kv_hook(i, k, v)
    vis = None if visible is None else visible[qr]
    attn = rnd(ops.attention(q, k, v, visible=vis, dtype=np.float32).astype(np.float32))
    hidden = (hidden[qr] + _lin(weights, p + "self_attn.o_proj", attn, kind)).astype(np.float32)
    n2 = rnd(ops.rms_norm(hidden, weights[p + "post_attention_layernorm.weight"], eps))
    gate = _lin(weights, p + "mlp.gate_proj", n2, kind)
    up = _lin(weights, p + "mlp.up_proj", n2, kind)
    mlp = _lin(weights, p + "mlp.down_proj", rnd(ops.swiglu(gate, up)), kind)
    return (hidden + mlp).astype(np.float32)


def forward_full(weights, cfg, token_ids, *, mask_kind, mask_geometry=None,
                 output_rows=None, n_layers=None, kv_hook=None, operand_round=None,
                 kv_round=None, last_layer_output_rows_only=False):
    """Raw fp32 logits for ``output_rows`` (default: every row) of ``token_ids``.

    ``mask_kind`` is ``"d2f_hybrid"`` (``mask_geometry = (prompt_len,
    block_size)``; BD3 uses origin 0) or ``"bidirectional"`` (Dream, no mask).
    ``n_layers`` limits the layer count (the CPU baseline's bounded sample).
    ``operand_round``: see :func:`layer_forward`; also applied to the final
    norm's output (the LM head's input). ``kv_round``: see :func:`layer_forward`.
    ``last_layer_output_rows_only``: the last layer computes only the rows the LM
    head reads (a shortcut for long canvases; see ``query_rows``).
    """
    ids = np.asarray(token_ids, dtype=np.int64)
    s = ids.shape[0]
    emb = weights["model.embed_tokens.weight"]
    hidden = np.asarray(emb[ids], dtype=np.float32)
    cos, sin = ops.rope_tables(np.arange(s), cfg["head_dim"], cfg["rope_theta"])
    if mask_kind == "d2f_hybrid":
        prompt_len, block_size = mask_geometry
        visible = ops.d2f_visible(np.arange(s), s, prompt_len=prompt_len,
                                  block_size=block_size)
    elif mask_kind == "bidirectional":
        visible = None
    else:
        raise ValueError(f"unsupported mask kind {mask_kind!r}")
    layers = cfg["n_layers"] if n_layers is None else n_layers
    rows = list(range(s)) if output_rows is None else [int(r) for r in output_rows]
    kept = sorted(set(rows))
    for i in range(layers):
        only = last_layer_output_rows_only and i == layers - 1
        hidden = layer_forward(weights, cfg, i, hidden, cos, sin, visible, kv_hook, operand_round,
                               kv_round, query_rows=kept if only else None)
    if last_layer_output_rows_only and layers > 0:
        h = hidden[[kept.index(r) for r in rows]]
    else:
        h = hidden[rows]
    h = (operand_round or _keep)(ops.rms_norm(h, weights["model.norm.weight"], cfg["eps"]))
    logits = ops.linear(h, weights["lm_head.weight"], None, weight_kind=cfg["weight_kind"])
    return logits.astype(np.float32)


def window_logits(weights, cfg, token_ids, scope, *, mask_kind, mask_geometry,
                  logits_convention, operand_round=None, kv_round=None,
                  last_layer_output_rows_only=False):
    """Convention-applied logits for ``scope`` positions (``execute_window``).

    Raw row selection per ``_required_raw_row`` (``mlx_d2f_forward.py:74-93``);
    rows are returned in ``scope`` order (``backend_runner.py:385-390``).
    """
    raw_rows = [ops.required_raw_row(int(p), logits_convention=logits_convention)
                for p in scope]
    uniq = sorted(set(raw_rows))
    logits = forward_full(weights, cfg, token_ids, mask_kind=mask_kind,
                          mask_geometry=mask_geometry, output_rows=uniq,
                          operand_round=operand_round, kv_round=kv_round,
                          last_layer_output_rows_only=last_layer_output_rows_only)
    index = {r: j for j, r in enumerate(uniq)}
    return logits[[index[r] for r in raw_rows]]
