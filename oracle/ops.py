"""Per-op CPU restatement of the reference's hot-path math (oracle; test-only).

All references are to the reference's ``python/src/edllm/`` tree. Arrays are
numpy; "fp32" functions reproduce the reference dtype choreography in float32
and "fp64" variants give the higher-precision truth the tolerances are quoted
against.
"""
from __future__ import annotations

import math

import numpy as np

# ---------------------------------------------------------------------------
# bf16 helpers (the reference's resident weight dtype; numpy has no bf16)
# ---------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as float32.

    This is the conversion MLX's ``astype(bfloat16)`` performs on the casts in
    ``backends/mlx_ops.py:122-127`` (``x.astype(weight.dtype)``) and on every
    bf16 matmul output. NaN stays NaN; overflow rounds to +-inf.
    """
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    rounded = ((u + np.uint64(0x7FFF) + lsb) & np.uint64(0xFFFF0000)).astype(np.uint32)
    out = rounded.view(np.float32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def bf16_bits(x) -> np.ndarray:
    """The uint16 bit patterns of ``bf16_round(x)`` (device upload format)."""
    r = bf16_round(x)
    return (r.view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    """float32 values of uint16 bf16 bit patterns."""
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


# ---------------------------------------------------------------------------
# RMSNorm  (backends/mlx_ops.py:21-35; spec graph/numpyref.py:80-85)
# ---------------------------------------------------------------------------


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """fp32 RMSNorm exactly as ``mlx_ops.rms_norm`` on an fp32 residual stream.

    variance = mean(xf*xf) in fp32; normalized = xf * rsqrt(variance + eps),
    cast back to the input dtype (fp32, a no-op); then ``* weight`` where a bf16
    weight promotes to fp32.
    """
    xf = np.asarray(x, dtype=np.float32)
    variance = np.mean(xf * xf, axis=-1, keepdims=True, dtype=np.float32)
    normalized = xf * (np.float32(1.0) / np.sqrt(variance + np.float32(eps)))
    return (normalized * np.asarray(weight, dtype=np.float32)).astype(np.float32)


def rms_norm64(x, weight, eps: float) -> np.ndarray:
    """float64 truth of the same RMSNorm (``graph/numpyref.py:80-85``)."""
    xf = np.asarray(x, dtype=np.float64)
    variance = np.mean(xf * xf, axis=-1, keepdims=True)
    return xf / np.sqrt(variance + eps) * np.asarray(weight, dtype=np.float64)


# ---------------------------------------------------------------------------
# RoPE  (backends/mlx_forward.py:1566-1595 tables; mlx_ops.py:133-144 apply)
# ---------------------------------------------------------------------------


def rope_tables(positions, head_dim: int, rope_theta: float):
    """fp32 cos/sin tables ``[len(positions), 1, head_dim]`` for absolute positions.

    ``inv_freq = 1 / theta ** (arange(0, half, f32) / half)`` in float32 (a
    Python-float theta keeps float32 under numpy's promotion rules), linear
    scaling factor 1; ``freqs = pos (f32) * inv_freq``; the cos/sin halves are
    duplicated (``mlx_forward.py:1586-1595``). The reference builds rows
    ``0..S-1``; a row subset is the same rows at those positions.
    """
    half = head_dim // 2
    inv_freq = np.float32(1.0) / (
        np.float32(rope_theta) ** (np.arange(0, half, dtype=np.float32) / np.float32(half))
    )
    inv_freq = (inv_freq / np.float32(1.0)).astype(np.float32)
    pos = np.asarray(positions, dtype=np.float32)
    freqs = (pos[:, None] * inv_freq[None, :]).astype(np.float32)
    cos_half = np.cos(freqs)[:, None, :]
    sin_half = np.sin(freqs)[:, None, :]
    return (np.concatenate([cos_half, cos_half], axis=-1).astype(np.float32),
            np.concatenate([sin_half, sin_half], axis=-1).astype(np.float32))


def apply_split_half_rope(x, cos, sin) -> np.ndarray:
    """``x*cos + rotate_half(x)*sin`` in fp32, ``rotate_half(x) = [-x2, x1]``."""
    xf = np.asarray(x, dtype=np.float32)
    half = xf.shape[-1] // 2
    rotated = np.concatenate([-xf[..., half:], xf[..., :half]], axis=-1)
    return (xf * cos + rotated * sin).astype(np.float32)


# ---------------------------------------------------------------------------
# SwiGLU  (backends/mlx_ops.py:147-154)
# ---------------------------------------------------------------------------


def swiglu(gate, up) -> np.ndarray:
    """``g * sigmoid(g) * u`` in fp32."""
    g = np.asarray(gate, dtype=np.float32)
    u = np.asarray(up, dtype=np.float32)
    sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return (g * sig * u).astype(np.float32)


# ---------------------------------------------------------------------------
# 4-bit affine group quantization, MLX packing
#   (backends/mlx_ops.py:43-60 QuantizedWeight, :113-121 quantized_matmul)
# ---------------------------------------------------------------------------

Q4_GROUP = 64


def q4_unpack(w_q) -> np.ndarray:
    """uint32 ``[N, K/8]`` -> uint8 nibbles ``[N, K]``.

    MLX packing: word ``j`` of row ``n`` holds ``k = 8j .. 8j+7``, nibble ``i``
    (bits ``4i .. 4i+3``, low nibble first) is ``k = 8j + i``.
    """
    w = np.asarray(w_q, dtype=np.uint32)
    n, words = w.shape
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))
    nib = (w[:, :, None] >> shifts[None, None, :]) & np.uint32(0xF)
    return nib.reshape(n, words * 8).astype(np.uint8)


def q4_pack(nibbles) -> np.ndarray:
    """Inverse of :func:`q4_unpack`: uint8 ``[N, K]`` (values 0..15) -> uint32."""
    q = np.asarray(nibbles, dtype=np.uint32)
    n, k = q.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    q = q.reshape(n, k // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))
    return np.bitwise_or.reduce(q << shifts[None, None, :], axis=2).astype(np.uint32)


def q4_dequant(w_q, scales, biases, *, dtype=np.float32) -> np.ndarray:
    """``W[n, k] = scale[n, k//64] * q[n, k] + bias[n, k//64]`` ([N, K]).

    ``scales``/``biases`` are float values of the resident bf16 tensors. In
    float32 the product ``scale*q`` is exact (8-bit mantissa times a 4-bit
    integer) so the only rounding is the final add, fused or not.
    """
    q = q4_unpack(w_q).astype(dtype)
    n, k = q.shape
    s = np.repeat(np.asarray(scales, dtype=dtype), Q4_GROUP, axis=1)[:, :k]
    b = np.repeat(np.asarray(biases, dtype=dtype), Q4_GROUP, axis=1)[:, :k]
    return (s * q + b).astype(dtype)


def round_half_away(x) -> np.ndarray:
    """float32 round to nearest, halves away from zero (C ``roundf``; Metal's
    ``round``). ``x - trunc(x)`` is exact in float32, so no addition can
    round a value just below a half up to it."""
    a = np.asarray(x, dtype=np.float32)
    t = np.trunc(a)
    frac = a - t
    step = np.where(np.abs(frac) >= np.float32(0.5), np.sign(a), np.float32(0)).astype(np.float32)
    return (t + step).astype(np.float32)


def q4_quantize(w, *, return_fp32: bool = False):
    """4-bit affine group-64 quantization: ``mx.quantize(w, group_size=64, bits=4)``
    as ``quantize_linear_weight`` calls it (``backends/mlx_ops.py:63-94``) on the
    resident bf16 weight (``backends/mlx_dream.py:1957-1963, 2073-2108``).

    MLX (``mlx>=0.31,<0.32``, absent here) is restated from its published affine
    quantization, per group of 64 along K, in float32:
      ``scale = max((w_max - w_min) / 15, 1e-7)``; the edge is ``w_min`` (scale
      positive) when ``|w_min| > |w_max|``, else ``w_max`` (scale negated);
      ``q0 = round(edge / scale)``; unless ``q0 == 0``: ``scale = edge / q0`` and
      ``bias = edge``, else ``bias = 0``;
      ``q = clip(round((w - bias) / scale), 0, 15)``;
    scales/biases stored as bf16 (round to nearest even). ``round`` is taken as
    halves away from zero (the Metal kernel's); MLX's CPU fallback rounds halves
    to even, so an exact .5 quotient is where the two can differ.

    Returns ``(w_q uint32 [N, K/8], scales, biases)`` (float32 values of bf16);
    with ``return_fp32`` also the float32 scale and bias before the bf16 store.
    """
    a = bf16_round(np.asarray(w, dtype=np.float32))
    n, k = a.shape
    if k % Q4_GROUP:
        raise ValueError(f"in-dim {k} not divisible by {Q4_GROUP}")
    g = a.reshape(n, k // Q4_GROUP, Q4_GROUP)
    f32 = np.float32
    w_max = g.max(axis=-1)
    w_min = g.min(axis=-1)
    scale = np.maximum((w_max - w_min) / f32(15), f32(1e-7)).astype(f32)
    side = np.abs(w_min) > np.abs(w_max)
    scale = np.where(side, scale, -scale).astype(f32)
    edge = np.where(side, w_min, w_max).astype(f32)
    q0 = round_half_away(edge / scale)
    at_zero = q0 == 0
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(at_zero, scale, edge / q0).astype(f32)
    bias = np.where(at_zero, f32(0), edge).astype(f32)
    q = round_half_away((g - bias[..., None]) / scale[..., None])
    q = np.clip(q, f32(0), f32(15)).astype(np.uint8).reshape(n, k)
    out = (q4_pack(q), bf16_round(scale), bf16_round(bias))
    return out + (scale, bias) if return_fp32 else out


class Q4Weight:
    """A q4 g64 linear weight: packed words + float scales/biases (bf16 values).

    Mirrors ``QuantizedWeight`` (``backends/mlx_ops.py:43-60``); ``shape`` is the
    logical ``(out, in)``.
    """

    def __init__(self, w_q, scales, biases):
        self.w_q = np.asarray(w_q, dtype=np.uint32)
        self.scales = np.asarray(scales, dtype=np.float32)
        self.biases = np.asarray(biases, dtype=np.float32)
        self.shape = (self.w_q.shape[0], self.w_q.shape[1] * 8)
        self._dense32 = None

    def dense(self) -> np.ndarray:
        if self._dense32 is None:
            self._dense32 = q4_dequant(self.w_q, self.scales, self.biases)
        return self._dense32


# ---------------------------------------------------------------------------
# linear  (backends/mlx_ops.py:97-130)
# ---------------------------------------------------------------------------


def linear(x, weight, bias=None, *, weight_kind: str) -> np.ndarray:
    """``x @ W.T (+ bias)`` with the reference's dtype choreography.

    * ``weight_kind="q4"``: ``mx.quantized_matmul`` on an fp32 activation; the
      output dtype follows x (fp32) (``mlx_ops.py:113-121``).
    * ``weight_kind="bf16"``: ``(x.astype(bf16) @ W.T).astype(fp32)`` -- the input
      is rounded to bf16 and so is the matmul's bf16 output (``:122-125``).
    * ``weight_kind="fp32"``: plain fp32 matmul (``:126-127``).

    The bias is added in the output dtype (``:128-129``).
    """
    xf = np.asarray(x, dtype=np.float32)
    if weight_kind == "q4":
        y = xf @ weight.dense().T
    elif weight_kind == "bf16":
        y = bf16_round(bf16_round(xf) @ np.asarray(weight, dtype=np.float32).T)
    elif weight_kind == "fp32":
        y = xf @ np.asarray(weight, dtype=np.float32).T
    else:
        raise ValueError(f"unknown weight kind {weight_kind!r}")
    y = y.astype(np.float32)
    if bias is not None:
        y = (y + np.asarray(bias, dtype=np.float32)).astype(np.float32)
    return y


def q4_linear64(x, w: Q4Weight) -> np.ndarray:
    """float64 truth of a q4 linear on the given activation values."""
    dense = q4_dequant(w.w_q, w.scales, w.biases, dtype=np.float64)
    return np.asarray(x, dtype=np.float64) @ dense.T


# ---------------------------------------------------------------------------
# d2f_hybrid attention mask  (backends/mlx_ops.py:191-224, :227-288;
# staircase form model_coverage/reference.py:158-180)
# ---------------------------------------------------------------------------


def effective_block(positions, *, prompt_len: int, block_size: int) -> np.ndarray:
    """``eff(p) = -1 if p < prompt_len else (p - prompt_len) // block_size``."""
    p = np.asarray(positions, dtype=np.int64)
    return np.where(p < prompt_len, np.int64(-1), (p - prompt_len) // block_size)


def d2f_visible(q_positions, kv_len: int, *, prompt_len: int, block_size: int) -> np.ndarray:
    """Boolean ``[len(q_positions), kv_len]``: visible iff ``eff(col) <= eff(row)``."""
    cols = effective_block(np.arange(kv_len), prompt_len=prompt_len, block_size=block_size)
    rows = effective_block(q_positions, prompt_len=prompt_len, block_size=block_size)
    return cols[None, :] <= rows[:, None]


# ---------------------------------------------------------------------------
# GQA scaled-dot-product attention  (backends/mlx_ops.py:347-443)
# ---------------------------------------------------------------------------


def attention(q, k, v, *, visible=None, dtype=np.float64) -> np.ndarray:
    """Masked GQA SDPA: q ``[rq, Hq, hd]``, k/v ``[rk, Hkv, hd]`` -> ``[rq, Hq*hd]``.

    Query head ``h`` reads compact K/V head ``h // (Hq // Hkv)``; scale
    ``1/sqrt(hd)``; ``visible`` (bool ``[rq, rk]``) applies the additive 0/-inf
    bias; ``None`` is the bidirectional kind (no mask). The reference promotes
    q/k/v to fp32 and runs MLX's fused SDPA; this restatement computes in
    ``dtype`` (float64 truth by default).
    """
    qf = np.asarray(q, dtype=dtype)
    kf = np.asarray(k, dtype=dtype)
    vf = np.asarray(v, dtype=dtype)
    rq, hq, hd = qf.shape
    rk, hkv, _ = kf.shape
    group = hq // hkv
    scale = dtype(1.0 / math.sqrt(hd))
    out = np.empty((rq, hq, hd), dtype=dtype)
    for h in range(hq):
        kh = kf[:, h // group, :]
        vh = vf[:, h // group, :]
        s = (qf[:, h, :] @ kh.T) * scale
        if visible is not None:
            s = np.where(visible, s, -np.inf)
        m = np.max(s, axis=-1, keepdims=True)
        p = np.exp(s - m)
        p /= np.sum(p, axis=-1, keepdims=True)
        out[:, h, :] = p @ vh
    return out.reshape(rq, hq * hd)


# ---------------------------------------------------------------------------
# Dream logits convention  (backends/mlx_d2f_forward.py:74-93; mlx_ops.py:157-159)
# ---------------------------------------------------------------------------


def required_raw_row(position: int, *, logits_convention: str) -> int:
    """``dream_ar_shift``: row p reads raw row p-1 (row 0 reads 0); ``raw``: p."""
    if logits_convention == "dream_ar_shift":
        return position - 1 if position >= 1 else 0
    if logits_convention == "raw":
        return position
    raise ValueError(f"unknown logits_convention: {logits_convention!r}")


# ---------------------------------------------------------------------------
# Scoring  (backends/diffusion_runtime.py:179-192, :290-299, :203-253)
# ---------------------------------------------------------------------------


def raw_max_prob(logits):
    """float64 softmax per row, then (max probability, first argmax).

    ``probs = exp(l - max) / sum``; ``max_prob = probs.max()``;
    ``argmax`` keeps the lowest index among equal maxima (``np.argmax``).
    """
    probs = np.array(logits, dtype=np.float64, copy=True)
    probs -= np.max(probs, axis=-1, keepdims=True)
    np.exp(probs, out=probs)
    probs /= np.sum(probs, axis=-1, keepdims=True)
    return probs.max(axis=-1), probs.argmax(axis=-1).tolist()


def topk_count_choices(confidence, transfer_count: int) -> list:
    """``np.argsort(-confidence)[:transfer_count]`` (numpy's default quicksort)."""
    chosen = np.argsort(-np.asarray(confidence))[:transfer_count]
    return [int(i) for i in chosen]


SAMPLING_STEP = 0x9E3779B97F4A7C15
MASK64 = (1 << 64) - 1


def mix64(value: int) -> int:
    """splitmix64's finalizer on a Python int (mod 2**64)."""
    z = value & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def sampling_uniform_bits(seed: int, step: int, position: int, token: int) -> int:
    """The 64-bit counter hash keyed by (seed, forward, position, token).

    ``key = mix(seed + G)``; ``key = mix(key + (step+1) G)``;
    ``key = mix(key + (position+1) G)``; ``bits = mix(key + (token+1) G)``
    (``backends/diffusion_runtime.py:203-253``).

    Pinned by ``tests/golden/sampling_vectors.json``: noise rows and sampled
    tokens/scores written by the reference's own ``sampling_noise`` and
    ``_sampled_max_prob_confidence`` (``tests/golden/make_sampling_vectors.py``),
    matched bit for bit; ``mix64`` also by the published splitmix64 sequence.
    """
    g = SAMPLING_STEP
    key = mix64((seed & MASK64) + g)
    key = mix64(key + ((step + 1) & MASK64) * g)
    key = mix64(key + ((position + 1) & MASK64) * g)
    return mix64(key + (token + 1) * g)


def sampling_noise(seed: int, step: int, position: int, vocab: int) -> np.ndarray:
    """Gumbel noise ``-log(-log u)`` (float32) for one row; u from 23 hash bits."""
    toks = np.arange(vocab, dtype=np.int64)
    bits = np.array([sampling_uniform_bits(seed, step, position, int(t)) >> 41 for t in toks],
                    dtype=np.float32)
    u = (bits + np.float32(0.5)) * np.float32(2.0 ** -23)
    return -np.log(-np.log(u))


def sampled_max_prob(logits, *, temperature: float, seed: int, step: int, positions):
    """Sampled token ``argmax(l + T*g)`` and its raw float64 probability.

    (``backends/diffusion_runtime.py:256-275``.)
    """
    rows = np.asarray(logits, dtype=np.float32)
    scores = np.empty(rows.shape[0], dtype=np.float64)
    tokens = []
    for r, pos in enumerate(positions):
        values = rows[r].astype(np.float64)
        noise = sampling_noise(seed, step, int(pos), rows.shape[1]).astype(np.float64)
        token = int(np.argmax(values + float(temperature) * noise))
        top = values.max()
        w = np.exp(values - top)
        scores[r] = w[token] / w.sum()
        tokens.append(token)
    return scores, tokens
