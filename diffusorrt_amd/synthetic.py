"""Seeded synthetic models and inputs for the denoise-step workloads.

There is no network for checkpoints, so every workload runs on random-init
weights generated deterministically on the CPU from a seed (``torch.Generator``,
the same stream on every machine with this torch build), then uploaded.

Geometry constants follow the reference's model contracts
(``backends/cuda_profile.py:63-74, 151-162``; ``model_definitions.py:418-448,
1140-1200``).

Weight choices (the reference ships no synthetic recipe):
  * bf16 weights: every linear and the embedding ~ N(0, 0.02) rounded to bf16;
    RMSNorm weights are 1 (the usual init); BD3 ties ``lm_head`` to the
    embedding (the package stores both keys with equal content).
  * q4 weights (MLX affine g64 packing): nibbles uniform in 0..15 (random
    uint32 words), per-group scale ~ U(0.003, 0.006) and bias
    ``-7.5*scale + U(-0.002, 0.002)``, both rounded to bf16, so dequantized
    weights are centred with std ~0.02. ``lm_head`` is quantized too
    (``backends/mlx_dream.py:2082-2084``) and is generated independently of
    the (bf16, never quantized) embedding.
  * Dream q/k/v biases ~ N(0, 0.02) bf16.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

Q4_GROUP = 64


@dataclass(frozen=True)
class ModelGeometry:
    """Model-lifetime geometry (mirrors ``abi/lifetimes.py:46-55`` plus the
    per-architecture flags the forward needs)."""

    name: str
    layer_count: int
    hidden_size: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float
    qk_norm: bool
    qkv_bias: bool
    logits_convention: str
    mask_token_id: int
    eos_token_id: int
    tie_word_embeddings: bool
    max_position_embeddings: int = 40960
    # linear RoPE scaling: positions are divided by this factor
    # (backends/mlx_forward.py:1584-1588)
    rope_scaling_factor: float = 1.0

    def scaled(self, **overrides) -> "ModelGeometry":
        values = dict(self.__dict__)
        values.update(overrides)
        return ModelGeometry(**values)


# Qwen3-0.6B BD3LM (backends/cuda_profile.py:151-162; model_definitions.py:1179-1200)
BD3_QWEN3_06B = ModelGeometry(
    name="bd3lm-qwen3-0.6b", layer_count=28, hidden_size=1024, num_heads=16,
    num_kv_heads=8, head_dim=128, intermediate_size=3072, vocab_size=151936,
    rms_norm_eps=1e-6, rope_theta=1e6, qk_norm=True, qkv_bias=False,
    logits_convention="raw", mask_token_id=151669, eos_token_id=151645,
    tie_word_embeddings=True)

# Dream on Qwen2.5-7B (backends/cuda_profile.py:63-74; model_definitions.py:1140-1157)
DREAM_QWEN25_7B = ModelGeometry(
    name="dream-qwen2.5-7b", layer_count=28, hidden_size=3584, num_heads=28,
    num_kv_heads=4, head_dim=128, intermediate_size=18944, vocab_size=152064,
    rms_norm_eps=1e-6, rope_theta=1e6, qk_norm=False, qkv_bias=True,
    logits_convention="dream_ar_shift", mask_token_id=151666, eos_token_id=151643,
    tie_word_embeddings=False, max_position_embeddings=131072)

LINEAR_SUFFIXES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                   "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


def linear_shapes(g: ModelGeometry) -> dict:
    """``(out, in)`` of each per-layer linear."""
    d, hd = g.hidden_size, g.head_dim
    return {
        "self_attn.q_proj": (g.num_heads * hd, d),
        "self_attn.k_proj": (g.num_kv_heads * hd, d),
        "self_attn.v_proj": (g.num_kv_heads * hd, d),
        "self_attn.o_proj": (d, g.num_heads * hd),
        "mlp.gate_proj": (g.intermediate_size, d),
        "mlp.up_proj": (g.intermediate_size, d),
        "mlp.down_proj": (d, g.intermediate_size),
    }


@dataclass
class Q4Tensor:
    """A q4 g64 affine weight in MLX packing (``backends/mlx_ops.py:43-60``):
    ``w_q`` int32 view of uint32 words ``[N, K/8]`` (8 nibbles along K, low
    nibble first), ``scales``/``biases`` bf16 ``[N, K/64]``."""

    w_q: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor

    @property
    def shape(self):
        return (int(self.w_q.shape[0]), int(self.w_q.shape[1]) * 8)

    def to(self, device) -> "Q4Tensor":
        return Q4Tensor(self.w_q.to(device), self.scales.to(device), self.biases.to(device))


@dataclass
class SyntheticModel:
    geometry: ModelGeometry
    weight_kind: str  # "bf16" or "q4"
    weights: dict = field(default_factory=dict)


def _bf16_normal(gen, shape, std=0.02):
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(torch.bfloat16)


def random_q4(gen, n: int, k: int, *, scale_lo=0.003, scale_hi=0.006,
              centred=True, bias_lo=-0.1, bias_hi=0.1) -> Q4Tensor:
    """Random q4 words + bf16 scales/biases.

    ``centred=True`` (model weights): bias = -7.5*scale + U(-0.002, 0.002).
    ``centred=False`` (the isolated-linear workload): bias ~ U(bias_lo, bias_hi).
    """
    if k % Q4_GROUP:
        raise ValueError(f"in-dim {k} not divisible by {Q4_GROUP}")
    words = torch.randint(0, 256, (n, k // 2), generator=gen, dtype=torch.uint8)
    w_q = words.view(torch.int32).reshape(n, k // 8)
    groups = k // Q4_GROUP
    scales = torch.empty((n, groups), dtype=torch.float32).uniform_(scale_lo, scale_hi, generator=gen)
    if centred:
        jitter = torch.empty((n, groups), dtype=torch.float32).uniform_(-0.002, 0.002, generator=gen)
        biases = -7.5 * scales.to(torch.bfloat16).float() + jitter
    else:
        biases = torch.empty((n, groups), dtype=torch.float32).uniform_(bias_lo, bias_hi, generator=gen)
    return Q4Tensor(w_q.contiguous(), scales.to(torch.bfloat16), biases.to(torch.bfloat16))


def build_model(g: ModelGeometry, weight_kind: str, seed: int) -> SyntheticModel:
    """Generate all weights in a fixed key order from ``seed`` (CPU tensors)."""
    if weight_kind not in ("bf16", "q4"):
        raise ValueError(f"weight_kind must be bf16 or q4, got {weight_kind!r}")
    gen = torch.Generator().manual_seed(int(seed))
    w: dict = {}
    d = g.hidden_size
    w["model.embed_tokens.weight"] = _bf16_normal(gen, (g.vocab_size, d))
    ones_d = torch.ones(d, dtype=torch.bfloat16)
    shapes = linear_shapes(g)
    for i in range(g.layer_count):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = ones_d
        w[p + "post_attention_layernorm.weight"] = ones_d
        if g.qk_norm:
            w[p + "self_attn.q_norm.weight"] = torch.ones(g.head_dim, dtype=torch.bfloat16)
            w[p + "self_attn.k_norm.weight"] = torch.ones(g.head_dim, dtype=torch.bfloat16)
        for suffix in LINEAR_SUFFIXES:
            n, k = shapes[suffix]
            if weight_kind == "bf16":
                w[p + suffix + ".weight"] = _bf16_normal(gen, (n, k))
            else:
                w[p + suffix + ".weight"] = random_q4(gen, n, k)
            if g.qkv_bias and suffix in ("self_attn.q_proj", "self_attn.k_proj",
                                         "self_attn.v_proj"):
                w[p + suffix + ".bias"] = _bf16_normal(gen, (n,))
    w["model.norm.weight"] = ones_d
    if weight_kind == "bf16":
        w["lm_head.weight"] = (w["model.embed_tokens.weight"] if g.tie_word_embeddings
                               else _bf16_normal(gen, (g.vocab_size, d)))
    else:
        w["lm_head.weight"] = random_q4(gen, g.vocab_size, d)
    return SyntheticModel(geometry=g, weight_kind=weight_kind, weights=w)


def prompt_ids(seed: int, length: int, *, high: int = 151643) -> list:
    """Prompt token ids uniform in ``[0, high)`` (special tokens excluded)."""
    gen = torch.Generator().manual_seed(int(seed))
    return torch.randint(0, high, (length,), generator=gen, dtype=torch.int64).tolist()


def to_oracle_weights(model: SyntheticModel):
    """numpy view of the weights for the oracle (bf16 -> float32 values; q4 ->
    packed uint32 + float scales/biases)."""
    import numpy as np

    out = {}
    for key, value in model.weights.items():
        if isinstance(value, Q4Tensor):
            out[key] = (value.w_q.numpy().view(np.uint32), value.scales.float().numpy(),
                        value.biases.float().numpy())
        else:
            out[key] = value.float().numpy()
    return out


def oracle_config(g: ModelGeometry, weight_kind: str) -> dict:
    return {"n_layers": g.layer_count, "d": g.hidden_size, "n_heads": g.num_heads,
            "n_kv_heads": g.num_kv_heads, "head_dim": g.head_dim, "eps": g.rms_norm_eps,
            "rope_theta": g.rope_theta, "qk_norm": g.qk_norm, "weight_kind": weight_kind,
            "vocab": g.vocab_size}
