"""Writes execution packages in the reference's on-disk format for the loader tests.

Layout (the reference's ``python/src/edllm/``): ``model.json`` with
``merged_weights_ref`` / ``package_format`` / ``weight_storage_dtype`` /
``output_hash`` / ``model_config`` (``converter/convert_hf_masked_diffusion.py:292-330``;
``model_config`` in the normalized form of ``model_definitions.py:589-627``), and the
weights as one fp32 NPZ (``npz_v1``) or as safetensors shards under ``weights/``
with a JSON index (``safetensors_sharded_v1``, ``weight_store.py:359-532``).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import torch

from diffusorrt_amd.synthetic import LINEAR_SUFFIXES, ModelGeometry, linear_shapes

ARCH_NAME = {("raw", True): "A2DQwen3BD3LM", ("dream_ar_shift", False): "DreamModel"}


def model_config(g: ModelGeometry, architecture: str | None = None) -> dict:
    arch = architecture or ARCH_NAME[(g.logits_convention, g.qk_norm)]
    return {
        "architecture": arch, "layer_count": g.layer_count, "num_hidden_layers": g.layer_count,
        "hidden_size": g.hidden_size, "attention_heads": g.num_heads,
        "num_key_value_heads": g.num_kv_heads, "num_kv_heads": g.num_kv_heads,
        "head_dim": g.head_dim, "intermediate_size": g.intermediate_size,
        "vocab_size": g.vocab_size, "max_position_embeddings": g.max_position_embeddings,
        "rope_theta": g.rope_theta, "rope_scaling": {"rope_type": "linear", "factor": 1.0},
        "rms_norm_eps": g.rms_norm_eps, "mask_token_id": g.mask_token_id,
        "tie_word_embeddings": g.tie_word_embeddings, "bos_token_id": 0,
        "eos_token_id": g.eos_token_id, "pad_token_id": 0, "block_size": 32, "step_budget": 4,
        "attention_mask_kind": "bidirectional",
        "block_schedule": {"kind": "fixed", "block_size": 32},
    }


def random_weights(g: ModelGeometry, seed: int, dtype=torch.float32) -> dict:
    """Floating-point weights of the architecture (not bf16-exact in fp32, so the
    load-time cast is exercised): linears and embedding ~ N(0, 0.02), norms ~
    1 + N(0, 0.05), biases ~ N(0, 0.02). Tied packages store ``lm_head.weight``
    equal to the embedding, as the reference's writer does."""
    gen = torch.Generator().manual_seed(seed)

    def normal(shape, std=0.02, mean=0.0):
        return (torch.randn(shape, generator=gen) * std + mean).to(dtype)

    d = g.hidden_size
    w = {"model.embed_tokens.weight": normal((g.vocab_size, d))}
    shapes = linear_shapes(g)
    for i in range(g.layer_count):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = normal((d,), 0.05, 1.0)
        w[p + "post_attention_layernorm.weight"] = normal((d,), 0.05, 1.0)
        if g.qk_norm:
            w[p + "self_attn.q_norm.weight"] = normal((g.head_dim,), 0.05, 1.0)
            w[p + "self_attn.k_norm.weight"] = normal((g.head_dim,), 0.05, 1.0)
        for s in LINEAR_SUFFIXES:
            w[p + s + ".weight"] = normal(shapes[s])
            if g.qkv_bias and s in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"):
                w[p + s + ".bias"] = normal((shapes[s][0],))
    w["model.norm.weight"] = normal((d,), 0.05, 1.0)
    w["lm_head.weight"] = (w["model.embed_tokens.weight"].clone() if g.tie_word_embeddings
                           else normal((g.vocab_size, d)))
    return w


def _sha256(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def write_package(root, g: ModelGeometry, weights: dict, *, fmt: str = "safetensors",
                  max_shard_bytes: int = 1 << 20, legacy_manifest: bool = False,
                  architecture: str | None = None) -> Path:
    """Write a package under ``root``; returns its directory.

    ``fmt="npz"`` stores fp32 arrays in ``weights.npz`` (legacy manifest without
    storage fields when ``legacy_manifest``); ``fmt="safetensors"`` stores the
    tensors in their own dtype, split into shards of about ``max_shard_bytes``."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    manifest = {"version": {"major": 2, "minor": 0, "patch": 0}, "fixture_mode": False,
                "decode_family": "masked_diffusion",
                "model_config": model_config(g, architecture)}
    if fmt == "npz":
        path = root / "weights.npz"
        arrays = {k: v.detach().float().numpy() for k, v in weights.items()}
        with path.open("wb") as f:
            np.savez(f, **arrays)
        manifest["merged_weights_ref"] = "weights.npz"
        manifest["output_hash"] = _sha256(path)
        if not legacy_manifest:
            manifest["package_format"] = "npz_v1"
            manifest["weight_storage_dtype"] = "fp32"
    elif fmt == "safetensors":
        from safetensors.torch import save_file

        wdir = root / "weights"
        wdir.mkdir()
        shards, batch, records, size, total = [], {}, [], 0, 0

        def flush():
            nonlocal batch, records, size
            if not batch:
                return
            fname = f"shard-{len(shards) + 1:05d}.safetensors"
            save_file(batch, str(wdir / fname), metadata={"format": "diffusorrt"})
            shards.append({"ref": f"weights/{fname}", "sha256": _sha256(wdir / fname),
                           "byte_length": (wdir / fname).stat().st_size, "tensors": records})
            batch, records, size = {}, [], 0

        for name, t in weights.items():
            t = t.detach().contiguous()
            nbytes = t.numel() * t.element_size()
            if batch and size + nbytes > max_shard_bytes:
                flush()
            batch[name] = t
            records.append({"name": name, "dtype": str(t.dtype).removeprefix("torch."),
                            "shape": list(t.shape), "byte_length": nbytes})
            size += nbytes
            total += nbytes
        flush()
        index = {"schema_version": 1, "format": "safetensors", "storage_dtype": "preserved",
                 "tensor_count": len(weights), "total_tensor_bytes": total, "shards": shards}
        (wdir / "weights.index.json").write_text(
            json.dumps(index, sort_keys=True, separators=(",", ":")) + "\n")
        manifest["merged_weights_ref"] = "weights/weights.index.json"
        manifest["output_hash"] = _sha256(wdir / "weights.index.json")
        manifest["package_format"] = "safetensors_sharded_v1"
        manifest["weight_storage_dtype"] = "preserved"
    else:
        raise ValueError(fmt)
    (root / "model.json").write_text(json.dumps(manifest, indent=1, sort_keys=True))
    return root


def rewrite_manifest(root, **changes) -> None:
    path = Path(root) / "model.json"
    m = json.loads(path.read_text())
    for k, v in changes.items():
        if v is None:
            m.pop(k, None)
        else:
            m[k] = v
    path.write_text(json.dumps(m))
