"""Execution-package reading on the CPU: manifest, weight-store index, verified
shards, geometry and the tensor set (no device work)."""
from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from diffusorrt_amd import package as P

from helpers import tiny_dream_geometry, tiny_geometry
from package_writer import random_weights, rewrite_manifest, write_package


@pytest.fixture(scope="module")
def bd3():
    g = tiny_geometry(layer_count=1, vocab_size=256, max_position_embeddings=2048)
    return g, random_weights(g, seed=3, dtype=torch.bfloat16)


def _write(tmp_path, bd3, **kw):
    g, w = bd3
    return write_package(tmp_path / "pkg", g, w, **kw)


def test_sharded_store_reads_back_every_tensor(tmp_path, bd3):
    g, w = bd3
    root = _write(tmp_path, bd3, max_shard_bytes=200_000)
    manifest, spec, geo = P.read_package(root)
    assert spec.format == P.SAFETENSORS_SHARDED_V1 and spec.storage_dtype == "preserved"
    index = P.read_weight_store_index(root, spec)
    assert len(index.shards) > 2 and index.tensor_names == frozenset(w)
    got = dict(P.iter_package_tensors(root, spec))
    assert set(got) == set(w)
    for k, v in w.items():
        assert got[k].dtype == torch.bfloat16 and torch.equal(got[k], v), k
    # geometry round trip (architecture flags from the table)
    for f in ("layer_count", "hidden_size", "num_heads", "num_kv_heads", "head_dim",
              "intermediate_size", "vocab_size", "mask_token_id", "eos_token_id",
              "tie_word_embeddings", "max_position_embeddings"):
        assert getattr(geo, f) == getattr(g, f), f
    assert geo.qk_norm and not geo.qkv_bias and geo.logits_convention == "raw"
    P.check_tensor_names(geo, P.package_tensor_names(root, spec))


@pytest.mark.parametrize("legacy", [False, True])
def test_npz_store_reads_fp32(tmp_path, legacy):
    g = tiny_dream_geometry(layer_count=1, vocab_size=256)
    w = random_weights(g, seed=4)
    root = write_package(tmp_path / "pkg", g, w, fmt="npz", legacy_manifest=legacy)
    _, spec, geo = P.read_package(root)
    assert spec.format == P.NPZ_V1 and spec.storage_dtype == "fp32"
    assert geo.qkv_bias and not geo.qk_norm and geo.logits_convention == "dream_ar_shift"
    got = dict(P.iter_package_tensors(root, spec))
    for k, v in w.items():
        assert got[k].dtype == torch.float32 and torch.equal(got[k], v), k
    P.check_tensor_names(geo, P.package_tensor_names(root, spec))


def test_npz_digest_is_verified(tmp_path):
    g = tiny_geometry(layer_count=1, vocab_size=256)
    root = write_package(tmp_path / "pkg", g, random_weights(g, 5), fmt="npz")
    rewrite_manifest(root, output_hash="0" * 64)
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_npz_digest_mismatch"):
        list(P.iter_package_tensors(root, spec))


def _first_shard(root):
    return sorted((root / "weights").glob("shard-*.safetensors"))[0]


def test_tampered_shard_fails_digest(tmp_path, bd3):
    root = _write(tmp_path, bd3)
    shard = _first_shard(root)
    data = bytearray(shard.read_bytes())
    data[-1] ^= 0x01  # same size, one bit of tensor data flipped
    shard.write_bytes(bytes(data))
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_shard_digest_mismatch"):
        list(P.iter_package_tensors(root, spec))


def test_truncated_shard_fails_size(tmp_path, bd3):
    root = _write(tmp_path, bd3)
    shard = _first_shard(root)
    shard.write_bytes(shard.read_bytes()[:-8])
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_shard_size_mismatch"):
        list(P.iter_package_tensors(root, spec))


def test_index_digest_bound_to_manifest(tmp_path, bd3):
    root = _write(tmp_path, bd3)
    rewrite_manifest(root, output_hash="a" * 64)
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_index_digest_mismatch"):
        P.read_weight_store_index(root, spec)


def _index_payload(root):
    return json.loads((root / "weights" / "weights.index.json").read_text())


def _reindex(root, index):
    (root / "weights" / "weights.index.json").write_text(json.dumps(index))
    rewrite_manifest(root, output_hash="")  # no digest binding: reach the contract checks


@pytest.mark.parametrize("mutate, error", [
    (lambda ix: ix.update(schema_version=2), "weight_store_index_version_unsupported"),
    (lambda ix: ix.update(format="npz"), "weight_store_index_format_unsupported"),
    (lambda ix: ix.update(storage_dtype="fp32"), "weight_store_index_storage_dtype_invalid"),
    (lambda ix: ix.update(tensor_count=ix["tensor_count"] + 1),
     "weight_store_index_tensor_count_mismatch"),
    (lambda ix: ix.update(total_tensor_bytes=ix["total_tensor_bytes"] + 2),
     "weight_store_index_tensor_bytes_mismatch"),
    (lambda ix: ix.update(extra=1), "weight_store_index_contract_invalid"),
    (lambda ix: ix["shards"][0].update(ref="../outside.safetensors"),
     "weight_store_shard_ref_unsafe"),
    (lambda ix: ix["shards"][0].update(ref="/abs.safetensors"), "weight_store_shard_ref_unsafe"),
    (lambda ix: ix["shards"][0].update(sha256="XYZ"), "weight_store_shard_digest_invalid"),
    (lambda ix: ix["shards"].append(dict(ix["shards"][0])), "weight_store_shard_ref_duplicated"),
    (lambda ix: ix["shards"][1]["tensors"].append(dict(ix["shards"][0]["tensors"][0])),
     "weight_store_tensor_name_duplicated"),
    (lambda ix: ix["shards"][0]["tensors"][0].update(shape=[-1]),
     "weight_store_tensor_shape_invalid"),
])
def test_index_contract_fails_closed(tmp_path, bd3, mutate, error):
    root = _write(tmp_path, bd3, max_shard_bytes=200_000)
    ix = _index_payload(root)
    mutate(ix)
    _reindex(root, ix)
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match=error):
        P.read_weight_store_index(root, spec)


def test_duplicate_json_keys_refused(tmp_path, bd3):
    root = _write(tmp_path, bd3)
    text = (root / "weights" / "weights.index.json").read_text()
    (root / "weights" / "weights.index.json").write_text(
        text.replace('{"format"', '{"format":"safetensors","format"', 1))
    rewrite_manifest(root, output_hash="")
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_index_malformed"):
        P.read_weight_store_index(root, spec)


def test_shard_record_mismatch_is_caught_after_digest(tmp_path, bd3):
    root = _write(tmp_path, bd3, max_shard_bytes=200_000)
    ix = _index_payload(root)
    ix["shards"][0]["tensors"][0]["dtype"] = "float32"
    _reindex(root, ix)
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_shard_tensor_dtype_mismatch"):
        list(P.iter_package_tensors(root, spec))


def test_symlinks_are_refused(tmp_path, bd3):
    root = _write(tmp_path, bd3)
    shard = _first_shard(root)
    moved = tmp_path / "elsewhere.safetensors"
    shard.rename(moved)
    os.symlink(moved, shard)
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_shard_symlink_forbidden"):
        list(P.iter_package_tensors(root, spec))
    # a linked directory component is refused too
    root2 = _write(tmp_path / "b", bd3)
    (root2 / "weights").rename(tmp_path / "wdir")
    os.symlink(tmp_path / "wdir", root2 / "weights")
    _, spec2, _ = P.read_package(root2)
    with pytest.raises(ValueError, match="symlink_forbidden"):
        P.read_weight_store_index(root2, spec2)


def test_manifest_storage_identity(tmp_path, bd3):
    root = _write(tmp_path, bd3)
    rewrite_manifest(root, weight_storage_dtype=None)
    with pytest.raises(ValueError, match="package_weight_storage_identity_incomplete"):
        P.read_package(root)
    rewrite_manifest(root, weight_storage_dtype="fp32")
    with pytest.raises(ValueError, match="safetensors_sharded_v1 requires"):
        P.read_package(root)
    rewrite_manifest(root, package_format="tarball", weight_storage_dtype="preserved")
    with pytest.raises(ValueError, match="weight_artifact_format_unknown"):
        P.read_package(root)
    rewrite_manifest(root, merged_weights_ref=None)
    with pytest.raises(ValueError, match="package_weights_ref_missing"):
        P.read_package(root)
    (root / "model.json").write_text('{"a": 1, "a": 2}')
    with pytest.raises(ValueError, match="package_manifest_malformed"):
        P.read_package(root)
    (root / "model.json").unlink()
    with pytest.raises(ValueError, match="package_manifest_artifact_missing"):
        P.read_package(root)


def test_geometry_from_model_config():
    from package_writer import model_config

    g = tiny_geometry()
    cfg = model_config(g)
    geo = P.geometry_from_model_config(cfg)
    assert geo.rope_scaling_factor == 1.0 and geo.rope_theta == g.rope_theta
    cfg2 = dict(cfg, rope_scaling={"type": "linear", "factor": 2.0})
    assert P.geometry_from_model_config(cfg2).rope_scaling_factor == 2.0
    with pytest.raises(P.PackageUnsupported):
        P.geometry_from_model_config(dict(cfg, rope_scaling={"rope_type": "yarn", "factor": 4.0}))
    with pytest.raises(ValueError, match="unsupported_architecture_family"):
        P.geometry_from_model_config(dict(cfg, architecture="GPT2"))
    with pytest.raises(P.PackageUnsupported):
        P.geometry_from_model_config(dict(cfg, architecture="LLaDAModelLM"))
    for alias in ("A2DQwen3", "a2d-qwen3", "qwen3_bd3lm"):
        geo = P.geometry_from_model_config(dict(cfg, architecture=alias))
        assert geo.qk_norm and not geo.qkv_bias and geo.logits_convention == "raw"
    geo = P.geometry_from_model_config(dict(cfg, architecture="dream"))
    assert geo.qkv_bias and not geo.qk_norm and geo.logits_convention == "dream_ar_shift"
    with pytest.raises(ValueError, match="lacks hidden_size"):
        P.geometry_from_model_config({k: v for k, v in cfg.items() if k != "hidden_size"})


def test_tensor_set_is_exact():
    g = tiny_geometry(layer_count=2)
    d = tiny_dream_geometry(layer_count=2)
    names_g, names_d = P.expected_weight_names(g), P.expected_weight_names(d)
    # 2 layers x (2 norms + 7 linears + 2 qk norms) + embed + norm + lm_head
    assert len(names_g) == 2 * 11 + 3
    # 2 layers x (2 norms + 7 linears + 3 biases) + 3
    assert len(names_d) == 2 * 12 + 3
    P.check_tensor_names(g, names_g)
    with pytest.raises(ValueError, match="package_weight_missing"):
        P.check_tensor_names(d, names_d - {"model.layers.1.self_attn.v_proj.bias"})
    with pytest.raises(ValueError, match="package_weight_unexpected"):
        P.check_tensor_names(g, names_g | {"model.layers.0.self_attn.q_proj.bias"})
    with pytest.raises(ValueError, match="package_weight_missing"):
        P.check_tensor_names(g, names_g - {"lm_head.weight"})
    # quantized set: the seven projections and the LM head, never embeddings/norms/biases
    q = sorted(n for n in names_d if P.is_quantized_linear(n))
    assert len(q) == 2 * 7 + 1 and "model.embed_tokens.weight" not in q
    assert not any(n.endswith((".bias", "norm.weight")) for n in q)
    for n in names_d:
        assert len(P.expected_shape(d, n)) in (1, 2)
    assert P.expected_shape(d, "model.layers.0.self_attn.k_proj.bias") == (128,)
    assert P.expected_shape(g, "model.layers.1.mlp.down_proj.weight") == (256, 512)


def test_npz_object_arrays_are_never_unpickled(tmp_path):
    g = tiny_geometry(layer_count=1, vocab_size=256)
    root = write_package(tmp_path / "pkg", g, random_weights(g, 6), fmt="npz")
    arrays = dict(np.load(root / "weights.npz"))
    arrays["model.norm.weight"] = np.array([{"x": 1}], dtype=object)
    with (root / "weights.npz").open("wb") as f:
        np.savez(f, **arrays)
    rewrite_manifest(root, output_hash="")
    _, spec, _ = P.read_package(root)
    with pytest.raises(ValueError, match="weight_store_npz_tensor_invalid"):
        list(P.iter_package_tensors(root, spec))
