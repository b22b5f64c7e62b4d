"""Execution-package loading for the ``rocm`` runtime: manifest, weight store and
the load-time weight preparation on the device.

A package directory (written by the reference's converter,
``converter/convert_hf_masked_diffusion.py:231-330``; paths here are relative to
the reference's ``python/src/edllm/``) holds ``model.json`` (``model.py:2376``).
Its ``merged_weights_ref`` names the weights in one of two encodings
(``weight_store.py:35-42, 135-157``):

* ``npz_v1``: one NPZ of fp32 arrays, read with ``allow_pickle=False``. A legacy
  manifest without ``package_format`` / ``weight_storage_dtype`` is this.
* ``safetensors_sharded_v1``: a bounded JSON index naming safetensors shards,
  each with its sha256, byte length and exact tensor set, dtypes preserved
  (``weight_store.py:211-357``).

Every file is opened relative to the package directory, one path component at
a time, without following symbolic links (``package_artifacts.py:21-45, 119-...``).
Errors are ``ValueError`` named ``<scope>_<artifact>_<reason>`` as in the
reference (``weight_store_shard_digest_mismatch``, ...).

Load-time preparation (``backends/mlx_dream.py:1957-1963, 1998-1999, 2073-2108``)
runs in this library's HIP kernels: floating-point tensors are cast to the
resident bf16 dtype (``drt_op_cast_bf16``), and with ``linear_quant_bits=4`` the
seven per-layer projections and ``lm_head.weight`` are quantized, affine with
group 64, into the MLX packing (``drt_op_q4_quantize``). Embeddings, norms and
biases are never quantized. One tensor at a time is resident in floating point
on the device, so a 7B package needs no more than its largest tensor beyond
the runtime's own weights.
"""
from __future__ import annotations

import ctypes as C
import errno
import hashlib
import io
import json
import os
import stat
from contextlib import ExitStack, contextmanager
from dataclasses import dataclass, field
from pathlib import Path, PurePosixPath
from typing import Iterator

from .synthetic import LINEAR_SUFFIXES, ModelGeometry, Q4Tensor

MANIFEST_REF = "model.json"
MAX_MANIFEST_BYTES = 16 * 1024 * 1024
NPZ_V1 = "npz_v1"
SAFETENSORS_SHARDED_V1 = "safetensors_sharded_v1"
PRESERVED_DTYPE = "preserved"
WEIGHT_STORE_INDEX_VERSION = 1
MAX_WEIGHT_INDEX_BYTES = 16 * 1024 * 1024
_INDEX_FIELDS = frozenset({"schema_version", "format", "storage_dtype", "tensor_count",
                           "total_tensor_bytes", "shards"})
_SHARD_FIELDS = frozenset({"ref", "sha256", "byte_length", "tensors"})
_TENSOR_FIELDS = frozenset({"name", "dtype", "shape", "byte_length"})

# Runtime architectures this backend executes (model_definitions.py:417-449):
# key -> (aliases, shifted logits, qk-norm, q/k/v bias).
ARCHITECTURES = {
    "qwen2_dream": (("DreamModel", "qwen2_dream", "dream", "qwen2", "dream_stub"),
                    True, False, True),
    "qwen3_mdlm": (("A2DQwen3", "a2d-qwen3", "qwen3_mdlm"), False, True, False),
    "qwen3_bd3lm": (("A2DQwen3BD3LM", "qwen3_bd3lm"), False, True, False),
}
# Known to the reference, not executed here (a different block structure).
UNSUPPORTED_ARCHITECTURES = ("LLaDAModelLM", "llada")


class PackageUnsupported(NotImplementedError):
    """A well-formed package this backend does not execute."""


# ---------------------------------------------------------------------------
# Package-relative file access
# ---------------------------------------------------------------------------


def _err(scope: str, artifact: str, reason: str) -> ValueError:
    return ValueError("_".join(p for p in (scope, artifact, reason) if p))


def package_ref_parts(ref, *, scope: str, artifact: str) -> tuple[str, ...]:
    """The components of a package-relative reference, or ``<scope>_<artifact>_ref_unsafe``
    for an empty, absolute, NUL-bearing or ``.``/``..``/empty-component reference
    (``package_artifacts.py:21-45``)."""
    text = ref if isinstance(ref, str) else ""
    parts = text.replace("\\", "/").split("/")
    if (not text or "\x00" in text or text.startswith("/")
            or any(p in ("", ".", "..") for p in parts)):
        raise _err(scope, artifact, "ref_unsafe")
    return tuple(PurePosixPath(text).parts)


@contextmanager
def open_artifact(package_dir, ref, *, scope: str, artifact: str,
                  max_bytes: int | None = None) -> Iterator[tuple[io.BufferedReader, os.stat_result]]:
    """Open a regular file of the package for reading, walking the reference one
    component at a time from the package directory with ``O_NOFOLLOW``: a symbolic
    link anywhere below the package directory is refused."""
    parts = package_ref_parts(ref, scope=scope, artifact=artifact)
    try:
        root = Path(package_dir).resolve(strict=True)
    except (OSError, TypeError, ValueError) as exc:
        raise _err(scope, "package", "dir_unavailable") from exc
    dir_flags = os.O_RDONLY | os.O_DIRECTORY | os.O_NOFOLLOW
    with ExitStack() as stack:
        try:
            fd = os.open(root, dir_flags)
        except OSError as exc:
            raise _err(scope, "package", "dir_unavailable") from exc
        stack.callback(os.close, fd)
        for i, part in enumerate(parts):
            last = i == len(parts) - 1
            flags = (os.O_RDONLY | os.O_NOFOLLOW | os.O_NONBLOCK) if last else dir_flags
            try:
                nfd = os.open(part, flags, dir_fd=fd)
            except OSError as exc:
                if exc.errno == errno.ENOENT:
                    raise _err(scope, artifact, "artifact_missing") from exc
                if exc.errno == errno.ELOOP:
                    raise _err(scope, artifact, "symlink_forbidden") from exc
                if exc.errno == errno.ENOTDIR:
                    # a directory component that is not a directory: a link to
                    # one (O_DIRECTORY | O_NOFOLLOW) or a file
                    try:
                        linked = stat.S_ISLNK(os.stat(part, dir_fd=fd,
                                                      follow_symlinks=False).st_mode)
                    except OSError:
                        linked = False
                    raise _err(scope, artifact,
                               "symlink_forbidden" if linked else "ref_unsafe") from exc
                raise _err(scope, artifact, "artifact_unavailable") from exc
            if not last:
                stack.callback(os.close, nfd)
                fd = nfd
                continue
            st = os.fstat(nfd)
            if not stat.S_ISREG(st.st_mode):
                os.close(nfd)
                raise _err(scope, artifact, "not_regular_file")
            if max_bytes is not None and st.st_size > max_bytes:
                os.close(nfd)
                raise _err(scope, artifact, "too_large")
            # the descriptor is blocking for the reads that follow
            os.set_blocking(nfd, True)
            with os.fdopen(nfd, "rb") as handle:
                yield handle, st


def _same_file(a: os.stat_result, b: os.stat_result) -> bool:
    return (a.st_dev, a.st_ino, a.st_size, a.st_mtime_ns) == (b.st_dev, b.st_ino, b.st_size,
                                                              b.st_mtime_ns)


def _load_json_unique_keys(payload: bytes, *, scope: str, artifact: str):
    """JSON with duplicate keys and non-finite numbers refused
    (``weight_store.py:61-82``)."""
    def pairs(items):
        out = {}
        for k, v in items:
            if k in out:
                raise _err(scope, artifact, "malformed")
            out[k] = v
        return out

    def constant(_):
        raise _err(scope, artifact, "malformed")

    try:
        return json.loads(payload, object_pairs_hook=pairs, parse_constant=constant)
    except (json.JSONDecodeError, RecursionError, UnicodeDecodeError) as exc:
        raise _err(scope, artifact, "malformed") from exc


def read_manifest(package_dir) -> dict:
    """``model.json`` of the package, a JSON object."""
    with open_artifact(package_dir, MANIFEST_REF, scope="package", artifact="manifest",
                       max_bytes=MAX_MANIFEST_BYTES) as (handle, _):
        payload = handle.read(MAX_MANIFEST_BYTES + 1)
    manifest = _load_json_unique_keys(payload, scope="package", artifact="manifest")
    if not isinstance(manifest, dict):
        raise _err("package", "manifest", "malformed")
    return manifest


# ---------------------------------------------------------------------------
# Weight store (weight_store.py)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class WeightArtifactSpec:
    """The package's storage decision (``weight_store.py:85-132``)."""

    format: str
    primary_ref: str
    storage_dtype: str
    digest: str = ""

    def __post_init__(self):
        if self.format not in (NPZ_V1, SAFETENSORS_SHARDED_V1):
            raise ValueError(f"weight_artifact_format_unknown: {self.format!r}")
        if not isinstance(self.primary_ref, str) or not self.primary_ref:
            raise ValueError("weight_artifact_primary_ref_invalid")
        package_ref_parts(self.primary_ref, scope="weight_store", artifact="primary")
        if self.format == NPZ_V1 and self.storage_dtype != "fp32":
            raise ValueError("npz_v1 requires weight_storage_dtype='fp32'")
        if self.format == SAFETENSORS_SHARDED_V1 and self.storage_dtype != PRESERVED_DTYPE:
            raise ValueError("safetensors_sharded_v1 requires weight_storage_dtype='preserved'")
        if self.digest and not _hex_sha256(self.digest):
            raise ValueError("weight_artifact_digest_invalid")


def _hex_sha256(value) -> bool:
    return (isinstance(value, str) and len(value) == 64
            and all(c in "0123456789abcdef" for c in value))


def weight_artifact_spec(manifest: dict) -> WeightArtifactSpec:
    """``weight_store.py:135-157``: the legacy NPZ when neither ``package_format``
    nor ``weight_storage_dtype`` is recorded, else exactly what is recorded."""
    primary = manifest.get("merged_weights_ref")
    if not isinstance(primary, str) or not primary:
        raise ValueError("package_weights_ref_missing")
    digest = manifest.get("output_hash", "")
    if digest is None:
        digest = ""
    if not isinstance(digest, str):
        raise ValueError("weight_artifact_digest_invalid")
    fmt = manifest.get("package_format")
    dtype = manifest.get("weight_storage_dtype")
    if fmt is None and dtype is None:
        return WeightArtifactSpec(NPZ_V1, primary, "fp32", digest)
    if not isinstance(fmt, str) or not isinstance(dtype, str):
        raise ValueError("package_weight_storage_identity_incomplete")
    return WeightArtifactSpec(fmt, primary, dtype, digest)


@dataclass(frozen=True)
class TensorRecord:
    name: str
    dtype: str
    shape: tuple
    byte_length: int


@dataclass(frozen=True)
class ShardRecord:
    ref: str
    sha256: str
    byte_length: int
    tensors: tuple


@dataclass(frozen=True)
class WeightStoreIndex:
    shards: tuple
    tensor_count: int
    total_tensor_bytes: int
    digest: str

    @property
    def tensor_names(self) -> frozenset:
        return frozenset(t.name for s in self.shards for t in s.tensors)


def _require(ok: bool, error_id: str) -> None:
    if not ok:
        raise ValueError(error_id)


def _text(v) -> bool:
    return isinstance(v, str) and v != ""


def _int_at_least(least: int):
    return lambda v: type(v) is int and v >= least


def _record(obj, fields: frozenset, error_id: str, checks) -> dict:
    """``obj`` must be a JSON object with exactly ``fields``; each ``(key,
    predicate, error id)`` of ``checks`` is then tried in order."""
    _require(isinstance(obj, dict) and set(obj) == fields, error_id)
    for key, ok, err in checks:
        _require(ok(obj[key]), err)
    return obj


# The weight-store index contract (weight_store.py:201-296) as check tables; the
# error identifiers are the reference's, so a caller sees the same failures.
_TENSOR_CHECKS = (
    ("name", _text, "weight_store_tensor_name_invalid"),
    ("dtype", _text, "weight_store_tensor_dtype_invalid"),
    ("shape", lambda v: isinstance(v, list) and all(type(d) is int and d >= 0 for d in v),
     "weight_store_tensor_shape_invalid"),
    ("byte_length", _int_at_least(0), "weight_store_tensor_bytes_invalid"),
)
_INDEX_CHECKS = (
    ("schema_version", lambda v: type(v) is int and v == WEIGHT_STORE_INDEX_VERSION,
     "weight_store_index_version_unsupported"),
    ("format", lambda v: v == "safetensors", "weight_store_index_format_unsupported"),
    ("storage_dtype", lambda v: v == PRESERVED_DTYPE, "weight_store_index_storage_dtype_invalid"),
    ("tensor_count", _int_at_least(1), "weight_store_index_tensor_count_invalid"),
    ("total_tensor_bytes", _int_at_least(1), "weight_store_index_tensor_bytes_invalid"),
    ("shards", lambda v: isinstance(v, list) and len(v) > 0, "weight_store_index_shards_invalid"),
)


def _tensor_record(p) -> TensorRecord:
    r = _record(p, _TENSOR_FIELDS, "weight_store_tensor_record_invalid", _TENSOR_CHECKS)
    return TensorRecord(r["name"], r["dtype"], tuple(r["shape"]), r["byte_length"])


def _shard_record(sp, seen_refs: set) -> ShardRecord:
    def fresh_ref(ref) -> bool:
        package_ref_parts(ref, scope="weight_store", artifact="shard")
        _require(ref not in seen_refs, "weight_store_shard_ref_duplicated")
        seen_refs.add(ref)
        return True

    r = _record(sp, _SHARD_FIELDS, "weight_store_shard_record_invalid", (
        ("ref", _text, "weight_store_shard_ref_invalid"),
        ("ref", fresh_ref, "weight_store_shard_ref_invalid"),
        ("sha256", _hex_sha256, "weight_store_shard_digest_invalid"),
        ("byte_length", _int_at_least(1), "weight_store_shard_bytes_invalid"),
        ("tensors", lambda v: isinstance(v, list) and len(v) > 0,
         "weight_store_shard_tensors_invalid"),
    ))
    return ShardRecord(r["ref"], r["sha256"], r["byte_length"],
                       tuple(_tensor_record(t) for t in r["tensors"]))


def parse_weight_store_index(payload: bytes) -> WeightStoreIndex:
    """Validate the index contract (``weight_store.py:211-296``): the record's
    fields, each shard and tensor record, unique shard refs and tensor names,
    and the declared tensor count and byte total."""
    idx = _record(_load_json_unique_keys(payload, scope="weight_store", artifact="index"), _INDEX_FIELDS,
                  "weight_store_index_contract_invalid", _INDEX_CHECKS)
    refs: set = set()
    shards = tuple(_shard_record(sp, refs) for sp in idx["shards"])
    records = [t for sh in shards for t in sh.tensors]
    names = {t.name for t in records}
    _require(len(names) == len(records), "weight_store_tensor_name_duplicated")
    _require(len(names) == idx["tensor_count"], "weight_store_index_tensor_count_mismatch")
    _require(sum(t.byte_length for t in records) == idx["total_tensor_bytes"],
             "weight_store_index_tensor_bytes_mismatch")
    return WeightStoreIndex(shards, idx["tensor_count"], idx["total_tensor_bytes"],
                            hashlib.sha256(payload).hexdigest())


def read_weight_store_index(package_dir, spec: WeightArtifactSpec) -> WeightStoreIndex:
    """``weight_store.py:299-318``: bounded read, stable file, digest bound to the spec."""
    if spec.format != SAFETENSORS_SHARDED_V1:
        raise ValueError("weight_store_index_requires_sharded_safetensors")
    with open_artifact(package_dir, spec.primary_ref, scope="weight_store", artifact="index",
                       max_bytes=MAX_WEIGHT_INDEX_BYTES) as (handle, st):
        payload = handle.read(MAX_WEIGHT_INDEX_BYTES + 1)
        if not _same_file(os.fstat(handle.fileno()), st):
            raise ValueError("weight_store_index_changed")
    index = parse_weight_store_index(payload)
    if spec.digest and index.digest != spec.digest:
        raise ValueError("weight_store_index_digest_mismatch")
    return index


_TORCH_DTYPE_NAMES = ("float32", "bfloat16", "float16", "float64", "int32", "int64", "uint8",
                      "int8", "bool")


def _read_shard(package_dir, shard: ShardRecord) -> dict:
    """One shard's tensors (torch, CPU), after its size and sha256 match the index
    (``weight_store.py:321-346``) and its tensor set, shapes and dtypes match the
    records (``backends/mlx_dream.py:1991-2001``)."""
    from safetensors.torch import load as st_load

    with open_artifact(package_dir, shard.ref, scope="weight_store",
                       artifact="shard") as (handle, st):
        if st.st_size != shard.byte_length:
            raise ValueError("weight_store_shard_size_mismatch")
        data = handle.read()
        if not _same_file(os.fstat(handle.fileno()), st) or len(data) != shard.byte_length:
            raise ValueError("weight_store_shard_changed")
    if hashlib.sha256(data).hexdigest() != shard.sha256:
        raise ValueError("weight_store_shard_digest_mismatch")
    try:
        loaded = st_load(data)
    except Exception as exc:  # a malformed safetensors header
        raise ValueError("weight_store_shard_malformed") from exc
    expected = {t.name: t for t in shard.tensors}
    if set(loaded) != set(expected):
        raise ValueError("weight_store_shard_tensor_set_mismatch")
    for name, rec in expected.items():
        t = loaded[name]
        if tuple(int(d) for d in t.shape) != rec.shape:
            raise ValueError("weight_store_shard_tensor_shape_mismatch")
        if str(t.dtype).removeprefix("torch.") != rec.dtype.lower():
            raise ValueError("weight_store_shard_tensor_dtype_mismatch")
    return loaded


def iter_package_tensors(package_dir, spec: WeightArtifactSpec, *, verify_digest: bool = True):
    """Yield ``(name, CPU torch tensor)`` for every tensor of the weight store, one
    shard (or one NPZ member) at a time."""
    import numpy as np
    import torch

    if spec.format == SAFETENSORS_SHARDED_V1:
        index = read_weight_store_index(package_dir, spec)
        for shard in index.shards:
            tensors = _read_shard(package_dir, shard)
            for rec in shard.tensors:
                yield rec.name, tensors.pop(rec.name)
        return
    with open_artifact(package_dir, spec.primary_ref, scope="weight_store",
                       artifact="npz") as (handle, st):
        if verify_digest and spec.digest:
            h = hashlib.sha256()
            for chunk in iter(lambda: handle.read(1 << 20), b""):
                h.update(chunk)
            if h.hexdigest() != spec.digest:
                raise ValueError("weight_store_npz_digest_mismatch")
            handle.seek(0)
        try:
            archive = np.load(handle, allow_pickle=False)
        except Exception as exc:
            raise ValueError("weight_store_npz_malformed") from exc
        with archive:
            for name in archive.files:
                try:
                    value = archive[name]
                except ValueError as exc:  # an object array: refused, never unpickled
                    raise ValueError("weight_store_npz_tensor_invalid") from exc
                if value.dtype.kind == "f" and value.dtype != np.float32:
                    raise ValueError("weight_store_npz_tensor_dtype_invalid")
                yield name, torch.from_numpy(np.ascontiguousarray(value))
        if not _same_file(os.fstat(handle.fileno()), st):
            raise ValueError("weight_store_npz_changed")


# ---------------------------------------------------------------------------
# Geometry and the weight set
# ---------------------------------------------------------------------------


def resolve_architecture(name) -> str:
    for key, (aliases, *_rest) in ARCHITECTURES.items():
        if name in aliases:
            return key
    if name in UNSUPPORTED_ARCHITECTURES:
        raise PackageUnsupported(f"the rocm runtime does not execute architecture {name!r}")
    raise ValueError(f"unsupported_architecture_family: {str(name).lower()}")


def rope_linear_factor(value) -> float:
    """The linear RoPE factor of a normalized ``rope_scaling``
    (``runtime_config.py:112-...``); other scaling types are refused."""
    if value is None:
        return 1.0
    if not isinstance(value, dict) or set(value) - {"rope_type", "type", "factor"}:
        raise ValueError("rope_scaling contains unsupported fields")
    kind = value.get("rope_type", value.get("type", "linear"))
    if kind != "linear":
        raise PackageUnsupported(f"rope_scaling type {kind!r} is not offered")
    factor = float(value.get("factor", 1.0))
    if not factor > 0:
        raise ValueError("rope_scaling factor must be positive")
    return factor


def geometry_from_model_config(cfg: dict, name: str = "package") -> ModelGeometry:
    """The runtime geometry of a package's ``model_config`` (the normalized form of
    ``model_definitions.py:589-627``); architecture flags from
    ``model_definitions.py:417-449``."""
    if not isinstance(cfg, dict):
        raise ValueError("package_model_config_missing")
    arch = resolve_architecture(cfg.get("architecture"))
    _aliases, shifted, qk_norm, qkv_bias = ARCHITECTURES[arch]

    def integer(*keys, default=None):
        for k in keys:
            if k in cfg:
                v = cfg[k]
                if type(v) is not int:
                    raise ValueError(f"model_config {k} must be an integer")
                return v
        if default is None:
            raise ValueError(f"model_config lacks {keys[0]}")
        return default

    hidden = integer("hidden_size")
    heads = integer("attention_heads", "num_attention_heads")
    geo = ModelGeometry(
        name=name,
        layer_count=integer("layer_count", "num_hidden_layers"),
        hidden_size=hidden,
        num_heads=heads,
        num_kv_heads=integer("num_kv_heads", "num_key_value_heads", default=heads),
        head_dim=integer("head_dim", default=hidden // heads),
        intermediate_size=integer("intermediate_size"),
        vocab_size=integer("vocab_size"),
        rms_norm_eps=float(cfg.get("rms_norm_eps", 1e-6)),
        rope_theta=float(cfg.get("rope_theta", 1000000.0)),
        qk_norm=qk_norm,
        qkv_bias=qkv_bias,
        logits_convention="dream_ar_shift" if shifted else "raw",
        mask_token_id=integer("mask_token_id"),
        eos_token_id=integer("eos_token_id", default=0),
        tie_word_embeddings=bool(cfg.get("tie_word_embeddings", False)),
        max_position_embeddings=integer("max_position_embeddings", default=40960),
        rope_scaling_factor=rope_linear_factor(cfg.get("rope_scaling")),
    )
    if min(geo.layer_count, geo.hidden_size, geo.num_heads, geo.num_kv_heads, geo.head_dim,
           geo.intermediate_size, geo.vocab_size) <= 0:
        raise ValueError("model_config dimensions must be positive")
    return geo


def expected_weight_names(g: ModelGeometry) -> frozenset:
    """The exact tensor set the forward reads: embedding, per-layer norms and
    projections (q/k/v bias exactly when the architecture declares it, q/k norms
    with qk-norm), final norm and ``lm_head.weight`` (the backend plan requires
    that key, ``graph/backend_plan.py:160-166``; tied packages store it beside the
    embedding, ``model_definitions.py:725-728``)."""
    names = {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"}
    for i in range(g.layer_count):
        p = f"model.layers.{i}."
        names.add(p + "input_layernorm.weight")
        names.add(p + "post_attention_layernorm.weight")
        for s in LINEAR_SUFFIXES:
            names.add(p + s + ".weight")
        if g.qk_norm:
            names.add(p + "self_attn.q_norm.weight")
            names.add(p + "self_attn.k_norm.weight")
        if g.qkv_bias:
            for s in ("q_proj", "k_proj", "v_proj"):
                names.add(p + f"self_attn.{s}.bias")
    return frozenset(names)


def expected_shape(g: ModelGeometry, name: str) -> tuple:
    from .synthetic import linear_shapes

    if name in ("model.embed_tokens.weight", "lm_head.weight"):
        return (g.vocab_size, g.hidden_size)
    if name == "model.norm.weight" or name.endswith("layernorm.weight"):
        return (g.hidden_size,)
    if name.endswith(("q_norm.weight", "k_norm.weight")):
        return (g.head_dim,)
    suffix = name.split(".", 3)[3]
    base, kind = suffix.rsplit(".", 1)
    n, k = linear_shapes(g)[base]
    return (n,) if kind == "bias" else (n, k)


def package_tensor_names(package_dir, spec: WeightArtifactSpec) -> frozenset:
    """The names of the tensors the weight store holds (the index's records, or
    the NPZ members), read without loading any tensor."""
    import numpy as np

    if spec.format == SAFETENSORS_SHARDED_V1:
        return read_weight_store_index(package_dir, spec).tensor_names
    with open_artifact(package_dir, spec.primary_ref, scope="weight_store",
                       artifact="npz") as (handle, _):
        try:
            with np.load(handle, allow_pickle=False) as archive:
                return frozenset(archive.files)
        except Exception as exc:
            raise ValueError("weight_store_npz_malformed") from exc


def check_tensor_names(g: ModelGeometry, names) -> None:
    """Fail closed, before any device work, when the store's tensor set is not
    exactly the one the forward reads (the converter's own check,
    ``converter/convert_hf_masked_diffusion.py:287-291``, and the bias
    declaration check of ``backends/mlx_dream.py:1880-1914``)."""
    expected = expected_weight_names(g)
    names = set(names)
    missing = sorted(expected - names)
    if missing:
        raise ValueError(f"package_weight_missing: {len(missing)} tensor(s), e.g. {missing[0]!r}")
    unexpected = sorted(names - expected)
    if unexpected:
        raise ValueError(f"package_weight_unexpected: {len(unexpected)} tensor(s), "
                         f"e.g. {unexpected[0]!r}")


def is_quantized_linear(name: str) -> bool:
    """``backends/mlx_dream.py:2040-2065``: the seven per-layer projection weights
    and ``lm_head.weight``; never embeddings, norms or biases."""
    if name == "lm_head.weight":
        return True
    return name.startswith("model.layers.") and any(
        name.endswith("." + s + ".weight") for s in LINEAR_SUFFIXES)


# ---------------------------------------------------------------------------
# Loading onto the device
# ---------------------------------------------------------------------------


@dataclass
class PackageModel:
    """A package's weights prepared on the device, in the form ``Runtime`` takes:
    bf16 tensors, and ``Q4Tensor`` bundles for the quantized linears."""

    geometry: ModelGeometry
    weight_kind: str  # "q4" or "bf16"
    weights: dict = field(default_factory=dict)
    manifest: dict = field(default_factory=dict)
    spec: WeightArtifactSpec | None = None


def read_package(package_dir):
    """Manifest, weight-store spec and geometry of a package (no tensor is read)."""
    manifest = read_manifest(package_dir)
    spec = weight_artifact_spec(manifest)
    name = str(manifest.get("model_definition_key") or manifest.get("model_descriptor_key")
               or Path(package_dir).name)
    geometry = geometry_from_model_config(manifest.get("model_config"), name=name)
    return manifest, spec, geometry


def load_package(package_dir, *, linear_quant_bits: int | None = None,
                 linear_quant_group_size: int = 64, device_ordinal: int = 0,
                 verify_digest: bool = True) -> PackageModel:
    """Read a package and prepare its weights on ``cuda:<device_ordinal>``.

    ``linear_quant_bits``: ``None`` keeps bf16 linears; ``4`` quantizes them
    (group 64 only). 8-bit quantization is a reference option this backend does
    not offer (``PackageUnsupported``)."""
    import torch

    from . import _lib

    if linear_quant_bits not in (None, 4):
        raise PackageUnsupported(f"linear_quant_bits={linear_quant_bits!r}: the rocm runtime "
                                 "runs bf16 or 4-bit linears")
    if linear_quant_bits == 4 and int(linear_quant_group_size) != 64:
        raise PackageUnsupported("4-bit linears need linear_quant_group_size=64")
    if not torch.cuda.is_available():
        raise RuntimeError("loading a package onto the rocm runtime needs a visible AMD GPU")
    lib = _lib.load()
    manifest, spec, g = read_package(package_dir)
    check_tensor_names(g, package_tensor_names(package_dir, spec))
    expected = expected_weight_names(g)
    device = torch.device("cuda", device_ordinal)
    stream = torch.cuda.current_stream(device)
    sp = C.c_void_p(stream.cuda_stream)
    q4 = linear_quant_bits == 4
    weights: dict = {}
    seen = set()
    with torch.cuda.device(device):
        for name, host in iter_package_tensors(package_dir, spec, verify_digest=verify_digest):
            if name in seen:
                raise ValueError(f"duplicate tensor name: {name!r}")
            seen.add(name)
            if name not in expected:
                raise ValueError(f"package_weight_unexpected: {name!r}")
            shape = expected_shape(g, name)
            if tuple(host.shape) != shape:
                raise ValueError(f"package_weight_shape_mismatch: {name!r} "
                                 f"{tuple(host.shape)} != {shape}")
            if host.dtype not in (torch.float32, torch.bfloat16):
                raise PackageUnsupported(f"{name!r}: {host.dtype} package tensors are not "
                                         "supported (float32 or bfloat16)")
            src = host.contiguous().to(device)
            if q4 and is_quantized_linear(name):
                n, k = shape
                w_q = torch.empty((n, k // 8), dtype=torch.int32, device=device)
                scales = torch.empty((n, k // 64), dtype=torch.bfloat16, device=device)
                biases = torch.empty((n, k // 64), dtype=torch.bfloat16, device=device)
                _lib.check(lib.drt_op_q4_quantize(
                    src.data_ptr(), _lib.F32 if src.dtype == torch.float32 else _lib.BF16, n, k,
                    w_q.data_ptr(), scales.data_ptr(), biases.data_ptr(), sp))
                weights[name] = Q4Tensor(w_q, scales, biases)
            elif src.dtype == torch.float32:
                out = torch.empty(shape, dtype=torch.bfloat16, device=device)
                _lib.check(lib.drt_op_cast_bf16(src.data_ptr(), out.data_ptr(), src.numel(), sp))
                weights[name] = out
            else:
                weights[name] = src
            stream.synchronize()  # the fp source is released before the next tensor
            del src, host
    missing = sorted(expected - seen)
    if missing:
        raise ValueError(f"package_weight_missing: {len(missing)} tensor(s), e.g. {missing[0]!r}")
    return PackageModel(geometry=g, weight_kind="q4" if q4 else "bf16", weights=weights,
                        manifest=manifest, spec=spec)
