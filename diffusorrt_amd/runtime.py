"""The ``rocm`` device runtime: Python surface over ``libdrt_rocm.so``.

Mirrors the compiled-provider contract the reference's host code drives
(``model.py:873-920, 1026-1087`` and ``backends/device_runtime.py:108-183,
277-365`` of the reference's ``python/src/edllm/``):

    runtime = Runtime(package_dir_or_model, engine_config={...})
    with runtime.session(session_config={...}) as session:
        session.start_device(tokens, prompt_len=..., block_size=..., mask_token_id=...,
                             exact_kv=False, steps=..., memory_budget_bytes=0,
                             temperature=0.0, seed=0)
        scores, tokens, forwarded = session.propose_device(frontier, window_end=...,
                                                           frozen_prefix=...)
        session.commit_device(positions, tokens)
        window = session.execute_window(token_ids, scope, mask_geometry=(p, b))
        session.device_metrics()

PyTorch is only the plumbing that puts the weights in device memory; all
compute happens in the library's HIP kernels. As in the reference, the runtime
opens an execution-package directory (``package.load_package``: manifest,
verified weight store, bf16 cast and 4-bit quantization on the device when
``engine_config["linear_quant_bits"] == 4``); it also takes a prepared model
object (``geometry``, ``weight_kind``, ``weights``: the seeded synthetic models).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from .abi import AttentionMaskKind, CommitPolicy, DecodeStrategy
from .synthetic import LINEAR_SUFFIXES, ModelGeometry, Q4Tensor, SyntheticModel

_TORCH_DTYPES = None


def _dtype_code(t) -> int:
    import torch

    table = {torch.float32: _lib.F32, torch.float64: _lib.F64, torch.bfloat16: _lib.BF16,
             torch.int32: _lib.I32, torch.int64: _lib.I64, torch.uint8: _lib.U8,
             torch.float16: _lib.F16}
    try:
        return table[t.dtype]
    except KeyError:
        raise ValueError(f"dtype {t.dtype} has no ABI encoding") from None


def rope_tables(positions: int, head_dim: int, rope_theta: float, factor: float = 1.0):
    """Half-width fp32 rotary tables ``[positions, head_dim/2]``.

    Same float32 recipe as the reference's ``_rope_tables``
    (``backends/mlx_forward.py:1566-1595``): ``inv_freq = 1 / theta **
    (arange(0, half, f32) / half) / max(1e-6, factor)`` (linear scaling),
    ``freqs = pos * inv_freq``; the kernels duplicate the halves.
    """
    half = head_dim // 2
    inv_freq = np.float32(1.0) / (
        np.float32(rope_theta) ** (np.arange(0, half, dtype=np.float32) / np.float32(half)))
    inv_freq = (inv_freq / np.float32(max(1e-6, float(factor)))).astype(np.float32)
    freqs = (np.arange(positions, dtype=np.float32)[:, None] * inv_freq[None, :]).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


@dataclass
class WindowLogits:
    """``execute_window`` result (``backends/device_runtime.py:354-363``)."""

    logits: bytes  # '<f4' [n_rows * n_vocab]
    n_rows: int
    n_vocab: int
    forwarded_rows: int

    def array(self) -> np.ndarray:
        return np.frombuffer(self.logits, dtype="<f4").reshape(self.n_rows, self.n_vocab)


def engine_request(engine_config: dict, weight_kind: str) -> tuple:
    """Validate an engine request (``EngineConfig``, ``abi/lifetimes.py:30-43``) for
    weights of ``weight_kind``; returns ``(linear_quant_bits, d2f_exact_kv_cache)``.

    ``d2f_exact_kv_cache = 1`` is what ``cuda_engine_config(precision,
    exact_kv=True)`` sends for Dream's block_threshold (``model.py:905-916, 991``;
    ``backends/device_runtime.py:53-58``): accepted, since this runtime's
    block_threshold sessions always run over the exact prompt + frozen-block K/V;
    fixed-quota sessions refuse ``exact_kv`` at ``start_device``. The approximate,
    cross-request and canvas caches are not offered.
    """
    ec = dict(engine_config or {})
    quant_bits = 4 if weight_kind == "q4" else -1
    bits = ec.get("linear_quant_bits", quant_bits)
    if (-1 if bits is None else bits) != quant_bits:
        raise ValueError("engine_config linear_quant_bits disagrees with the weights")
    for key in ("prefix_kv_cache", "block_kv_cache", "layer0_kv_cache_enabled",
                "cross_request_cache", "canvas_cache"):
        if int(ec.get(key, 0)):
            raise ValueError(f"engine_config {key} is not offered by the rocm runtime")
    exact_kv_cache = ec.get("d2f_exact_kv_cache", 0)
    if exact_kv_cache not in (0, 1):
        raise ValueError("engine_config d2f_exact_kv_cache must be 0 or 1")
    if int(ec.get("compute_dtype", 0)) != 0:
        raise ValueError("engine_config compute_dtype must be 0 (bf16)")
    return quant_bits, int(exact_kv_cache)


class Runtime:
    """Owns the model in device layouts and one HIP stream (one per process is typical)."""

    def __init__(self, model, *, device: str = "rocm",
                 engine_config: dict | None = None, precision: dict | None = None,
                 device_ordinal: int = 0, creation_memory_budget_bytes: int = 0,
                 max_forward_rows: int = 2048, kv_dtype: str = "f16",
                 max_positions: int | None = None):
        import os

        import torch

        if device != "rocm":
            raise ValueError(f"this runtime serves device='rocm', not {device!r}")
        if not torch.cuda.is_available():
            raise RuntimeError("the rocm runtime needs a visible AMD GPU")
        lib = _lib.load()
        ec = dict(engine_config or {})
        if isinstance(model, (str, os.PathLike)):
            # an execution-package directory (model.py:888-920): weights read,
            # cast and quantized on the device as the engine config asks
            from .package import load_package

            bits = ec.get("linear_quant_bits")
            model = load_package(model, linear_quant_bits=None if bits in (None, -1) else int(bits),
                                 linear_quant_group_size=int(ec.get("linear_quant_group_size", 64)),
                                 device_ordinal=device_ordinal)
        g: ModelGeometry = model.geometry
        quant_bits, exact_kv_cache = engine_request(ec, model.weight_kind)
        self.d2f_exact_kv_cache = bool(exact_kv_cache)
        self.geometry = g
        self.weight_kind = model.weight_kind
        self._device = torch.device("cuda", device_ordinal)
        positions = int(max_positions or g.max_position_embeddings)
        self._engine = _lib.EngineConfig(
            compute_dtype=0, linear_quant_bits=quant_bits,
            linear_quant_group_size=64, window_exec=0, device_ordinal=device_ordinal,
            max_forward_rows=int(max_forward_rows),
            kv_dtype=_lib.BF16 if kv_dtype == "bf16" else _lib.F16,
            d2f_exact_kv_cache=exact_kv_cache,
            creation_memory_budget_bytes=int(creation_memory_budget_bytes))
        self._geo = _lib.ModelGeometry(
            layer_count=g.layer_count, hidden_size=g.hidden_size, num_heads=g.num_heads,
            num_kv_heads=g.num_kv_heads, vocab_size=g.vocab_size,
            max_position_embeddings=positions, head_dim=g.head_dim,
            intermediate_size=g.intermediate_size, rms_norm_eps=g.rms_norm_eps,
            rope_theta=g.rope_theta, qk_norm=int(g.qk_norm), qkv_bias=int(g.qkv_bias),
            logits_convention=(_lib.LOGITS_DREAM_AR_SHIFT if g.logits_convention == "dream_ar_shift"
                               else _lib.LOGITS_RAW))
        keep = []  # device tensors borrowed for the duration of drt_runtime_create
        descs = []

        def add(name, tensor):
            t = tensor.to(self._device).contiguous()
            keep.append(t)
            d = _lib.Tensor()
            d.name = name.encode()
            d.data = t.data_ptr()
            d.dtype = _dtype_code(t)
            d.ndim = t.dim()
            for i, s in enumerate(t.shape):
                d.shape[i] = int(s)
            descs.append(d)

        for name, value in model.weights.items():
            if isinstance(value, Q4Tensor):
                base = name[: -len(".weight")]
                add(base + ".weight", value.w_q)
                add(base + ".scales", value.scales)
                add(base + ".biases", value.biases)
            else:
                add(name, value)
        cos, sin = rope_tables(positions, g.head_dim, g.rope_theta,
                               getattr(g, "rope_scaling_factor", 1.0))
        add("rope.cos", torch.from_numpy(cos))
        add("rope.sin", torch.from_numpy(sin))
        arr = (_lib.Tensor * len(descs))(*descs)
        handle = C.c_uint64(0)
        torch.cuda.synchronize(self._device)
        _lib.check(lib.drt_runtime_create(C.byref(self._engine), C.byref(self._geo), arr,
                                          len(descs), C.byref(handle)))
        del keep
        self._handle = handle.value
        self._lib = lib

    @property
    def handle(self) -> int:
        if not self._handle:
            raise RuntimeError("runtime is closed")
        return self._handle

    def session(self, session_config: dict) -> "DeviceSession":
        """``runtime.session(session_config={decode_strategy, commit_policy,
        attention_mask_kind, block_size, steps, max_tokens})``; a context manager."""
        sc = _lib.SessionConfig(
            decode_strategy=int(session_config.get("decode_strategy", -1)),
            commit_policy=int(session_config.get("commit_policy", int(CommitPolicy.FIXED_QUOTA))),
            attention_mask_kind=int(session_config.get("attention_mask_kind", 0)),
            block_size=int(session_config.get("block_size", 0)),
            steps=int(session_config.get("steps", 0)),
            max_tokens=int(session_config.get("max_tokens", 0)),
            trace_canvas=int(session_config.get("trace_canvas", 0)),
            error_fixing=int(session_config.get("error_fixing", 0)))
        reserved = tuple(session_config.get("reserved", (0,) * 8))
        if len(reserved) != 8:
            raise ValueError("session_config reserved holds 8 ints")
        for i, v in enumerate(reserved):
            sc.reserved[i] = int(v)
        out = C.c_uint64(0)
        _lib.check(self._lib.drt_session_open(self.handle, C.byref(sc), C.byref(out)))
        return DeviceSession(self, out.value, sc)

    def close(self) -> None:
        if self._handle:
            h, self._handle = self._handle, 0
            _lib.check(self._lib.drt_release_handle(h))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceSession:
    """One request on the device; scores stay on the device, only
    (scores, tokens) of the frontier cross to the host per proposal."""

    def __init__(self, runtime: Runtime, handle: int, config):
        self._rt = runtime
        self._handle = handle
        self._config = config
        self._lib = runtime._lib
        self.vocab_size = runtime.geometry.vocab_size

    @property
    def handle(self) -> int:
        if not self._handle:
            raise RuntimeError("session is closed")
        return self._handle

    def start_device(self, tokens, *, prompt_len: int, block_size: int, mask_token_id: int,
                     exact_kv: bool, steps: int, memory_budget_bytes: int = 0,
                     temperature: float = 0.0, seed: int = 0) -> None:
        toks = _lib.i32_array(tokens)
        self._canvas_len = len(tokens)
        _lib.check(self._lib.drt_session_start(
            self.handle, toks, len(tokens), int(prompt_len), int(block_size), int(mask_token_id),
            int(bool(exact_kv)), int(steps), int(memory_budget_bytes), float(temperature),
            int(seed) & ((1 << 64) - 1)))

    def propose_device(self, frontier, *, window_end: int, frozen_prefix: int):
        n = len(frontier)
        scores = (C.c_double * n)()
        tokens = (C.c_int32 * n)()
        fwd = C.c_int32(0)
        _lib.check(self._lib.drt_session_propose(
            self.handle, _lib.i32_array(frontier), n, int(window_end), int(frozen_prefix),
            scores, tokens, C.byref(fwd)))
        return list(scores), [int(t) for t in tokens], int(fwd.value)

    def commit_device(self, positions, tokens) -> None:
        if len(positions) != len(tokens):
            raise ValueError("commit_device needs one token per position")
        _lib.check(self._lib.drt_session_commit(
            self.handle, _lib.i32_array(positions), _lib.i32_array(tokens), len(positions)))

    def bd3_decode(self, *, prompt_len: int, max_tokens: int, steps: int, eos_token_id: int,
                   requires_prompt_block_alignment: bool = True, max_forwards: int) -> tuple:
        """Run up to ``max_forwards`` steps of the BD3 fixed-quota loop natively (the
        policy state persists in the session between calls). Returns
        ``(forwards, committed, done)``."""
        fwd, com, done = C.c_int32(0), C.c_int32(0), C.c_int32(0)
        _lib.check(self._lib.drt_session_bd3_decode(
            self.handle, int(prompt_len), int(max_tokens), int(steps), int(eos_token_id),
            int(bool(requires_prompt_block_alignment)), int(max_forwards), C.byref(fwd),
            C.byref(com), C.byref(done)))
        return fwd.value, com.value, bool(done.value)

    def canvas(self) -> list:
        """The session's canvas (prompt + generated positions, as committed)."""
        n = int(self._canvas_len)
        out = (C.c_int32 * max(1, n))()
        size = C.c_int32(0)
        _lib.check(self._lib.drt_session_canvas(self.handle, out, n, C.byref(size)))
        return list(out[:size.value])

    def execute_window(self, token_ids, scope, mask_geometry=None) -> WindowLogits:
        n_scope = len(scope)
        out = np.empty((n_scope, self.vocab_size), dtype=np.float32)
        n_vocab = C.c_int32(0)
        fwd = C.c_int32(0)
        p, b = (mask_geometry if mask_geometry is not None else (0, 0))
        _lib.check(self._lib.drt_session_execute_window(
            self.handle, _lib.i32_array(token_ids), len(token_ids), _lib.i32_array(scope), n_scope,
            int(p), int(b), out.ctypes.data_as(C.POINTER(C.c_float)), out.size,
            C.byref(n_vocab), C.byref(fwd)))
        return WindowLogits(logits=out.tobytes(), n_rows=n_scope, n_vocab=int(n_vocab.value),
                            forwarded_rows=int(fwd.value))

    def device_metrics(self) -> dict:
        m = _lib.Metrics()
        _lib.check(self._lib.drt_session_metrics(self.handle, C.byref(m)))
        out = {}
        for name, _ in _lib.Metrics._fields_:
            v = getattr(m, name)
            if name.startswith("prof_"):
                for i, cls in enumerate(("attention", "linear", "lm_head", "attention_combine")):
                    out[f"rocm_{name}_{cls}"] = v[i]
            else:
                out["rocm_" + name] = v
        return out

    def set_profiling(self, enable: bool) -> None:
        """Time each attention / range-combine / linear / LM-head dispatch (dispatch
        timestamps)."""
        _lib.check(self._lib.drt_session_set_profiling(self.handle, int(bool(enable))))

    def close(self) -> None:
        if self._handle:
            h, self._handle = self._handle, 0
            _lib.check(self._lib.drt_release_handle(h))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def bd3_session_config(block_size: int, steps: int, max_tokens: int) -> dict:
    return {"decode_strategy": int(DecodeStrategy.BD3_FIXED_QUOTA),
            "commit_policy": int(CommitPolicy.FIXED_QUOTA),
            "attention_mask_kind": int(AttentionMaskKind.D2F_HYBRID),
            "block_size": block_size, "steps": steps, "max_tokens": max_tokens}


def block_threshold_session_config(block_size: int, steps: int, max_tokens: int) -> dict:
    return {"decode_strategy": int(DecodeStrategy.BLOCK_THRESHOLD),
            "commit_policy": int(CommitPolicy.THRESHOLD),
            "attention_mask_kind": int(AttentionMaskKind.D2F_HYBRID),
            "block_size": block_size, "steps": steps, "max_tokens": max_tokens}


def fixed_quota_session_config(block_size: int, steps: int, max_tokens: int) -> dict:
    return {"decode_strategy": int(DecodeStrategy.FIXED_QUOTA),
            "commit_policy": int(CommitPolicy.FIXED_QUOTA),
            "attention_mask_kind": int(AttentionMaskKind.BIDIRECTIONAL),
            "block_size": block_size, "steps": steps, "max_tokens": max_tokens}
