"""Per-op kernel table on device tensors (the reference's ``KernelTable`` seam).

Signatures follow ``backends/kernel_table.py:118-126`` / ``backends/mlx_ops.py``
of the reference's ``python/src/edllm/``:

    rms_norm(x, weight, eps)
    linear(x, weight, bias=None)          # weight: DeviceQ4Weight | DeviceBF16Weight
    rope(x[rows, H, hd], cos[rows, 1, hd], sin[rows, 1, hd])
    swiglu(gate, up)
    attention(q[rq, Hq, hd], k[rk, Hkv, hd], v, *, head_dim, kind,
              mask_geometry=None, q_positions=None) -> [rq, Hq*hd]

Every op runs a HIP kernel of ``libdrt_rocm.so`` on the tensors' device and
current torch stream. Validation raises ``ValueError`` before any launch, like
the reference's fail-closed checks.
"""
from __future__ import annotations

import ctypes as C
import math

from . import _lib

KV_TILE_ELEMS = 8192  # one 32-key tile: K block + V block, 2-byte elements


def _torch():
    import torch

    return torch


def _stream(t):
    torch = _torch()
    return C.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t) -> C.c_void_p:
    return C.c_void_p(t.data_ptr())


def _require_cuda(*tensors):
    for t in tensors:
        if t is not None and (not t.is_cuda or not t.is_contiguous()):
            raise ValueError("kernel table ops take contiguous device tensors")


class DeviceQ4Weight:
    """A q4 g64 affine linear weight repacked into the device tile layout.

    Built once from an MLX-packed ``QuantizedWeight`` (``w_q`` uint32 ``[N, K/8]``
    as int32, ``scales``/``biases`` bf16 ``[N, K/64]``; ``mlx_ops.py:43-60``)."""

    def __init__(self, w_q, scales, biases):
        torch = _torch()
        _require_cuda(w_q, scales, biases)
        n, kw = w_q.shape
        k = kw * 8
        if scales.shape != (n, k // 64) or biases.shape != (n, k // 64):
            raise ValueError("scales/biases must be [N, K/64]")
        if w_q.dtype != torch.int32 or scales.dtype != torch.bfloat16 or biases.dtype != torch.bfloat16:
            raise ValueError("q4 weight needs int32 words and bf16 scales/biases")
        self.shape = (int(n), int(k))
        self.qw = torch.empty(n * k // 8, dtype=torch.int32, device=w_q.device)
        self.sb = torch.empty(n * (k // 64), dtype=torch.int32, device=w_q.device)
        _lib.check(_lib.load().drt_op_q4_repack(_ptr(w_q), _ptr(scales), _ptr(biases), n, k,
                                                _ptr(self.qw), _ptr(self.sb), _stream(w_q)))


class DeviceBF16Weight:
    """A bf16 ``[N, K]`` linear weight repacked into the device tile layout."""

    def __init__(self, w):
        torch = _torch()
        _require_cuda(w)
        if w.dtype != torch.bfloat16 or w.dim() != 2:
            raise ValueError("bf16 weight must be a 2-D bfloat16 tensor")
        n, k = w.shape
        self.shape = (int(n), int(k))
        self.wb = torch.empty_like(w)
        _lib.check(_lib.load().drt_op_bf16_repack(_ptr(w), n, k, _ptr(self.wb), _stream(w)))


def linear(x, weight, bias=None):
    """``x @ W.T (+ bias)`` with the reference's dtype rules (``mlx_ops.py:97-130``).

    q4: fp32 (or bf16) x -> fp32 y. bf16 weight: ``bf16(bf16(x) @ W.T)`` as fp32."""
    torch = _torch()
    _require_cuda(x, bias)
    lib = _lib.load()
    n, k = weight.shape
    if x.dim() != 2 or x.shape[1] != k:
        raise ValueError(f"linear x must be [M, {k}]")
    m = x.shape[0]
    y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.shape != (n,)):
        raise ValueError("linear bias must be bf16 [N]")
    bptr = _ptr(bias) if bias is not None else None
    if isinstance(weight, DeviceQ4Weight):
        if x.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("q4 linear x must be fp32 or bf16")
        ws_bytes = lib.drt_op_q4_linear_workspace_bytes(m, n, k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        _lib.check(lib.drt_op_q4_linear(_ptr(weight.qw), _ptr(weight.sb), _ptr(x),
                                        _lib.BF16 if x.dtype == torch.bfloat16 else _lib.F32,
                                        m, n, k, bptr, _ptr(y), _ptr(ws), ws_bytes, _stream(x)))
    elif isinstance(weight, DeviceBF16Weight):
        xb = x.to(torch.bfloat16).contiguous()
        ws_bytes = lib.drt_op_bf16_linear_workspace_bytes(m, n, k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
        _lib.check(lib.drt_op_bf16_linear(_ptr(weight.wb), _ptr(xb), m, n, k, bptr, _ptr(y),
                                          _ptr(ws), ws_bytes, _stream(x)))
    else:
        raise ValueError("linear weight must be a DeviceQ4Weight or DeviceBF16Weight")
    return y


def rms_norm(x, weight, eps: float):
    """fp32 RMSNorm over the last axis with a bf16 weight (``mlx_ops.py:21-35``)."""
    torch = _torch()
    _require_cuda(x, weight)
    if x.dtype != torch.float32 or weight.dtype != torch.bfloat16:
        raise ValueError("rms_norm takes fp32 x and a bf16 weight")
    d = x.shape[-1]
    if weight.shape != (d,):
        raise ValueError("rms_norm weight must match the last axis")
    y = torch.empty_like(x)
    rows = x.numel() // d
    _lib.check(_lib.load().drt_op_rms_norm(_ptr(x), _ptr(weight), float(eps), _ptr(y), rows, d,
                                           _stream(x)))
    return y


def rope(x, cos, sin):
    """Split-half RoPE on fp32 ``x [rows, H, hd]`` with ``cos/sin [rows, 1, hd]``."""
    torch = _torch()
    _require_cuda(x)
    rows, h, hd = x.shape
    c = cos.reshape(rows, hd).to(device=x.device, dtype=torch.float32).contiguous()
    s = sin.reshape(rows, hd).to(device=x.device, dtype=torch.float32).contiguous()
    y = torch.empty_like(x)
    _lib.check(_lib.load().drt_op_rope(_ptr(x), _ptr(c), _ptr(s), _ptr(y), rows, h, hd,
                                       _stream(x)))
    return y


def swiglu(gate, up):
    """``silu(gate) * up`` in fp32 (``mlx_ops.py:147-154``)."""
    torch = _torch()
    _require_cuda(gate, up)
    if gate.shape != up.shape or gate.dtype != torch.float32 or up.dtype != torch.float32:
        raise ValueError("swiglu takes two fp32 tensors of one shape")
    y = torch.empty_like(gate)
    _lib.check(_lib.load().drt_op_swiglu(_ptr(gate), _ptr(up), _ptr(y), gate.numel(), _stream(gate)))
    return y


class PrefixKVCache:
    """Tiled K/V cache for ``layers`` layers on one device.

    The build's prefix-cache object: rows are written once (``store``) at
    absolute positions and read by :meth:`attention`. Layout per (layer, kv
    head): 32-key tiles of 8192 elements (K block then V block) in the MFMA
    operand order of the attention kernel. Unwritten slots stay zero."""

    def __init__(self, layers: int, kv_heads: int, capacity: int, *, dtype="f16", device=None):
        torch = _torch()
        self.layers, self.kv_heads = int(layers), int(kv_heads)
        self.tiles = (int(capacity) + 31) // 32
        self.capacity = self.tiles * 32
        self.head_stride = self.tiles * KV_TILE_ELEMS
        self.kv_dtype = _lib.BF16 if dtype == "bf16" else _lib.F16
        tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
        self.data = torch.zeros((self.layers, self.kv_heads, self.head_stride), dtype=tdt,
                                device=device or "cuda")
        self.length = 0

    @property
    def nbytes(self) -> int:
        return self.data.numel() * self.data.element_size()

    def store(self, layer: int, k, v, pos0: int) -> None:
        """Write ``k/v [n, Hkv, 128]`` (fp32 or bf16) at positions ``pos0..pos0+n-1``."""
        torch = _torch()
        _require_cuda(k, v)
        n = k.shape[0]
        if k.shape != v.shape or k.shape[1:] != (self.kv_heads, 128):
            raise ValueError("store takes k, v of shape [n, kv_heads, 128]")
        if pos0 < 0 or pos0 + n > self.capacity:
            raise ValueError("store positions exceed the cache capacity")
        if k.dtype not in (torch.float32, torch.bfloat16) or v.dtype != k.dtype:
            raise ValueError("store takes fp32 or bf16 k/v")
        src = _lib.BF16 if k.dtype == torch.bfloat16 else _lib.F32
        layer_view = self.data[layer]
        _lib.check(_lib.load().drt_op_kv_pack(_ptr(k), _ptr(v), src, n, self.kv_heads, pos0,
                                              _ptr(layer_view), self.head_stride, self.kv_dtype,
                                              _stream(k)))
        self.length = max(self.length, pos0 + n)

    def attention(self, layer: int, q, *, n_keys: int, row_pos0: int, kind: str,
                  mask_geometry=None, out_dtype=None):
        """Attention of ``q [rows, Hq, 128]`` (cache dtype) over keys ``[0, n_keys)``."""
        torch = _torch()
        _require_cuda(q)
        rows, hq, hd = q.shape
        if hd != 128 or hq % self.kv_heads:
            raise ValueError("attention needs head_dim 128 and Hq % Hkv == 0")
        if n_keys < 1 or n_keys > self.capacity:
            raise ValueError("n_keys outside the cache")
        want = torch.bfloat16 if self.kv_dtype == _lib.BF16 else torch.float16
        if q.dtype != want:
            raise ValueError(f"q must be {want} to match the cache")
        mk, p, b = _mask_args(kind, mask_geometry)
        out_dtype = out_dtype or torch.float32
        odt = _lib.F32 if out_dtype == torch.float32 else _lib.BF16
        out = torch.empty((rows, hq * 128), dtype=out_dtype, device=q.device)
        lib = _lib.load()
        ws_bytes = lib.drt_op_attention_workspace_bytes(rows, hq, self.kv_heads, n_keys)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        _lib.check(lib.drt_op_attention(_ptr(q), _ptr(self.data[layer]), self.head_stride,
                                        self.kv_dtype, rows, hq, self.kv_heads, n_keys, row_pos0,
                                        mk, p, b, _ptr(out), odt, _ptr(ws), ws_bytes, _stream(q)))
        return out


def _mask_args(kind, mask_geometry):
    if kind in ("full", "bidirectional"):
        if mask_geometry is not None:
            raise ValueError("mask geometry is only consumed by the d2f_hybrid kind")
        return _lib.MASK_BIDIRECTIONAL, 0, 1
    if kind == "d2f_hybrid":
        if mask_geometry is None:
            raise ValueError("d2f_hybrid requires mask geometry")
        if isinstance(mask_geometry, dict):
            p, b = int(mask_geometry["prompt_len"]), int(mask_geometry["block_size"])
        else:
            p, b = (int(v) for v in mask_geometry)
        if p < 0 or b < 1:
            raise ValueError("bad d2f_hybrid mask geometry")
        return _lib.MASK_D2F_HYBRID, p, b
    raise ValueError(f"unsupported attention mask kind: {kind}")


def attention(q, k, v, *, head_dim: int, kind: str, mask_geometry=None, q_positions=None,
              kv_dtype: str = "bf16"):
    """Reference-signature attention (``mlx_ops.py:347-443``) via a temporary cache.

    ``q_positions`` (absolute positions of the q rows) must be contiguous; by
    default q rows are the last ``rq`` positions of the ``rk`` keys. The output
    dtype follows ``q`` like the reference's ``.astype(out_dtype)``."""
    torch = _torch()
    if head_dim != 128:
        raise ValueError("attention head_dim must be 128")
    rq, hq, _ = q.shape
    rk, hkv, _ = k.shape
    if k.shape != v.shape:
        raise ValueError(f"attention K/V shapes disagree: {tuple(k.shape)} != {tuple(v.shape)}")
    if hq % hkv:
        raise ValueError("attention query heads must be divisible by compact K/V heads")
    if q_positions is None:
        pos0 = rk - rq
        if pos0 < 0:
            raise ValueError("more query rows than keys needs explicit q_positions")
    else:
        qp = [int(p) for p in q_positions]
        if len(qp) != rq or any(b - a != 1 for a, b in zip(qp, qp[1:])):
            raise ValueError("q_positions must be one contiguous run per query row")
        pos0 = qp[0]
        if pos0 < 0 or qp[-1] >= rk:
            raise ValueError("q_positions outside the kv range")
    cache = PrefixKVCache(1, hkv, rk, dtype=kv_dtype, device=q.device)
    kd = k if k.dtype in (torch.float32, torch.bfloat16) else k.float()
    vd = v if v.dtype == kd.dtype else v.to(kd.dtype)
    cache.store(0, kd.contiguous(), vd.contiguous(), 0)
    qc = q.to(torch.bfloat16 if kv_dtype == "bf16" else torch.float16).contiguous()
    out = cache.attention(0, qc, n_keys=rk, row_pos0=pos0, kind=kind, mask_geometry=mask_geometry,
                          out_dtype=torch.float32)
    return out.to(q.dtype)


KERNEL_OP_NAMES = ("rms_norm", "linear", "rope", "swiglu", "attention")


class KernelTable:
    """The op table a forward dispatches through (``kernel_table.py:118-126``)."""

    backend = "rocm"
    rms_norm = staticmethod(rms_norm)
    linear = staticmethod(linear)
    rope = staticmethod(rope)
    swiglu = staticmethod(swiglu)
    attention = staticmethod(attention)
