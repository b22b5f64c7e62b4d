"""ctypes binding of ``libdrt_rocm.so`` (the C-ABI declared in include/drt_rocm.h).

The library is loaded from this package directory only. There is no fallback:
when it is missing, every call raises :class:`LibraryNotBuilt`.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdrt_rocm.so"

# AbiStatus (abi/forward.py:20-26 in the reference)
OK, VERSION_MISMATCH, INVALID_ARGUMENT, UNSUPPORTED, INTERNAL_ERROR = range(5)
STATUS_NAMES = {OK: "OK", VERSION_MISMATCH: "VERSION_MISMATCH",
                INVALID_ARGUMENT: "INVALID_ARGUMENT", UNSUPPORTED: "UNSUPPORTED",
                INTERNAL_ERROR: "INTERNAL_ERROR"}
# DType (abi/buffers.py:22-28) + F16
F32, F64, BF16, I32, I64, U8, F16 = range(7)
MASK_BIDIRECTIONAL, MASK_D2F_HYBRID, MASK_FULL = range(3)
LOGITS_RAW, LOGITS_DREAM_AR_SHIFT = range(2)


class LibraryNotBuilt(RuntimeError):
    pass


class AbiError(RuntimeError):
    """A non-OK AbiStatus from the native library."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class AbiInvalidArgument(AbiError, ValueError):
    pass


class AbiUnsupported(AbiError, NotImplementedError):
    pass


class EngineConfig(C.Structure):
    _fields_ = [("compute_dtype", C.c_int32), ("linear_quant_bits", C.c_int32),
                ("linear_quant_group_size", C.c_int32), ("layer0_kv_cache_enabled", C.c_int32),
                ("prefix_kv_cache", C.c_int32), ("block_kv_cache", C.c_int32),
                ("d2f_exact_kv_cache", C.c_int32), ("cross_request_cache", C.c_int32),
                ("canvas_cache", C.c_int32), ("canvas_cache_budget_bytes", C.c_int64),
                ("window_exec", C.c_int32), ("device_ordinal", C.c_int32),
                ("max_forward_rows", C.c_int32), ("kv_dtype", C.c_int32),
                ("creation_memory_budget_bytes", C.c_int64)]


class ModelGeometry(C.Structure):
    _fields_ = [("layer_count", C.c_int32), ("hidden_size", C.c_int32),
                ("num_heads", C.c_int32), ("num_kv_heads", C.c_int32),
                ("vocab_size", C.c_int32), ("max_position_embeddings", C.c_int32),
                ("head_dim", C.c_int32), ("intermediate_size", C.c_int32),
                ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float),
                ("qk_norm", C.c_int32), ("qkv_bias", C.c_int32),
                ("logits_convention", C.c_int32)]


class SessionConfig(C.Structure):
    _fields_ = [("decode_strategy", C.c_int32), ("commit_policy", C.c_int32),
                ("attention_mask_kind", C.c_int32), ("block_size", C.c_int32),
                ("steps", C.c_int32), ("max_tokens", C.c_int32),
                ("trace_canvas", C.c_int32), ("error_fixing", C.c_int32),
                ("reserved", C.c_int32 * 8)]


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("dtype", C.c_int32),
                ("ndim", C.c_int32), ("shape", C.c_int64 * 4)]


class Metrics(C.Structure):
    _fields_ = [("forward_count", C.c_int64), ("active_rows", C.c_int64),
                ("commit_rows", C.c_int64), ("lm_rows", C.c_int64),
                ("kv_cache_len", C.c_int64), ("kv_cache_bytes", C.c_int64),
                ("last_forward_ms", C.c_double), ("total_forward_ms", C.c_double),
                ("prof_ms", C.c_double * 4), ("prof_bytes", C.c_double * 4),
                ("prof_launches", C.c_int64 * 4)]


_VP, _I32, _I64, _U64, _SZ = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_size_t
_PI32, _PF64, _PF32 = C.POINTER(C.c_int32), C.POINTER(C.c_double), C.POINTER(C.c_float)

# name -> (restype, argtypes); the complete export list of include/drt_rocm.h
SIGNATURES = {
    "drt_abi_version": (None, [_PI32, _PI32, _PI32]),
    "drt_last_error": (_SZ, [C.c_char_p, _SZ]),
    "drt_release_handle": (_I32, [_U64]),
    "drt_runtime_create": (_I32, [C.POINTER(EngineConfig), C.POINTER(ModelGeometry),
                                  C.POINTER(Tensor), _I32, C.POINTER(C.c_uint64)]),
    "drt_session_open": (_I32, [_U64, C.POINTER(SessionConfig), C.POINTER(C.c_uint64)]),
    "drt_session_start": (_I32, [_U64, _PI32, _I32, _I32, _I32, _I32, _I32, _I32, _I64,
                                 C.c_double, _U64]),
    "drt_session_propose": (_I32, [_U64, _PI32, _I32, _I32, _I32, _PF64, _PI32, _PI32]),
    "drt_session_commit": (_I32, [_U64, _PI32, _PI32, _I32]),
    "drt_session_bd3_decode": (_I32, [_U64, _I32, _I32, _I32, _I32, _I32, _I32, _PI32, _PI32,
                                      _PI32]),
    "drt_session_canvas": (_I32, [_U64, _PI32, _I32, _PI32]),
    "drt_session_execute_window": (_I32, [_U64, _PI32, _I32, _PI32, _I32, _I32, _I32, _PF32,
                                          _I64, _PI32, _PI32]),
    "drt_session_metrics": (_I32, [_U64, C.POINTER(Metrics)]),
    "drt_session_set_profiling": (_I32, [_U64, _I32]),
    "drt_op_q4_repack": (_I32, [_VP, _VP, _VP, _I32, _I32, _VP, _VP, _VP]),
    "drt_op_q4_quantize": (_I32, [_VP, _I32, _I32, _I32, _VP, _VP, _VP, _VP]),
    "drt_op_cast_bf16": (_I32, [_VP, _VP, _I64, _VP]),
    "drt_op_q4_linear_workspace_bytes": (_SZ, [_I32, _I32, _I32]),
    "drt_op_q4_linear": (_I32, [_VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _VP, _VP, _SZ,
                                _VP]),
    "drt_op_q4_linear_noalloc": (_I32, [_VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _VP, _VP]),
    "drt_op_bf16_repack": (_I32, [_VP, _I32, _I32, _VP, _VP]),
    "drt_op_bf16_linear_workspace_bytes": (_SZ, [_I32, _I32, _I32]),
    "drt_op_bf16_linear": (_I32, [_VP, _VP, _I32, _I32, _I32, _VP, _VP, _VP, _SZ, _VP]),
    "drt_op_kv_pack": (_I32, [_VP, _VP, _I32, _I32, _I32, _I32, _VP, _I64, _I32, _VP]),
    "drt_op_attention_workspace_bytes": (_SZ, [_I32, _I32, _I32, _I32]),
    "drt_op_attention": (_I32, [_VP, _VP, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                _I32, _VP, _I32, _VP, _SZ, _VP]),
    "drt_op_rms_norm": (_I32, [_VP, _VP, C.c_float, _VP, _I32, _I32, _VP]),
    "drt_op_rope": (_I32, [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _VP]),
    "drt_op_swiglu": (_I32, [_VP, _VP, _VP, _I64, _VP]),
    "drt_op_lm_head_workspace_bytes": (_SZ, [_I32, _I32, _I32]),
    "drt_op_lm_head_score": (_I32, [_VP, _VP, _VP, _I32, _I32, _I32, _VP, C.c_float, _U64, _I32,
                                    _VP, _VP, _VP, _VP, _VP, _SZ, _VP]),
}

_lib = None


def load():
    """Load the in-tree library once (raises LibraryNotBuilt when absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LibraryNotBuilt(
            f"{LIB_PATH} is missing: build it with `python -m diffusorrt_amd.build` "
            "(or __graft_entry__.build())")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    lib = load()
    n = lib.drt_last_error(None, 0)
    buf = C.create_string_buffer(int(n) + 1)
    lib.drt_last_error(buf, n + 1)
    return buf.value.decode("utf-8", "replace")


def check(status: int) -> None:
    """Raise the Python exception matching a non-OK AbiStatus."""
    if status == OK:
        return
    msg = last_error()
    if status == INVALID_ARGUMENT:
        raise AbiInvalidArgument(status, msg)
    if status == UNSUPPORTED:
        raise AbiUnsupported(status, msg)
    raise AbiError(status, msg)


def abi_version() -> tuple:
    lib = load()
    a, b, c = C.c_int32(), C.c_int32(), C.c_int32()
    lib.drt_abi_version(C.byref(a), C.byref(b), C.byref(c))
    return (a.value, b.value, c.value)


def i32_array(values):
    arr = (C.c_int32 * len(values))(*[int(v) for v in values])
    return arr
