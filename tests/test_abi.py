"""The C-ABI boundary without a GPU: the library loads, exports every entry
point ``include/drt_rocm.h`` declares, binds each one in ``_lib``, and answers
the host-only calls; the wire enums keep the reference's values."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from diffusorrt_amd import _lib, abi, runtime
from oracle import ops as O

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "drt_rocm.h"


def _declared_functions() -> set:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"\b(drt_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from diffusorrt_amd import build
        build.build()
    return _lib.load()


def test_header_declares_the_bound_entry_points():
    declared = _declared_functions()
    assert len(declared) >= 20
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = C.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(_declared_functions()) if not hasattr(raw, n)]
    assert not missing, missing


def test_abi_version_and_last_error_are_host_only(lib):
    assert _lib.abi_version() == abi.ABI_VERSION == (0, 1, 0)
    assert isinstance(_lib.last_error(), str)


def test_invalid_handles_are_rejected_before_any_device_work(lib):
    """Unknown handles fail with INVALID_ARGUMENT (the reference raises before
    side effects) and set the last-error text."""
    st = lib.drt_release_handle(C.c_uint64(123456789))
    assert st == _lib.INVALID_ARGUMENT
    assert _lib.last_error()
    with pytest.raises(_lib.AbiInvalidArgument):
        _lib.check(lib.drt_session_set_profiling(C.c_uint64(987654321), 1))


def test_enum_wire_values_match_reference():
    """Values from the reference's abi/enums.py:14-43."""
    assert abi.DecodeStrategy.FIXED_QUOTA == 6 and abi.DecodeStrategy.BD3_FIXED_QUOTA == 7
    assert abi.DecodeStrategy.BLOCK_THRESHOLD == 0 and abi.DecodeStrategy.ENTROPY_COUNT == 5
    assert abi.CommitPolicy.FIXED_QUOTA == 3 and abi.CommitPolicy.THRESHOLD == 2
    assert (abi.AttentionMaskKind.BIDIRECTIONAL, abi.AttentionMaskKind.D2F_HYBRID,
            abi.AttentionMaskKind.FULL) == (0, 1, 2)
    assert (abi.ComputeDtype.BF16, abi.ComputeDtype.FP32) == (0, 1)
    assert (_lib.OK, _lib.INVALID_ARGUMENT, _lib.UNSUPPORTED) == (0, 2, 3)


def test_session_configs_encode_the_two_strategies():
    bd3 = runtime.bd3_session_config(32, 64, 256)
    assert bd3["decode_strategy"] == abi.DecodeStrategy.BD3_FIXED_QUOTA
    assert bd3["attention_mask_kind"] == abi.AttentionMaskKind.D2F_HYBRID
    fq = runtime.fixed_quota_session_config(256, 64, 256)
    assert fq["decode_strategy"] == abi.DecodeStrategy.FIXED_QUOTA
    assert fq["attention_mask_kind"] == abi.AttentionMaskKind.BIDIRECTIONAL
    assert fq["commit_policy"] == bd3["commit_policy"] == abi.CommitPolicy.FIXED_QUOTA


def test_runtime_rope_tables_match_oracle():
    cos, sin = runtime.rope_tables(300, 128, 1e6)
    ocos, osin = O.rope_tables(np.arange(300), 128, 1e6)
    np.testing.assert_array_equal(cos, ocos[:, 0, :64])
    np.testing.assert_array_equal(sin, osin[:, 0, :64])


def test_product_package_never_imports_the_oracle():
    pkg = ROOT / "diffusorrt_amd"
    for path in pkg.rglob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.M), path


def _reference_engine_config(scheme: str, exact_kv: bool) -> dict:
    """The dict ``cuda_engine_config`` builds (``backends/device_runtime.py:53-58``)."""
    config = {"compute_dtype": 0, "d2f_exact_kv_cache": int(exact_kv)}
    if scheme == "int8_weight_only":
        config.update(linear_quant_bits=8, linear_quant_group_size=64)
    return config


def test_engine_request_takes_the_reference_dream_block_threshold_config():
    """model.py:905-916 opens Dream's block_threshold runtime with
    cuda_engine_config(precision, exact_kv=True) (exact_kv from model.py:991)."""
    for kind in ("q4", "bf16"):
        assert runtime.engine_request(_reference_engine_config("bf16", True), kind)[1] == 1
        assert runtime.engine_request(_reference_engine_config("bf16", False), kind)[1] == 0
    assert runtime.engine_request({}, "q4") == (4, 0)
    with pytest.raises(ValueError):  # 8-bit linears are not offered
        runtime.engine_request(_reference_engine_config("int8_weight_only", True), "q4")
    for bad in ({"d2f_exact_kv_cache": 2}, {"prefix_kv_cache": 1}, {"canvas_cache": 1},
                {"compute_dtype": 1}):
        with pytest.raises(ValueError):
            runtime.engine_request(bad, "q4")


def test_session_config_struct_matches_the_reference_fields():
    """SessionDecodeConfig (abi/lifetimes.py:57-69): eight int32 fields then
    ``reserved`` (8 ints)."""
    names = [n for n, _ in _lib.SessionConfig._fields_]
    assert names == ["decode_strategy", "commit_policy", "attention_mask_kind", "block_size",
                     "steps", "max_tokens", "trace_canvas", "error_fixing", "reserved"]
    assert C.sizeof(_lib.SessionConfig) == 16 * 4
    text = HEADER.read_text()
    assert re.search(r"int32_t reserved\[8\];[^\n]*\n\} drt_session_config;", text)
