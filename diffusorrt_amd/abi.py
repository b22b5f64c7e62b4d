"""Integer encodings that cross the C-ABI.

Values are the reference's wire values (``abi/enums.py:14-56`` of the
reference's ``python/src/edllm/``): renumbering would break the contract, so they
are kept identical.
"""
from __future__ import annotations

from enum import IntEnum

ABI_VERSION = (0, 1, 0)
UNSET = -1


class DecodeStrategy(IntEnum):
    BLOCK_THRESHOLD = 0
    CONFIDENCE_THRESHOLD = 1
    D2F_BLOCK_PIPELINE = 2
    DILATED_UNMASK = 3
    ENTROPY_BUDGET = 4
    ENTROPY_COUNT = 5
    FIXED_QUOTA = 6
    BD3_FIXED_QUOTA = 7


class CommitPolicy(IntEnum):
    DILATED = 0
    ENTROPY_BUDGET = 1
    THRESHOLD = 2
    FIXED_QUOTA = 3


class ComputeDtype(IntEnum):
    BF16 = 0
    FP32 = 1


class AttentionMaskKind(IntEnum):
    BIDIRECTIONAL = 0
    D2F_HYBRID = 1
    FULL = 2


DECODE_STRATEGY_BY_NAME = {m.name.lower(): m for m in DecodeStrategy}
ATTENTION_MASK_KIND_BY_NAME = {m.name.lower(): m for m in AttentionMaskKind}


def encode(mapping: dict, name: str, field: str) -> int:
    try:
        return int(mapping[name])
    except KeyError:
        raise ValueError(f"{field}={name!r} has no ABI encoding") from None
