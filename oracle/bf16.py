"""bfloat16 helpers for the numpy oracle (bf16 values are carried as uint16 bit patterns)."""

from __future__ import annotations

import numpy as np

BF16_MAX_BITS = np.uint16(0x7F7F)  # +3.3895e38, torch.finfo(torch.bfloat16).max (quest.py:57)
BF16_MIN_BITS = np.uint16(0xFF7F)  # -3.3895e38, torch.finfo(torch.bfloat16).min (quest.py:58)
BF16_NAN_BITS = np.uint16(0x7FC0)


def to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round-to-nearest-even; NaN -> 0x7FC0 (as torch does)."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(
        np.uint16
    )
    return np.where(np.isnan(f), BF16_NAN_BITS, rounded).astype(np.uint16)


def round_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return to_f32(from_f32(x))


def orderable_u32(x: np.ndarray) -> np.ndarray:
    """Monotone map float32 -> uint32 (bigger float -> bigger key).

    ``-0.0`` is folded into ``+0.0`` and every NaN into the largest key, which is
    how the selection treats them (NaN ranks above +inf, as in torch.topk).
    """
    f = np.ascontiguousarray(x, dtype=np.float32) + np.float32(0.0)
    u = f.view(np.uint32)
    key = np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)
    return np.where(np.isnan(f), np.uint32(0xFFFFFFFF), key).astype(np.uint32)
