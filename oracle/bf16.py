"""Bit-exact bfloat16 helpers on numpy (oracle; test infrastructure only).

numpy has no bfloat16 dtype, so bf16 tensors are carried as ``uint16`` bit
patterns.  Conversions follow c10::BFloat16: float32 -> bf16 rounds to nearest,
ties to even, and every NaN becomes the canonical quiet NaN 0x7FC0.

Pinned by tests/test_oracle_bf16.py against torch's own ``.to(torch.bfloat16)``
on exhaustive tie/NaN/Inf/denormal sweeps.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16_bits(a) -> np.ndarray:
    """float32 array -> uint16 bf16 bit patterns, round-to-nearest-even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    # u + 0x7FFF + lsb stays below 2**32 for every non-NaN pattern (at most 0xFF807FFF);
    # NaNs, which may wrap, are overwritten below
    t = u >> np.uint32(16)
    t &= np.uint32(1)
    t += u
    t += np.uint32(0x7FFF)
    t >>= np.uint32(16)
    r = t.astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = np.uint16(0x7FC0)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """float32 -> float32 value rounded to the nearest bf16 (RNE)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def f16_bits_to_f32(b) -> np.ndarray:
    """uint16 IEEE half bit patterns -> float32 (exact)."""
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(a) -> np.ndarray:
    """float32 -> IEEE half bit patterns (numpy's RNE conversion)."""
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)
