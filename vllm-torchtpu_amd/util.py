"""Integer helpers of the RPA layout contract (reference util.py:20-35)."""

from __future__ import annotations

import torch


def cdiv(a: int, b: int) -> int:
    """Ceiling division (util.py:20-22)."""
    assert b != 0
    return (a + b - 1) // b


def align_to(x: int, a: int) -> int:
    """Round x up to a multiple of a (util.py:25-26)."""
    return cdiv(x, a) * a


def get_dtype_packing(dtype: torch.dtype) -> int:
    """Elements of `dtype` per 32-bit word (util.py:33-35)."""
    return 32 // (torch.empty((), dtype=dtype).element_size() * 8)


def next_power_of_2(x: int) -> int:
    """Smallest power of two >= x (util.py:38-50)."""
    assert x > 0
    return 1 if x == 1 else 1 << (x - 1).bit_length()
