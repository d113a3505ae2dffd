"""bf16 <-> fp32 conversion on raw bits (numpy has no bfloat16 dtype).

bf16 is the upper 16 bits of an IEEE fp32. Rounding fp32 -> bf16 is round to
nearest, ties to even, which is what torch's ``.to(torch.bfloat16)`` does for
finite values.
"""
import numpy as np


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def round_f32(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16 value (returned as float32)."""
    return bits_to_f32(f32_to_bits(x))
