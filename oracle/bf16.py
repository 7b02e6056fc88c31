"""bfloat16 bit helpers in numpy (bf16 is the upper 16 bits of an IEEE fp32).

Rounding is round-to-nearest-even with NaN mapped to 0x7fc0, the rule c10::BFloat16 uses
for every torch-eager bf16 op.  Pinned against torch's casts in tests/test_oracle.py.
"""
import numpy as np


def to_bits(x) -> np.ndarray:
    """fp32 values -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, 0x7FC0, rounded).astype(np.uint16)


def from_bits(bits) -> np.ndarray:
    """bf16 bit patterns -> fp32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """fp32 -> nearest bf16 value, returned as fp32."""
    return from_bits(to_bits(x))
