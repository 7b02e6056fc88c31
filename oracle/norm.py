"""RMSNorm of bf16 rows over the last axis (the attention module's q_norm / k_norm).

Test infrastructure only.  Formula of the modules the reference calls at
packed_attention.py:42-45 (Qwen3 RMSNorm, from qwen_tts; transformers' Qwen3RMSNorm is the
installed analogue): y = x.float(); y = y * rsqrt(mean(y ** 2) + eps); return
weight * y.to(bf16).  The mean is taken in float64 here, then rounded to fp32, so the oracle
gives the row's correctly rounded statistic; fp32 implementations (torch's, the GPU
kernel's) sum in their own orders and land on the same bf16 value except next to rounding
ties.  The tests pin this restatement against torch's own CPU module formula.
"""
import numpy as np

from . import bf16


def rms_norm_bf16(x_bits, weight_bits, eps):
    """x_bits (..., D) and weight_bits (D,) bf16 bit patterns -> bf16 bit patterns (..., D)."""
    x = bf16.from_bits(x_bits).astype(np.float64)
    mean = np.float32(np.mean(x * x, axis=-1, keepdims=True))
    r = np.float32(1.0) / np.sqrt(mean + np.float32(eps), dtype=np.float32)
    normed = bf16.round_bf16(bf16.from_bits(x_bits) * r)
    return bf16.to_bits(normed * bf16.from_bits(weight_bits))
