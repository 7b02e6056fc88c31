"""Rotary position embedding on the GPU.

``rotary`` is the drop-in for the reference's exact bf16 BSND rotary
(qwen3_tts_engine/rotary_triton_ascend.py:29-44): same arguments, same validation, a new
output tensor, and torch-eager rounding after every op (kernel ``q3t_rotary``); fp32 rows
are accepted too, with torch-eager fp32 rounding.
``rope_tables`` produces the default-RoPE cos/sin rows for integer positions
(kernel ``q3t_rope_tables``); ``inverse_frequencies`` is the host-side fp32 table it uses.
"""
import torch

from . import _lib

DEFAULT_THETA = 1_000_000.0
_INV_FREQ = {}


def rotary(hidden, cos, sin):
    """Rotate-half RoPE of a contiguous bf16 (batch, length, heads, width) tensor."""
    if hidden.ndim != 4 or hidden.device.type != 'cuda' or hidden.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError('Expected BF16 or FP32 BSND ROCm input')
    batch, length, heads, width = hidden.shape
    if heads < 1 or width not in (64, 128) or batch * length < 1:
        raise ValueError('Unsupported rotary shape')
    if cos.shape != (batch, length, width) or sin.shape != cos.shape:
        raise ValueError('Rotary coefficients must match batch, length and width')
    if any(t.device != hidden.device or t.dtype != hidden.dtype or not t.is_contiguous()
           for t in (hidden, cos, sin)):
        raise ValueError('Rotary tensors must be contiguous with matching dtype/device')
    output = torch.empty_like(hidden)
    status = _lib.library().q3t_rotary(hidden.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                       output.data_ptr(), batch * length, heads, width,
                                       _lib.DTYPE_CODES[hidden.dtype],
                                       _lib.stream_handle(hidden.device))
    _lib.check(status, 'rotary')
    return output


def inverse_frequencies(head_dim, theta=DEFAULT_THETA):
    """fp32 1 / theta**(2i/head_dim), computed as the default RoPE initialiser does."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64).to(torch.float32) / head_dim
    return 1.0 / (theta ** exponent)


def rope_tables(positions, head_dim, theta=DEFAULT_THETA, scaling=1.0, dtype=torch.bfloat16,
                inv_freq=None):
    """cos, sin of shape positions.shape + (head_dim,) for int64 device positions."""
    if positions.dtype != torch.int64 or positions.device.type != 'cuda':
        raise ValueError('positions must be an int64 ROCm tensor')
    if dtype not in (torch.bfloat16, torch.float32):
        raise ValueError('rope tables are produced in bf16 or fp32')
    if head_dim % 2 or head_dim < 2:
        raise ValueError('head_dim must be even')
    if inv_freq is None:
        key = (positions.device, head_dim, float(theta))
        inv_freq = _INV_FREQ.get(key)
        if inv_freq is None:  # cached so that captured graphs never see a host copy
            inv_freq = inverse_frequencies(head_dim, theta).to(positions.device)
            _INV_FREQ[key] = inv_freq
    inv_freq = inv_freq.to(device=positions.device, dtype=torch.float32).contiguous()
    flat = positions.contiguous().view(-1)
    cos = torch.empty(*positions.shape, head_dim, device=positions.device, dtype=dtype)
    sin = torch.empty_like(cos)
    status = _lib.library().q3t_rope_tables(flat.data_ptr(), flat.numel(), inv_freq.data_ptr(),
                                            head_dim // 2, float(scaling),
                                            _lib.DTYPE_CODES[dtype], cos.data_ptr(),
                                            sin.data_ptr(), _lib.stream_handle(positions.device))
    _lib.check(status, 'rope tables')
    return cos, sin
