"""Paired K/V writes into the slot arena (HIP kernel ``q3t_kv_write``).

``write`` keeps the signature and validation of the reference's one-token BNSD writer
(qwen3_tts_engine/kv_triton_ascend.py:39-53); ``write_tokens`` generalises it to several
consecutive tokens per request, which the code predictor's first step needs
(qwen3_tts_engine/predictor.py:19-24).  Both are bit-exact copies and never synchronise
the host; positions are trusted (rows outside the arena are skipped on the device).
"""
import torch

from . import _lib

_SUPPORTED = (torch.bfloat16, torch.float16, torch.float32)


def _validate(keys, values, target_keys, target_values, positions, single_token):
    if keys.ndim != 4 or values.shape != keys.shape or (single_token and keys.shape[2] != 1):
        raise ValueError('Expected matching single-token BNSD K/V' if single_token
                         else 'Expected matching BNSD K/V')
    batch, heads, _, width = keys.shape
    if (target_keys.shape != target_values.shape or target_keys.shape[:2] != (batch, heads)
            or target_keys.shape[-1] != width or not target_keys.is_contiguous()
            or not target_values.is_contiguous() or positions.shape != (batch,)
            or not positions.is_contiguous() or positions.dtype != torch.int64):
        raise ValueError('Invalid contiguous KV arena or position vector')
    tensors = (keys, values, target_keys, target_values)
    if any(t.device != keys.device or t.dtype != keys.dtype for t in tensors) or positions.device != keys.device:
        raise ValueError('KV tensors must share dtype and device')
    if keys.device.type != 'cuda' or keys.dtype not in _SUPPORTED:
        raise ValueError('Paired KV write supports bf16/fp16/fp32 ROCm tensors only')
    if keys.stride(3) != 1 or values.stride(3) != 1:
        raise ValueError('K/V rows must be unit-stride along head_dim')


def _launch(keys, values, target_keys, target_values, positions):
    batch, heads, tokens, width = keys.shape
    if batch == 0:
        return
    status = _lib.library().q3t_kv_write(
        keys.data_ptr(), values.data_ptr(), target_keys.data_ptr(), target_values.data_ptr(),
        positions.data_ptr(), batch, heads, tokens, width, keys.element_size(),
        _lib.i64x3((keys.stride(0), keys.stride(1), keys.stride(2))),
        _lib.i64x3((values.stride(0), values.stride(1), values.stride(2))),
        _lib.i64x3(target_keys.stride()[:3]), target_keys.shape[2],
        _lib.stream_handle(keys.device))
    _lib.check(status, 'kv write')


def write(keys, values, target_keys, target_values, positions, row_tiled=False):
    """target[b, h, positions[b]] = K/V[b, h, 0] for every row; one launch for K and V.

    ``row_tiled`` is accepted for signature compatibility; there is one kernel."""
    del row_tiled
    _validate(keys, values, target_keys, target_values, positions, single_token=True)
    _launch(keys, values, target_keys, target_values, positions)


def write_tokens(keys, values, target_keys, target_values, positions):
    """target[b, h, positions[b] + t] = K/V[b, h, t] for t < keys.shape[2]."""
    _validate(keys, values, target_keys, target_values, positions, single_token=False)
    _launch(keys, values, target_keys, target_values, positions)
