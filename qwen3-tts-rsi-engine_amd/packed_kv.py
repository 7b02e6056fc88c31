"""Copy one request's prefix across every plane of a packed KV arena on the GPU.

Drop-in for ``copy_packed_prefix`` (qwen3_tts_engine/packed_kv.py:6-31): the same
arguments, the same validation and ``ValueError`` raised before any device write; the copy
itself is the ``q3t_copy_strided`` HIP kernel (bit-exact element copy, any strides).
"""
import torch

from . import _lib


def _is_index(value) -> bool:
    return type(value) is int


def copy_packed_prefix(target, source, slot, row=0, length=None):
    """target[:, slot, :, :length] = source[:, row, :, :length]; other slots and the tail
    of the selected slot are preserved."""
    if (
        not isinstance(target, torch.Tensor)
        or not isinstance(source, torch.Tensor)
        or target.ndim != 5
        or source.ndim != 5
        or any(size <= 0 for size in (*target.shape, *source.shape))
        or (target.shape[0], target.shape[2], target.shape[4])
        != (source.shape[0], source.shape[2], source.shape[4])
        or target.device != source.device
        or target.dtype != source.dtype
        or target.untyped_storage().data_ptr() == source.untyped_storage().data_ptr()
    ):
        raise ValueError("Expected independent compatible packed KV tensors")
    length = source.shape[3] if length is None else length
    if (
        not _is_index(slot) or not 0 <= slot < target.shape[1]
        or not _is_index(row) or not 0 <= row < source.shape[1]
        or not _is_index(length) or not 0 < length <= min(target.shape[3], source.shape[3])
    ):
        raise ValueError("Expected a valid packed KV row and prefix length")
    copy_rows(target[:, slot, :, :length], source[:, row, :, :length])


def copy_rows(dst: torch.Tensor, src: torch.Tensor) -> None:
    """Element copy dst <- src of equal shape (<= 5 dims, any strides) by the HIP kernel."""
    if dst.shape != src.shape or dst.dtype != src.dtype:
        raise ValueError("copy requires equal shapes and dtypes")
    if dst.ndim > 5 or dst.ndim == 0:
        raise ValueError("copy supports 1 to 5 dimensions")
    device = _lib.require_gpu(dst, src)
    if dst.numel() == 0:
        return
    n = dst.ndim
    sizes = (_lib.c_i64 * n)(*dst.shape)
    ds = (_lib.c_i64 * n)(*dst.stride())
    ss = (_lib.c_i64 * n)(*src.stride())
    status = _lib.library().q3t_copy_strided(dst.data_ptr(), src.data_ptr(), dst.element_size(),
                                             n, sizes, ds, ss, _lib.stream_handle(device))
    _lib.check(status, "copy_rows")
