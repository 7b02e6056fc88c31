"""Byte-exact restatement of the slot arena's KV writes and copies (numpy, any dtype)."""
import numpy as np


def kv_write(target_keys, target_values, keys, values, positions):
    """target[b, h, positions[b] + t] = new[b, h, t]  (continuous.py:164-166 scatter_,
    kv_triton_ascend.py:31-36, predictor.py:19-23 for multi-token writes).
    Positions outside the arena are skipped, the product's documented device rule."""
    batch, heads, tokens, _ = keys.shape
    capacity = target_keys.shape[2]
    for b in range(batch):
        for t in range(tokens):
            pos = int(positions[b]) + t
            if 0 <= pos < capacity:
                target_keys[b, :, pos] = keys[b, :, t]
                target_values[b, :, pos] = values[b, :, t]
    return target_keys, target_values


def copy_packed_prefix(target, source, slot, row=0, length=None):
    """target[:, slot, :, :length] = source[:, row, :, :length]  (packed_kv.py:21-31)."""
    length = source.shape[3] if length is None else length
    target[:, slot, :, :length] = source[:, row, :, :length]
    return target


def move(planes, source, destination):
    """Whole-slot compaction copy in every plane (continuous.py:124-128)."""
    if source != destination:
        for plane in planes:
            plane[destination] = plane[source]
    return planes


def grown_capacity(capacity, required):
    """Capacity after ensure_capacity(required) (continuous.py:353-360): unchanged while
    required < capacity, else max(2*capacity, 2**bit_length(required))."""
    if required < capacity:
        return capacity
    return max(capacity * 2, 1 << int(required).bit_length())


def grow(planes, new_capacity):
    """New zeroed planes of the larger capacity holding the old contents
    (continuous.py:360-363)."""
    grown = []
    for plane in planes:
        shape = list(plane.shape)
        shape[2] = new_capacity
        new = np.zeros(shape, dtype=plane.dtype)
        new[:, :, :plane.shape[2]] = plane
        grown.append(new)
    return grown
