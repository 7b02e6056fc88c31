"""Graph batch bucket for a changing active request count.

Host-side integer rule of the reference's decode scheduler
(qwen3_tts_engine/batching.py:4-11): with no step, the active count rounds up to a power of
two; with a power-of-two step, counts above the step round up to a multiple of it.
"""


def _is_pow2(value: int) -> bool:
    return value > 0 and value & (value - 1) == 0


def decode_batch_size(active, max_slots, step=0):
    """Captured-graph batch that holds ``active`` requests in a ``max_slots`` arena."""
    if not (1 <= active <= max_slots) or not _is_pow2(max_slots):
        raise ValueError('Active count must fit a positive power-of-two slot arena')
    if step < 0 or (step != 0 and (not _is_pow2(step) or step > max_slots)):
        raise ValueError('Decode bucket step must be zero or a power of two within the arena')
    if step == 0 or active <= step:
        return 1 << (active - 1).bit_length()
    return -(-active // step) * step
