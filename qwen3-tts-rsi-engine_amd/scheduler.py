"""Integer slot state of continuous batching and the arena operations it drives.

Mirrors the bookkeeping of the reference's ``ContinuousModel`` (qwen3_tts_engine/continuous.py):

* admission (``admit_batch``, continuous.py:425-473): a new request takes slot
  ``len(states)``; the arena grows first if the longest prompt does not fit; each request's
  prefill KV prefix is copied into its slot (``load_packed``);
* cancellation and retirement (``tick``, continuous.py:545-555 and 645-656): visited in
  reverse slot order; the last slot's row is moved into the freed slot and its state takes
  the freed index, so slots stay dense;
* each decode tick (continuous.py:570-629): graph batch ``decode_batch_size(count)``,
  capacity check against the largest position, context ``C`` or, with ``bucket_kv``,
  ``min(C, max(64, next_pow2(max_position + 1)))``, positions padded with zeros to the graph
  batch; afterwards every request advances one frame and one position and retires once
  ``frames >= max_new_tokens - 1`` (continuous.py:638);
* capacity (``ensure_capacity``, continuous.py:353-363): unchanged while the requirement is
  below ``C``, else ``max(2C, 2**bit_length(required))`` with the contents copied.

Only the integer state lives here; with an arena attached, the moves, loads and regrowths
run as the package's HIP copy kernels, in the order the reference issues them.  Every
operation is also recorded in ``ops`` for inspection.

``compact_prefix=True`` keeps the integer state identical but shrinks the copies to what can
still be read: a compaction move copies the moved request's rows ``[:position + 1]`` instead
of the whole capacity, and a regrowth copies only the slots in use.  Rows past a request's
position are always written before they are read, so every attended row is unchanged.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .batching import decode_batch_size
from .slots import grow_arena


@dataclass
class SlotState:
    identifier: object
    position: int
    max_new_tokens: int
    frames: int = 0
    rope_delta: int = 0


@dataclass
class DecodeBatch:
    """What one decode tick launches: the graph batch, the attended context, and per-slot
    positions (zero-padded to the graph batch)."""
    batch: int
    context: int
    capacity: int
    positions: list = field(default_factory=list)
    identifiers: list = field(default_factory=list)
    rotary: list = field(default_factory=list)

    @property
    def count(self):
        return len(self.identifiers)

    def positions_tensor(self, device):
        return torch.tensor(self.positions, dtype=torch.int64, device=device)


def grown_capacity(capacity: int, required: int) -> int:
    if required < capacity:
        return capacity
    return max(2 * capacity, 1 << int(required).bit_length())


class SlotScheduler:
    """Dense slot table of a continuous batch (one model-owner thread drives it)."""

    def __init__(self, max_slots, capacity=512, decode_bucket_step=0, bucket_kv=False, arena=None,
                 compact_prefix=False):
        if max_slots < 1 or max_slots & (max_slots - 1):
            raise ValueError('Continuous slot count must be a positive power of two')
        decode_batch_size(1, max_slots, decode_bucket_step)  # validates the bucket step
        self.max_slots = max_slots
        self.decode_bucket_step = decode_bucket_step
        self.bucket_kv = bucket_kv
        self.arena = arena
        self.compact_prefix = compact_prefix
        self.capacity = arena.capacity if arena is not None else capacity
        self.states: list[SlotState] = []
        self.ops: list[tuple] = []

    # -- arena-level operations ----------------------------------------------------------
    def ensure_capacity(self, required: int) -> None:
        new = grown_capacity(self.capacity, required)
        if new == self.capacity:
            return
        self.ops.append(('grow', self.capacity, new))
        if self.arena is not None:
            active = len(self.states) if self.compact_prefix else None
            self.arena = grow_arena(self.arena, required, active=active)
        self.capacity = new

    def _retire(self, index: int) -> None:
        last = len(self.states) - 1
        if last != index:
            self.ops.append(('move', last, index))
            if self.arena is not None:
                length = self.states[last].position + 1 if self.compact_prefix else None
                self.arena.move(last, index, length=length)
            self.states[index] = self.states[last]
        self.states.pop()

    # -- request lifecycle ---------------------------------------------------------------
    def cancel(self, identifiers) -> None:
        wanted = set(identifiers)
        for index in range(len(self.states) - 1, -1, -1):
            if self.states[index].identifier in wanted:
                self._retire(index)

    def admit(self, requests, prefill_cache=None) -> list[int]:
        """requests: [(identifier, prompt_length, max_new_tokens)], prompts packed in rows
        0 .. n-1 of ``prefill_cache`` (a packed (2L, rows, Hkv, Lp, D) prefill KV) when an
        arena is attached.  Returns the slots taken."""
        requests = list(requests)
        if not requests:
            return []
        if len(self.states) + len(requests) > self.max_slots:
            raise ValueError('Insufficient continuous request slots')
        self.ensure_capacity(max(length for _, length, _ in requests))
        slots = []
        for row, (identifier, length, limit) in enumerate(requests):
            slot = len(self.states)
            self.ops.append(('load', slot, identifier, length))
            if self.arena is not None and prefill_cache is not None:
                self.arena.load_packed(slot, prefill_cache, row=row, length=length)
            self.states.append(SlotState(identifier, length, limit))
            slots.append(slot)
        return slots

    def decode_batch(self) -> DecodeBatch | None:
        if not self.states:
            return None
        count = len(self.states)
        batch = decode_batch_size(count, self.max_slots, self.decode_bucket_step)
        largest = max(state.position for state in self.states)
        self.ensure_capacity(largest)
        if self.bucket_kv:
            need = largest + 1
            context = min(self.capacity, max(64, 1 << (need - 1).bit_length()))
        else:
            context = self.capacity
        pad = [0] * (batch - count)
        self.ops.append(('decode', batch, context))
        return DecodeBatch(batch, context, self.capacity,
                           [s.position for s in self.states] + pad,
                           [s.identifier for s in self.states],
                           [s.position + s.rope_delta for s in self.states] + pad)

    def advance(self, stopped=()) -> list:
        """After a decode step: every request moves one frame and one position; requests at
        their frame limit (or listed in ``stopped``) retire in reverse slot order.  Returns
        the retired identifiers in that order."""
        stopped = set(stopped)
        finished = []
        for index, state in enumerate(self.states):
            state.frames += 1
            state.position += 1
            if state.identifier in stopped or state.frames >= state.max_new_tokens - 1:
                finished.append(index)
        done = []
        for index in reversed(finished):
            done.append(self.states[index].identifier)
            self._retire(index)
        return done

    def tick(self, submissions=(), cancelled=(), prefill_cache=None, stopped=()):
        """One scheduler iteration: cancellations, admissions, the decode batch, advance.
        Returns (DecodeBatch or None, retired identifiers)."""
        self.ops = []
        self.cancel(cancelled)
        self.admit(submissions, prefill_cache)
        batch = self.decode_batch()
        if batch is None:
            return None, []
        return batch, self.advance(stopped)
