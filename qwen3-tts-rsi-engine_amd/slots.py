"""KV state of continuous batching: slot arena, slot cache, predictor cache.

Drop-ins for the reference's ``SlotArena`` / ``SlotCache`` (qwen3_tts_engine/continuous.py:97-169)
and ``PredictorCache`` (qwen3_tts_engine/predictor.py:9-27): same constructors, attributes and
``update`` contract.  Every device-side byte move (decode K/V write, prefix load, slot
compaction, capacity regrowth) is a HIP kernel of this package.
"""
from __future__ import annotations

import types

import torch
from transformers.cache_utils import Cache

from . import kv_write
from .attention import PLAN_MAX_BATCH, decode_grid_for, decode_plan, plan_shape
from .packed_kv import copy_packed_prefix, copy_rows


def _attention_heads(reference):
    """(query heads, KV heads) of the talker's attention: the config's counts, or the first
    layer's query projection over head_dim where the config names no query-head count."""
    config = reference.config
    q_heads = getattr(config, 'num_attention_heads', None)
    if q_heads is None:
        attn = reference.layers[0].self_attn
        attn = getattr(attn, 'reference', attn)  # PackedAttention keeps the wrapped module
        q_heads = attn.q_proj.out_features // config.head_dim
    return q_heads, config.num_key_value_heads


class SlotArena:
    """Per-slot KV storage for every talker layer.

    ``packed_kv=True`` keeps all layers in one (2*layers, slots, kv_heads, capacity, head_dim)
    tensor (keys first), as continuous.py:109-113 does; otherwise one tensor per layer."""

    def __init__(self, reference, slots, capacity, native_kv_update=False, triton_kv_update=False,
                 packed_kv=False):
        self.reference = reference
        self.slots = slots
        self.capacity = capacity
        self.native_kv_update = native_kv_update
        self.triton_kv_update = triton_kv_update
        self.packed_kv = packed_kv
        weight = next(reference.parameters())
        config = reference.config
        shape = (slots, config.num_key_value_heads, capacity, config.head_dim)
        self.packed = None
        if packed_kv:
            layers = len(reference.layers)
            self.packed = torch.zeros((layers * 2, *shape), device=weight.device, dtype=weight.dtype)
            self.keys = list(self.packed[:layers].unbind(0))
            self.values = list(self.packed[layers:].unbind(0))
        else:
            self.keys = [torch.zeros(shape, device=weight.device, dtype=weight.dtype)
                         for _ in reference.layers]
            self.values = [torch.zeros_like(key) for key in self.keys]

    def load(self, slot, cache, row=0, length=None):
        """Copy the first ``length`` positions of one prefill cache row into ``slot``."""
        length = cache.get_seq_length() if length is None else length
        for i, layer in enumerate(cache.layers):
            copy_rows(self.keys[i][slot, :, :length], layer.keys[row, :, :length])
            copy_rows(self.values[i][slot, :, :length], layer.values[row, :, :length])

    def move(self, source, destination, length=None):
        """Compaction: slot row ``source`` overwrites ``destination`` in every layer.

        ``length=None`` copies the whole row, as the reference does (continuous.py:124-128).
        With ``length``, only positions ``[:length]`` are copied: a request at position p
        reads rows ``[0, p]`` and writes row p before reading it, so rows past its position
        are never read before they are written, and the copy shrinks from the capacity to
        the request's own length."""
        if source == destination:
            return
        if length is not None:
            length = min(int(length), self.capacity)
            if length <= 0:
                return
            if self.packed is not None:
                copy_rows(self.packed[:, destination, :, :length], self.packed[:, source, :, :length])
                return
            for keys, values in zip(self.keys, self.values):
                copy_rows(keys[destination, :, :length], keys[source, :, :length])
                copy_rows(values[destination, :, :length], values[source, :, :length])
            return
        if self.packed is not None:
            copy_rows(self.packed[:, destination], self.packed[:, source])
            return
        for keys, values in zip(self.keys, self.values):
            copy_rows(keys[destination], keys[source])
            copy_rows(values[destination], values[source])

    def load_packed(self, slot, cache, row=0, length=None):
        copy_packed_prefix(self.packed, cache, slot, row=row, length=length)

    def planes(self):
        """Every key plane followed by every value plane (the packed order)."""
        return self.keys + self.values


def grow_arena(old: SlotArena, required: int, active: int | None = None) -> SlotArena:
    """A larger arena holding ``old``'s contents, with the reference's capacity rule
    max(2*C, 2**bit_length(required)) (continuous.py:353-363).  ``required < C`` returns ``old``.

    ``active=None`` copies every slot, as the reference does; ``active=n`` copies only slots
    ``[0, n)`` (the dense slots in use: a free slot is loaded from a prefill before it is read)."""
    if required < old.capacity:
        return old
    capacity = max(old.capacity * 2, 1 << int(required).bit_length())
    new = SlotArena(old.reference, old.slots, capacity, old.native_kv_update, old.triton_kv_update,
                    packed_kv=old.packed_kv)
    used = old.slots if active is None else max(0, min(int(active), old.slots))
    if used == 0:
        return new
    if new.packed is not None:
        copy_rows(new.packed[:, :used, :, :old.capacity], old.packed[:, :used])
    else:
        for target, source in zip(new.planes(), old.planes()):
            copy_rows(target[:used, :, :old.capacity], source[:used])
    return new


class SlotCache(Cache):
    """HF ``Cache`` whose ``update`` writes one decode token per request into the arena at
    ``positions[b]`` and returns the arena views the attention reads."""

    def __init__(self, arena, positions, context_length=None, valid_length_kv=False):
        super().__init__(layers=[])
        self.arena = arena
        self.positions = positions
        self.context_length = arena.capacity if context_length is None else context_length
        self.actual_seq_lengths_kv = ([self.context_length] * positions.shape[0]
                                      if valid_length_kv else None)
        self.plan = None  # the step's plan of the requests (prepare), read by every layer
        self._plan = None

    def prepare(self):
        """Per-step hook, run after the positions change and before the layers (SlotGraph.compute
        does).  The reference rebuilds its scatter indices from the positions here
        (continuous.py:147-150); the HIP writer reads the positions directly, and this ranks and
        bundles the step's requests for the bundled grid once for all the step's layers
        (``decode_plan``), when the step's launches take that grid (unmasked over the arena, or
        masked over the context view); otherwise no plan is made.  The plan buffer is
        allocated on the first call (SlotGraph's eager pass, before capture) and refilled by a
        kernel after."""
        positions = self.positions
        batch = positions.shape[0]
        q_heads, kv_heads = _attention_heads(self.arena.reference)
        shape = plan_shape(batch, q_heads, kv_heads) if 0 < batch <= PLAN_MAX_BATCH else None
        if not (positions.is_cuda and positions.ndim == 1 and positions.dtype == torch.int64 and shape):
            self.plan = None
            return
        plane = self.arena.keys[0]
        if not any(decode_grid_for(batch, 1, q_heads, kv_heads, plane.shape[-1], ctx, plane.dtype,
                                   masked=masked) == 'bundled'
                   for ctx, masked in ((self.arena.capacity, False), (self.context_length, True))):
            self.plan = None
            return
        if self._plan is None or tuple(self._plan.shape) != shape or self._plan.device != positions.device:
            self._plan = torch.empty(shape, device=positions.device, dtype=torch.int32)
        self.plan = decode_plan(positions, self.arena.capacity, q_heads, kv_heads, out=self._plan)

    def update(self, keys, values, layer_idx, cache_kwargs):
        batch = keys.shape[0]
        target_keys = self.arena.keys[layer_idx][:batch]
        target_values = self.arena.values[layer_idx][:batch]
        kv_write.write(keys, values, target_keys, target_values, self.positions)
        if self.actual_seq_lengths_kv is not None:
            return target_keys, target_values
        return (target_keys[:, :, :self.context_length],
                target_values[:, :, :self.context_length])


class PredictorCache(Cache):
    """Fixed 16-position cache of the code predictor: step 0 writes positions [0, 2),
    step s >= 1 writes position s + 1; ``update`` returns the [:step + 2] views."""

    def __init__(self, reference, inputs, capacity=16):
        super().__init__(layers=[])
        config = reference.config
        shape = (inputs.shape[0], config.num_key_value_heads, capacity, config.head_dim)
        self.keys = [torch.zeros(shape, device=inputs.device, dtype=inputs.dtype)
                     for _ in range(config.num_hidden_layers)]
        self.values = [torch.zeros_like(tensor) for tensor in self.keys]
        self.step = 0
        self._starts = {}

    def positions_at(self, batch, start, device):
        """A device tensor of ``batch`` copies of ``start`` (the write position of a step),
        kept alive for graph replays."""
        key = (batch, start, device)
        if key not in self._starts:
            if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
                raise RuntimeError('PredictorCache positions must be created by an eager step before capture')
            self._starts[key] = torch.full((batch,), start, device=device, dtype=torch.int64)
        return self._starts[key]

    def update(self, keys, values, layer_index, cache_kwargs):
        start = 0 if self.step == 0 else self.step + 1
        end = self.step + 2
        if keys.shape[2] != end - start:
            raise ValueError('predictor step writes one token (two at step 0)')
        positions = self.positions_at(keys.shape[0], start, keys.device)
        kv_write.write_tokens(keys, values, self.keys[layer_index], self.values[layer_index], positions)
        return self.keys[layer_index][:, :, :end], self.values[layer_index][:, :, :end]

    def get_seq_length(self, layer_idx=0):
        return 0 if self.step == 0 else self.step + 1


class PrefillCache(Cache):
    """Per-layer KV of a padded prefill batch, held in one packed
    ``(2L, batch, kv_heads, length, head_dim)`` buffer (keys first), with the valid length
    of every row (``kv_lens``, int32, device).  ``layers[i].keys`` / ``.values`` are the
    ``(batch, kv_heads, length, head_dim)`` planes of layer i, as a ``DynamicCache``'s are."""

    def __init__(self, layers, batch, length, kv_heads, head_dim, device, dtype):
        super().__init__(layers=[])
        self.packed = torch.zeros(2 * layers, batch, kv_heads, length, head_dim, device=device, dtype=dtype)
        self.kv_lens = torch.full((batch,), length, device=device, dtype=torch.int32)
        self.cu_seqlens = torch.arange(0, (batch + 1) * length, length, device=device, dtype=torch.int32)
        self.length = length
        self.layers = [types.SimpleNamespace(keys=self.packed[i], values=self.packed[layers + i])
                       for i in range(layers)]

    def update(self, keys, values, layer_idx, cache_kwargs=None):
        raise ValueError('a PrefillCache is written by PackedAttention (install_packed_attention)')

    def get_seq_length(self, layer_idx=0):
        return self.length
