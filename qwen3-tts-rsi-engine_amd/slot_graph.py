"""The talker's decode step over the slot arena, captured in one HIP graph.

Drop-in for the reference's ``SlotGraph`` (qwen3_tts_engine/continuous.py:172-230): the same
constructor ``SlotGraph(arena, batch, context_length=None, valid_length_kv=False)``, the
static ``inputs`` / ``positions`` / ``rotary`` buffers of the graph batch, a ``SlotCache``
over the arena, ``compute`` (every decoder layer on one token per slot, then the final norm),
``capture``, ``run(inputs, positions, rotary)`` returning a copy of the output, and
``close``.

How it differs from the reference's procedure, for the GPU:

* the ``(batch, 1, 1, context)`` additive mask ``j <= positions[b]`` (continuous.py:191-192)
  is only built when some decoder layer's attention is not a ``PackedAttention``.  Wrapped
  layers bound every request's keys by the cache's positions inside the kernel (fused: one
  launch per layer doing RoPE, the K/V write and ragged attention), so the mask would be a
  per-step tensor nobody reads;
* warm-up and capture run with every position at -1.  The kernels write nothing for a
  request without a valid position, so no arena row is touched while the graph is recorded,
  and nothing has to be saved and restored afterwards (the reference writes position 0 of
  slots ``[:batch]`` in its warm-up and capture passes and copies those rows back,
  continuous.py:201-216).  Replays read the positions buffer as ``run`` fills it;
* capture is one eager pass (lazy library state: workspaces, GEMM heuristics) and then the
  recording on torch's own capture stream.
"""
from __future__ import annotations

import torch

from .packed_attention import PackedAttention
from .slots import SlotCache


class SlotGraph:
    def __init__(self, arena, batch, context_length=None, valid_length_kv=False):
        context = arena.capacity if context_length is None else context_length
        if not 1 <= context <= arena.capacity:
            raise ValueError("Attention context must fit the KV arena")
        self.arena = arena
        self.batch = batch
        self.context_length = context
        self.reference = talker = arena.reference
        weight = next(talker.parameters())
        self.inputs = weight.new_zeros(batch, 1, talker.config.hidden_size)
        self.positions = torch.zeros(batch, device=weight.device, dtype=torch.long)
        self.rotary = torch.zeros(3, batch, 1, device=weight.device, dtype=torch.long)
        self.cache = SlotCache(arena, self.positions, context, valid_length_kv)
        # keys the (optional) mask spans: the whole arena for valid-length attention, else the
        # context view the cache returns (continuous.py:184)
        width = arena.capacity if valid_length_kv else context
        self._keys = torch.arange(width, device=weight.device)
        self._needs_mask = not all(isinstance(layer.self_attn, PackedAttention) for layer in talker.layers)
        self.graph = None
        self.output = None

    def _mask(self, dtype):
        if not self._needs_mask:
            return None
        visible = self._keys[None, :] <= self.positions[:, None]
        mask = torch.full(visible.shape, torch.finfo(dtype).min, dtype=dtype, device=visible.device)
        return mask.masked_fill(visible, 0)[:, None, None, :]

    def compute(self):
        """One decode step of the current buffers; returns the final-norm hidden states."""
        talker = self.reference
        self.cache.prepare()
        hidden = self.inputs
        mask = self._mask(hidden.dtype)
        tables = talker.rotary_emb(hidden, self.rotary)
        for layer in talker.layers:
            hidden = layer(hidden, attention_mask=mask, position_ids=self.rotary[0],
                           past_key_values=self.cache, output_attentions=False, use_cache=True,
                           cache_position=self.positions, position_embeddings=tables)[0]
        return talker.norm(hidden)

    def capture(self):
        device = self.inputs.device
        with torch.inference_mode():
            self.positions.fill_(-1)  # no request: nothing is written while recording
            self.compute()
            torch.cuda.synchronize(device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                output = self.compute()
            torch.cuda.synchronize(device)
            self.positions.zero_()
        self.graph, self.output = graph, output

    def run(self, inputs, positions, rotary):
        with torch.inference_mode():
            self.inputs.copy_(inputs)
            self.positions.copy_(positions)
            self.rotary.copy_(rotary)
            self.graph.replay()
            return self.output.clone()

    def close(self):
        torch.cuda.synchronize(self.inputs.device)
        if self.graph is not None:
            self.graph.reset()
            self.graph = None
