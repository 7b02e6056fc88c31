"""Graph-captured decode step of the talker over the slot arena.

Drop-in for the reference's ``SlotGraph`` (qwen3_tts_engine/continuous.py:170-229) on HIP
graphs: static input, position and rotary buffers of the graph batch; ``compute`` builds the
``j <= pos[b]`` mask (0 / finfo.min, continuous.py:189-190), the rotary tables and runs every
decoder layer over a ``SlotCache``; ``capture`` warms up three times on a side stream,
captures one ``compute`` and then restores the arena rows at position 0 of slots
``[:batch]``, which the warm-up and capture passes wrote with their zero positions
(continuous.py:199-215); ``run`` copies the step's inputs into the static buffers, replays
and returns a copy of the output (continuous.py:217-223).

With ``install_packed_attention`` applied to the talker, every layer's attention inside the
graph is one fused ``decode_step`` launch (RoPE of q and k, the K/V write at the positions,
ragged GQA attention) between the module's own QKV projection / q-k norms and ``o_proj``.
"""
from __future__ import annotations

import torch

from .packed_kv import copy_rows
from .slots import SlotCache


class SlotGraph:
    def __init__(self, arena, batch, context_length=None, valid_length_kv=False):
        self.arena = arena
        self.batch = batch
        self.context_length = arena.capacity if context_length is None else context_length
        if not 1 <= self.context_length <= arena.capacity:
            raise ValueError("Attention context must fit the KV arena")
        self.reference = arena.reference
        weight = next(self.reference.parameters())
        self.inputs = torch.zeros(batch, 1, self.reference.config.hidden_size, device=weight.device,
                                  dtype=weight.dtype)
        self.positions = torch.zeros(batch, device=weight.device, dtype=torch.long)
        self.rotary = torch.zeros(3, batch, 1, device=weight.device, dtype=torch.long)
        self.indices = torch.arange(arena.capacity if valid_length_kv else self.context_length,
                                    device=weight.device)
        self.cache = SlotCache(arena, self.positions, self.context_length, valid_length_kv)
        self.graph = None
        self.output = None

    def compute(self):
        self.cache.prepare()
        hidden = self.inputs
        allowed = self.indices.view(1, -1) <= self.positions.view(-1, 1)
        mask = torch.where(allowed, 0.0, torch.finfo(hidden.dtype).min).to(hidden.dtype)[:, None, None, :]
        rotary = self.reference.rotary_emb(hidden, self.rotary)
        for layer in self.reference.layers:
            hidden = layer(hidden, attention_mask=mask, position_ids=self.rotary[0],
                           past_key_values=self.cache, output_attentions=False, use_cache=True,
                           cache_position=self.positions, position_embeddings=rotary)[0]
        return self.reference.norm(hidden)

    @torch.inference_mode()
    def capture(self):
        device = self.inputs.device
        saved = [(k[:self.batch, :, 0].clone(), v[:self.batch, :, 0].clone())
                 for k, v in zip(self.arena.keys, self.arena.values)]
        stream = torch.cuda.Stream(device=device)  # default priority
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            for _ in range(3):
                self.compute()
        torch.cuda.current_stream(device).wait_stream(stream)
        torch.cuda.synchronize(device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=stream):
            self.output = self.compute()
        for layer, (keys, values) in enumerate(saved):
            copy_rows(self.arena.keys[layer][:self.batch, :, 0], keys)
            copy_rows(self.arena.values[layer][:self.batch, :, 0], values)

    @torch.inference_mode()
    def run(self, inputs, positions, rotary):
        self.inputs.copy_(inputs)
        self.positions.copy_(positions)
        self.rotary.copy_(rotary)
        self.graph.replay()
        return self.output.clone()

    def close(self):
        torch.cuda.synchronize(self.inputs.device)
        if self.graph is not None:
            self.graph.reset()
