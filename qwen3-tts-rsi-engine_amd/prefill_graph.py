"""Graph-captured padded prefill of a prompt batch.

Drop-in for the reference's ``pad_prefill_batch`` and ``PrefillGraph``
(qwen3_tts_engine/prefill_graph.py:6-78): the same constructor, ``capture`` / ``run`` /
``close`` contract, outputs (the last valid token's hidden state and logits of each row, and
the per-layer KV of the batch) and ``packed_cache`` layout ``(2L, Bp, Hkv, Lp, D)``, keys
first, which ``SlotArena.load_packed`` copies into the arena (continuous.py:468-469).

The computation is laid out for the GPU instead of following the reference's steps:

* the reference builds a ``(Bp, 1, Lp, Lp)`` additive key-valid and causal mask
  (prefill_graph.py:36-37) and a ``DynamicCache`` whose per-layer tensors are stacked into
  ``packed_cache`` after the last layer (:47-49).  Here the rows of a padded batch are
  right-padded prompts, so key-valid and causal is "causal over the row's first n_b keys":
  every layer passes the row lengths (``mask.sum(-1)``, a device tensor, so the same graph
  serves any mask) to the MFMA prefill kernel, which skips the tiles above the diagonal and
  needs no mask tensor;
* each layer's RoPE and K/V write is one prologue kernel writing straight into that layer's
  planes of the packed buffer, so there is no per-layer concatenation and no final stack.

The talker's attention modules must have been swapped for ``PackedAttention``
(``install_packed_attention``): they recognise the ``PrefillCache`` the layers receive.
"""
from __future__ import annotations

import torch

from .packed_attention import PackedAttention
from .slots import PrefillCache


def pad_prefill_batch(embeddings, mask, batch):
    """Pad a prompt batch with ``batch - len(embeddings)`` dummy rows: zero embeddings, an
    all-ones mask (a full-length dummy prompt, never admitted as a request)
    (prefill_graph.py:6-15)."""
    extra = batch - embeddings.shape[0]
    if extra < 0 or mask.shape != embeddings.shape[:2]:
        raise ValueError('Prefill batch or attention-mask shape is invalid')
    if extra == 0:
        return embeddings, mask
    embeddings = torch.nn.functional.pad(embeddings, (0, 0, 0, 0, 0, extra))
    mask = torch.nn.functional.pad(mask, (0, 0, 0, extra), value=1)
    return embeddings, mask


def _attention_config(model):
    """(layers, kv_heads, head_dim) of the talker's decoder."""
    config = model.config
    kv_heads = getattr(config, 'num_key_value_heads', None)
    head_dim = getattr(config, 'head_dim', None)
    return len(model.layers), kv_heads, head_dim


class PrefillGraph:
    """One captured prefill of ``batch`` prompts right-padded to ``length`` tokens."""

    def __init__(self, talker, batch, length, packed_kv=False):
        model = talker.model
        if not any(isinstance(m, PackedAttention) for m in model.modules()):
            raise ValueError('PrefillGraph needs the talker attention swapped by install_packed_attention')
        weight = next(talker.parameters())
        layers, kv_heads, head_dim = _attention_config(model)
        self.talker = talker
        self.batch, self.length, self.packed_kv = batch, length, packed_kv
        self.inputs = weight.new_zeros(batch, length, talker.config.hidden_size)
        self.mask = torch.ones(batch, length, device=weight.device, dtype=torch.long)
        self.cache = PrefillCache(layers, batch, length, kv_heads, head_dim, weight.device, weight.dtype)
        self.packed_cache = None
        self._rows = torch.arange(batch, device=weight.device)
        self._positions = torch.arange(length, device=weight.device)
        self.graph = None
        self._outputs = None

    def compute(self):
        """Eager forward of the current inputs: (last hidden (B, 1, H), logits (B, V), cache)."""
        model = self.talker.model
        valid = self.mask.sum(-1)
        self.cache.kv_lens.copy_(valid)
        # positions 0 ... n-1 of each prompt, padding at 1, on all three rotary axes
        # (prefill_graph.py:34-35)
        ids = (self.mask.cumsum(-1) - 1).masked_fill(self.mask == 0, 1)
        rotary = model.rotary_emb(self.inputs, ids[None].expand(3, -1, -1))
        hidden = self.inputs
        for layer in model.layers:
            hidden = layer(hidden, attention_mask=None, position_ids=ids, past_key_values=self.cache,
                           output_attentions=False, use_cache=True, cache_position=self._positions,
                           position_embeddings=rotary)[0]
        last = model.norm(hidden)[self._rows, valid - 1].unsqueeze(1)
        logits = self.talker.codec_head(last)[:, -1]
        if self.packed_kv:
            self.packed_cache = self.cache.packed
        return last, logits, self.cache

    def capture(self):
        """One eager pass (lazy library state: decode workspaces, GEMM heuristics), then the
        captured pass on torch's capture stream."""
        with torch.inference_mode():
            self.compute()
            torch.cuda.synchronize(self.inputs.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                outputs = self.compute()
        self.graph, self._outputs = graph, outputs

    def run(self, embeddings, mask):
        """Replay on new prompts; the hidden states and logits are copies (later replays do
        not change them), the cache is this graph's own (copy its rows into the arena before
        the next replay, as continuous.py:465-471 does)."""
        with torch.inference_mode():
            self.inputs.copy_(embeddings)
            self.mask.copy_(mask)
            self.graph.replay()
            hidden, logits, cache = self._outputs
            return hidden.clone(), logits.clone(), cache

    def close(self):
        torch.cuda.synchronize(self.inputs.device)
        if self.graph is not None:
            self.graph.reset()
            self.graph = None
        self.packed_cache = None
