"""MI355X (gfx950) continuous-batching attention path of the Qwen3-TTS engine.

Host side in PyTorch-ROCm with the reference's call signatures; every computation runs in
hand-written HIP kernels behind the C ABI of ``libq3t_amd.so`` (include/qwen3tts_amd.h).

Modules
  batching        decode_batch_size                      (batching.py of the reference)
  packed_kv       copy_packed_prefix                     (packed_kv.py)
  kv_write        write / write_tokens                   (kv_triton_ascend.py, SlotCache.update)
  rotary          rotary / rope_tables                   (rotary_triton_ascend.py, rotary_emb)
  attention       attention / decode_attention / decode_step / decode_plan / decode_grid_for /
                  prefill_attention
                                                         (npu_attention.py, SDPA dispatch)
  slots           SlotArena / SlotCache / PredictorCache (continuous.py, predictor.py)
  packed_attention PackedAttention / install_packed_attention / restore_modules
  prefill         varlen prefill of packed prompts       (prefill_graph.py)
  scheduler       integer slot state of continuous batching (continuous.py tick/admit)
  slot_graph      SlotGraph: the graph-captured talker decode step (continuous.py SlotGraph)
  prefill_graph   PrefillGraph / pad_prefill_batch: the graph-captured padded prefill
                                                         (prefill_graph.py)
"""
from . import _lib
from .batching import decode_batch_size
from .packed_kv import copy_packed_prefix, copy_rows
from .kv_write import write, write_tokens
from .rotary import rotary, rope_tables, inverse_frequencies
from .attention import (attention, decode_attention, decode_step, decode_grid_for, decode_plan,
                        plan_shape, prefill_attention, reset_workspaces)
from .prefill import prefill_rope_write, prefill_step
from .packed_attention import PackedAttention, install_packed_attention, restore_modules
from .scheduler import SlotScheduler, DecodeBatch
from .slots import SlotArena, SlotCache, PredictorCache, PrefillCache, grow_arena
from .slot_graph import SlotGraph
from .prefill_graph import PrefillGraph, pad_prefill_batch

__all__ = [
    "decode_batch_size", "copy_packed_prefix", "copy_rows", "write", "write_tokens", "rotary",
    "rope_tables", "inverse_frequencies", "attention", "decode_attention", "decode_step", "decode_grid_for",
    "decode_plan",
    "plan_shape", "reset_workspaces",
    "prefill_attention", "prefill_rope_write", "prefill_step", "PackedAttention",
    "install_packed_attention", "restore_modules", "SlotScheduler", "DecodeBatch", "SlotArena",
    "SlotCache", "PredictorCache", "PrefillCache", "grow_arena", "SlotGraph", "PrefillGraph",
    "pad_prefill_batch", "library",
]

library = _lib.library
