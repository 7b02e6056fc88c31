"""Varlen prefill of packed prompts on the GPU.

The reference pads a prompt batch to (Bp, Lp) and runs causal self-attention over it,
then copies each request's valid KV prefix into its arena slot
(PrefillGraph.compute, qwen3_tts_engine/prefill_graph.py:31-50; ContinuousModel.admit_batch,
continuous.py:425-473 with copy_packed_prefix, packed_kv.py:6-31).  Here the valid rows are
packed by ``cu_seqlens`` (no padding), the prologue writes rotated keys straight into the
arena slots, and the attention reads them from there:

* ``prefill_rope_write`` - RoPE of query and key rows at positions 0 ... len-1 of each
  request (bf16-exact, as ``rotary``) and the paired K/V write into the arena
  (kernel ``q3t_prefill_rope_write``); with ``rotate_query=False`` the keys and values only,
  with ``value=None`` the keys only;
* ``prefill_attention`` - varlen causal GQA on bf16 MFMA tiles (kernel
  ``q3t_prefill_attention``, re-exported from ``attention``); given cos/sin it rotates the
  raw query rows as it loads them;
* ``prefill_step`` - one layer: the key prologue, then attention over the raw queries with
  their RoPE applied in the attention kernel (no rotated copy of the queries is written),
  reading the values from the projection's rows while the same launch copies them into the
  arena.
"""
import torch

from . import _lib
from .attention import prefill_attention


def _check_packed(name, t, tokens, heads, width):
    if t.ndim != 3 or t.shape[0] != tokens or t.shape[1] != heads or t.shape[2] != width:
        raise ValueError(f'{name} must be ({tokens}, {heads}, {width}) token rows')
    if t.dtype != torch.bfloat16 or t.stride(2) != 1:
        raise ValueError(f'{name} must be bf16 with unit stride along head_dim')


def prefill_rope_write(query, key, value, cos, sin, cu_seqlens, key_arena, value_arena, *,
                       kv_slots=None, q_out=None, rotate_query=True):
    """query (T, Hq, D), key/value (T, Hkv, D) packed by cu_seqlens (B+1, int32 device);
    cos/sin (T, D) rows of each token's position; arena planes (slots, Hkv, C, D).
    Writes rotated keys and values at positions 0 ... len_b-1 of slot b (or kv_slots[b])
    and returns the rotated queries (T, Hq, D), or None with ``rotate_query=False`` (the
    query rows are then not touched).  With ``value=None`` only the keys are written (the
    values are left to ``prefill_attention(new_values=...)``)."""
    if query.ndim != 3 or key.ndim != 3:
        raise ValueError('expected packed (tokens, heads, head_dim) rows')
    tokens, q_heads, head_dim = query.shape
    kv_heads = key.shape[1]
    _check_packed('query', query, tokens, q_heads, head_dim)
    _check_packed('key', key, tokens, kv_heads, head_dim)
    if value is not None:
        _check_packed('value', value, tokens, kv_heads, head_dim)
    if cos.shape != (tokens, head_dim) or sin.shape != cos.shape or cos.dtype != torch.bfloat16 \
            or sin.dtype != torch.bfloat16 or cos.stride(1) != 1 or sin.stride() != cos.stride():
        raise ValueError('cos/sin must be bf16 (tokens, head_dim) rows')
    if (key_arena.ndim != 4 or key_arena.shape != value_arena.shape or key_arena.shape[1] != kv_heads
            or key_arena.shape[3] != head_dim or key_arena.dtype != torch.bfloat16
            or value_arena.dtype != torch.bfloat16 or key_arena.stride() != value_arena.stride()
            or key_arena.stride(3) != 1):
        raise ValueError('arena planes must be matching bf16 (slots, kv_heads, capacity, head_dim) views')
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError('cu_seqlens must be an int32 (B+1,) tensor')
    batch = cu_seqlens.numel() - 1
    if kv_slots is not None and (kv_slots.dtype != torch.int64 or kv_slots.shape != (batch,)):
        raise ValueError('kv_slots must be an int64 (B,) tensor')
    if kv_slots is None and key_arena.shape[0] < batch:
        raise ValueError('the arena has fewer slots than requests')
    device = _lib.require_gpu(query, key, cos, sin, cu_seqlens, key_arena, value_arena,
                              *([value] if value is not None else []),
                              *([kv_slots] if kv_slots is not None else []))
    if not rotate_query:
        if q_out is not None:
            raise ValueError('q_out is only written with rotate_query=True')
    elif q_out is None:
        q_out = torch.empty_like(query, memory_format=torch.contiguous_format)
    else:
        _check_packed('q_out', q_out, tokens, q_heads, head_dim)
    a = _lib.PrefillRopeWriteArgs()
    a.batch, a.total_tokens, a.q_heads, a.kv_heads = batch, tokens, q_heads, kv_heads
    a.head_dim, a.capacity = head_dim, key_arena.shape[2]
    a.cu_seqlens = cu_seqlens.data_ptr()
    a.query, (a.q_stride_t, a.q_stride_h) = query.data_ptr(), query.stride()[:2]
    a.key, (a.k_stride_t, a.k_stride_h) = key.data_ptr(), key.stride()[:2]
    if value is not None:
        a.value, (a.v_stride_t, a.v_stride_h) = value.data_ptr(), value.stride()[:2]
    a.cos, a.sin, a.cs_stride_t = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    if q_out is not None:
        a.q_out, (a.qo_stride_t, a.qo_stride_h) = q_out.data_ptr(), q_out.stride()[:2]
    a.arena_keys = key_arena.data_ptr()
    if value is not None:
        a.arena_values = value_arena.data_ptr()
    a.a_stride_b, a.a_stride_h, a.a_stride_t = key_arena.stride()[:3]
    if kv_slots is not None:
        a.kv_slots = kv_slots.data_ptr()
    status = _lib.library().q3t_prefill_rope_write(a, _lib.stream_handle(device))
    _lib.check(status, 'prefill rope/write')
    return q_out


def prefill_step(query, key, value, cos, sin, cu_seqlens, max_seqlen, key_arena, value_arena, *,
                 kv_slots=None, scale=None, out=None):
    """One prefill layer over packed prompts: RoPE, arena write, causal GQA.
    Returns the attention output (T, Hq, D).  Two launches: the rotated keys into the arena,
    then attention, which rotates the queries as it loads them, reads the values from
    ``value`` and copies them into the arena."""
    prefill_rope_write(query, key, None, cos, sin, cu_seqlens, key_arena, value_arena,
                       kv_slots=kv_slots, rotate_query=False)
    return prefill_attention(query, key_arena, value_arena, cu_seqlens, max_seqlen, scale=scale,
                             kv_slots=kv_slots, out=out, cos=cos, sin=sin, new_values=value)
