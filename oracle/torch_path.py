"""The reference's torch decode layer on the CPU: the timed CPU baseline and a second,
independent check of the numpy oracle.

One talker attention layer as the reference runs it without native kernels:
  RoPE      apply_rotary_pos_emb, eager (packed_attention.py:61-65)
  KV write  Tensor.scatter_ at positions (continuous.py:164-166)
  mask      0 / finfo.min for j <= pos[b] over the whole context (continuous.py:191-192)
  attention scaled_dot_product_attention with KV heads repeated per query group
            (transformers' sdpa path, as probe_gqa_operator.py:54-56 checks it)
"""
import torch


def rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary(q, k, cos, sin):
    """q (B, Hq, S, D), k (B, Hkv, S, D), cos/sin (B, S, D): eager rotate-half RoPE."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def decode_layer(query, key, value, cos, sin, arena_keys, arena_values, positions, context=None,
                 scale=None):
    """query (B, 1, Hq, D), key/value (B, 1, Hkv, D) BSND rows; cos/sin (B, 1, D);
    arena planes (slots, Hkv, C, D) updated in place.  Returns (B, 1, Hq, D)."""
    batch, _, q_heads, head_dim = query.shape
    kv_heads = key.shape[2]
    context = arena_keys.shape[2] if context is None else context
    q, k = apply_rotary(query.transpose(1, 2), key.transpose(1, 2), cos, sin)
    v = value.transpose(1, 2)
    index = positions.view(batch, 1, 1, 1).expand(batch, kv_heads, 1, head_dim)
    target_k, target_v = arena_keys[:batch], arena_values[:batch]
    target_k.scatter_(2, index, k)
    target_v.scatter_(2, index, v)
    allowed = torch.arange(context)[None, :] <= positions[:, None]
    mask = torch.where(allowed, 0.0, torch.finfo(query.dtype).min).to(query.dtype)[:, None, None, :]
    group = q_heads // kv_heads
    keys = target_k[:, :, :context].repeat_interleave(group, dim=1)
    values = target_v[:, :, :context].repeat_interleave(group, dim=1)
    out = torch.nn.functional.scaled_dot_product_attention(
        q, keys, values, attn_mask=mask, scale=head_dim ** -0.5 if scale is None else scale)
    return out.transpose(1, 2)
