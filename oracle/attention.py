"""Softmax attention restated in float64 numpy.

Decode: out[b, s, h] = softmax(q[b, s, h] . K[b, h//G, :L_b]^T * scale + mask) . V[b, h//G, :L_b]
with L_b = positions[b] + 1 (SlotGraph.compute's mask j <= pos[b], continuous.py:191-192,
reaching SDPA through PackedAttention.forward, packed_attention.py:75-84).  With several
queries per request and no mask, query s sits at position p_b - S + 1 + s and is causal
(the predictor's 2x2 step, continuous.py:39-40; npu_attention.py:17-18).  A mask is
additive, or bool with True = attend, as torch SDPA takes it.

Prefill: every request of a cu_seqlens batch attends causally to its own keys
(prefill_graph.py:34-37 for the valid rows of a padded batch).
"""
import numpy as np


def _softmax_rows(scores):
    m = np.max(scores, axis=-1, keepdims=True)
    e = np.exp(scores - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def _mask_add(mask):
    mask = np.asarray(mask)
    if mask.dtype == np.bool_:
        return np.where(mask, 0.0, -np.inf)
    return mask.astype(np.float64)


def decode_attention(q, keys, values, positions, scale, mask=None):
    """q (B, S, Hq, D); keys/values (B, Hkv, ctx, D); positions (B,); mask None or
    (B, S, ctx).  Returns float64 (B, S, Hq, D)."""
    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    batch, qlen, q_heads, head_dim = q.shape
    group = q_heads // keys.shape[1]
    out = np.zeros((batch, qlen, q_heads, head_dim))
    for b in range(batch):
        length = int(positions[b]) + 1
        k = np.repeat(keys[b, :, :length], group, axis=0)      # (Hq, L, D)
        v = np.repeat(values[b, :, :length], group, axis=0)
        scores = np.einsum('shd,hld->shl', q[b], k) * scale     # (S, Hq, L)
        if mask is not None:
            scores = scores + _mask_add(mask[b][:, :length])[:, None, :]
        elif qlen > 1:
            limit = length - qlen + np.arange(qlen)             # last visible key per query
            visible = np.arange(length)[None, :] <= limit[:, None]
            scores = np.where(visible[:, None, :], scores, -np.inf)
        out[b] = np.einsum('shl,hld->shd', _softmax_rows(scores), v)
    return out


def prefill_attention(q, keys, values, cu_seqlens, scale, slots=None):
    """q (T, Hq, D) packed by cu_seqlens; keys/values (slots, Hkv, capacity, D) holding
    request b's keys at positions 0 ... len_b - 1 of slot b (or slots[b])."""
    q = np.asarray(q, dtype=np.float64)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    q_heads = q.shape[1]
    out = np.zeros_like(q)
    for b in range(len(cu) - 1):
        n = int(cu[b + 1] - cu[b])
        if n == 0:
            continue
        slot = b if slots is None else int(slots[b])
        group = q_heads // keys.shape[1]
        k = np.repeat(np.asarray(keys[slot, :, :n], dtype=np.float64), group, axis=0)
        v = np.repeat(np.asarray(values[slot, :, :n], dtype=np.float64), group, axis=0)
        qb = q[cu[b]:cu[b + 1]]                                 # (n, Hq, D)
        scores = np.einsum('thd,hld->thl', qb, k) * scale
        causal = np.arange(n)[None, :] <= np.arange(n)[:, None]
        scores = np.where(causal[:, None, :], scores, -np.inf)
        out[cu[b]:cu[b + 1]] = np.einsum('thl,hld->thd', _softmax_rows(scores), v)
    return out
