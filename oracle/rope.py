"""Rotate-half RoPE and its cos/sin tables, restated in numpy.

Rounding contract (rotary_triton_ascend.py:19-24, identical to torch-eager
apply_rotary_pos_emb in bf16, packed_attention.py:61-65):
    y1 = bf16(bf16(x1*c1) + bf16(-x2*s1)),  y2 = bf16(bf16(x2*c2) + bf16(x1*s2)).
numpy float32 multiply/add are single IEEE round-to-nearest-even ops (no fused multiply-add),
so each line below is exactly one rounding of the reference.
"""
import numpy as np

from . import bf16


def inv_freq(head_dim, theta=1_000_000.0):
    """fp32 1 / theta**(2i/D), the default RoPE initialiser (computed in float64, rounded)."""
    exponent = np.arange(0, head_dim, 2, dtype=np.float64) / head_dim
    return (1.0 / (theta ** exponent)).astype(np.float32)


def tables(positions, inv_frequencies, dtype="bf16", scaling=1.0):
    """cos, sin rows for integer positions: angle = fp32(inv_freq * pos); emb = [f, f]
    (the talker rotary_emb at continuous.py:193, prefill_graph.py:38).
    Returns bf16 bit patterns (uint16) or fp32 values."""
    pos = np.asarray(positions, dtype=np.int64)
    angle = inv_frequencies.astype(np.float32)[None, :] * pos.reshape(-1, 1).astype(np.float32)
    cos = (np.cos(angle.astype(np.float64)) * scaling).astype(np.float32)
    sin = (np.sin(angle.astype(np.float64)) * scaling).astype(np.float32)
    cos = np.concatenate([cos, cos], axis=-1).reshape(*pos.shape, -1)
    sin = np.concatenate([sin, sin], axis=-1).reshape(*pos.shape, -1)
    if dtype == "bf16":
        return bf16.to_bits(cos), bf16.to_bits(sin)
    return cos, sin


def rope_bf16(x_bits, cos_bits, sin_bits):
    """Exact bf16 rotate-half RoPE on bit patterns; cos/sin broadcast against x."""
    x = bf16.from_bits(x_bits)
    c = bf16.from_bits(cos_bits)
    s = bf16.from_bits(sin_bits)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c1, c2, s1, s2 = c[..., :half], c[..., half:], s[..., :half], s[..., half:]
    with np.errstate(over='ignore', invalid='ignore'):  # inf/NaN inputs propagate as IEEE says
        y1 = bf16.to_bits(bf16.round_bf16(x1 * c1) + bf16.round_bf16(-(x2 * s1)))
        y2 = bf16.to_bits(bf16.round_bf16(x2 * c2) + bf16.round_bf16(x1 * s2))
    return np.concatenate([y1, y2], axis=-1)


def rope_f32(x, cos, sin):
    """fp32 rotate-half RoPE with every product and sum rounded separately (torch eager)."""
    x = np.asarray(x, dtype=np.float32)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    c1, c2 = cos[..., :half].astype(np.float32), cos[..., half:].astype(np.float32)
    s1, s2 = sin[..., :half].astype(np.float32), sin[..., half:].astype(np.float32)
    return np.concatenate([x1 * c1 + (-(x2 * s1)), x2 * c2 + x1 * s2], axis=-1)


def mrope_select(cos3, sections, interleaved=False):
    """Per-dimension selection of the (3, ...) temporal/height/width tables used by a
    sectioned multimodal RoPE (packed_attention.py:66-69 calls qwen_tts's
    apply_multimodal_rotary_pos_emb with the module's mrope_section and interleaved flag).

    * consecutive sections [t, h, w] of each half (the Qwen2-VL form);
    * interleaved (the Qwen3-Omni talker form): frequency f of each half reads axis
      a in {1, 2} when f % 3 == a and f < 3 * sections[a], and the temporal axis otherwise,
      so with [24, 20, 20] the last frequencies 60 ... 63 are temporal.

    With three equal axes every selection equals the single-axis table
    (tests/test_text_rope.py:9-22)."""
    cos3 = np.asarray(cos3)
    width = cos3.shape[-1]
    half = width // 2
    if interleaved:
        axis_of = np.zeros(half, dtype=np.int64)
        for a in (1, 2):
            for f in range(a, min(half, 3 * sections[a]), 3):
                axis_of[f] = a
    else:
        axis_of = np.concatenate([np.full(n, i % 3) for i, n in enumerate(sections)])
    axis_of = np.concatenate([axis_of, axis_of])
    assert axis_of.shape[0] == width
    out = np.empty(cos3.shape[1:], dtype=cos3.dtype)
    for d in range(width):
        out[..., d] = cos3[axis_of[d], ..., d]
    return out
