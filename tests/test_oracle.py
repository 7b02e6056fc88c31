"""Pins of the CPU oracle against independent implementations (torch CPU ops), the
reference's own fixtures and known answers, closed forms and brute force on tiny inputs.

Nothing here retypes an oracle formula: every check compares the oracle with something that
was computed another way.  Runs on the CPU only.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import kv as okv
from oracle import norm as onorm
from oracle import rope as orope
from oracle import scheduler as osched


def _torch_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _is_nan(bits):
    return (bits & 0x7FFF) > 0x7F80


def _same_bf16(a, b):
    """Equal bit patterns, NaN payloads aside: torch's vectorised CPU cast writes NaN as
    0xffff while c10::BFloat16 (and the oracle, and the GPU kernels) write 0x7fc0."""
    return np.array_equal(_is_nan(a), _is_nan(b)) and np.array_equal(a[~_is_nan(a)], b[~_is_nan(b)])


# ---- bf16 rounding -----------------------------------------------------------------------

def test_bf16_rounding_matches_torch_casts():
    """Round-to-nearest-even with canonical NaN, against torch's own fp32 -> bf16 cast."""
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    # every rounding boundary class: exact ties (low half 0x8000), just above/below, zeros
    ties = (bits & 0xFFFF0000) | rng.choice(np.array([0x8000, 0x7FFF, 0x8001, 0, 0xFFFF], dtype=np.uint32),
                                            size=bits.size)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001,
                        0x00000001, 0x007FFFFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x3F808000,
                        0x3F818000], dtype=np.uint32)
    for u in (bits, ties, special):
        x = u.view(np.float32)
        expected = _torch_bits(torch.from_numpy(x.copy()).bfloat16())
        got = obf16.to_bits(x)
        assert _same_bf16(got, expected)
        assert np.all(got[_is_nan(got)] == 0x7FC0)


def test_bf16_from_bits_is_exact():
    b = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    via_torch = torch.from_numpy(b.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    got = obf16.from_bits(b)
    finite = np.isfinite(via_torch)
    assert np.array_equal(got[finite], via_torch[finite])
    assert np.array_equal(np.isnan(got), np.isnan(via_torch))


# ---- RoPE --------------------------------------------------------------------------------

def _torch_rope(x, cos, sin):
    """torch-eager rotate-half RoPE (the reference's apply_rotary_pos_emb arithmetic)."""
    half = x.shape[-1] // 2
    rotated = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rotated * sin


@pytest.mark.parametrize("width", [64, 128])
def test_rope_bf16_bit_exact_vs_torch_eager(width):
    gen = torch.Generator().manual_seed(1)
    x = (torch.randn(8, 5, 16, width, generator=gen) * 3).bfloat16()
    pos = torch.randint(0, 4096, (8, 5), generator=gen)
    cos_b, sin_b = orope.tables(pos.numpy(), orope.inv_freq(width))
    cos = torch.from_numpy(cos_b.view(np.int16)).view(torch.bfloat16)[:, :, None, :]
    sin = torch.from_numpy(sin_b.view(np.int16)).view(torch.bfloat16)[:, :, None, :]
    expected = _torch_bits(_torch_rope(x, cos, sin))
    got = orope.rope_bf16(_torch_bits(x), cos_b[:, :, None, :], sin_b[:, :, None, :])
    assert np.array_equal(got, expected)


def test_rope_bf16_special_values_vs_torch_eager():
    vals = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e38, -1e38, 1e-40, 3.0, -2.5], dtype=np.float32)
    rng = np.random.default_rng(2)
    x = torch.from_numpy(rng.choice(vals, size=(64, 128)).astype(np.float32)).bfloat16()
    c = torch.from_numpy(rng.choice(vals, size=(64, 128)).astype(np.float32)).bfloat16()
    s = torch.from_numpy(rng.choice(vals, size=(64, 128)).astype(np.float32)).bfloat16()
    expected = _torch_bits(_torch_rope(x, c, s))
    got = orope.rope_bf16(_torch_bits(x), _torch_bits(c), _torch_bits(s))
    assert _same_bf16(got, expected) and _is_nan(got).any()


def test_rope_f32_bit_exact_vs_torch_eager():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(4, 3, 8, 128, generator=gen)
    cos = torch.randn(4, 3, 1, 128, generator=gen)
    sin = torch.randn(4, 3, 1, 128, generator=gen)
    expected = _torch_rope(x, cos, sin).numpy()
    got = orope.rope_f32(x.numpy(), cos.numpy(), sin.numpy())
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32))


def test_rope_position_zero_is_identity_and_rotation_preserves_norm():
    inv = orope.inv_freq(128)
    c0, s0 = orope.tables(np.zeros(3, dtype=np.int64), inv, dtype="f32")
    x = np.random.default_rng(4).standard_normal((3, 128)).astype(np.float32)
    assert np.array_equal(orope.rope_f32(x, c0, s0), x)
    c, s = orope.tables(np.array([1, 77, 4095]), inv, dtype="f32")
    y = orope.rope_f32(x, c, s)
    assert np.allclose(np.linalg.norm(y.astype(np.float64), axis=-1),
                       np.linalg.norm(x.astype(np.float64), axis=-1), rtol=1e-6)


def test_rope_is_complex_multiplication():
    """Rotate-half pairs dimension i with i + D/2: (x1 + i x2) * exp(i theta)."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 64)).astype(np.float32)
    pos = np.array([0, 1, 2, 100, 1000, 65535])
    c, s = orope.tables(pos, orope.inv_freq(64), dtype="f32")
    y = orope.rope_f32(x, c, s).astype(np.float64)
    z = (x[:, :32].astype(np.float64) + 1j * x[:, 32:]) * (c[:, :32].astype(np.float64) + 1j * s[:, :32])
    assert np.allclose(y[:, :32], z.real, atol=1e-5) and np.allclose(y[:, 32:], z.imag, atol=1e-5)


def test_inverse_frequencies_match_torch_initialiser_within_one_ulp():
    """The default RoPE initialiser computes theta ** (2i/D) with torch's fp32 pow, which is
    not correctly rounded; the oracle rounds the float64 value.  Both agree to one ulp."""
    for width in (64, 128):
        torch_inv = (1.0 / (1e6 ** (torch.arange(0, width, 2, dtype=torch.int64).float() / width))).numpy()
        ulps = np.abs(orope.inv_freq(width).view(np.int32).astype(np.int64) - torch_inv.view(np.int32))
        assert ulps.max() <= 1


def test_rope_tables_match_torch_default_rope():
    """cos/sin of positions * inv_freq (torch fp32 angle, torch cos/sin), within one bf16 ulp."""
    width = 128
    inv = torch.from_numpy(orope.inv_freq(width))
    pos = torch.tensor([0, 1, 5, 37, 120, 256, 1023, 4095, 30000])
    angle = pos[:, None].float() * inv[None, :]
    emb = torch.cat([angle, angle], dim=-1)
    cos_t, sin_t = _torch_bits(emb.cos().bfloat16()), _torch_bits(emb.sin().bfloat16())
    cos_o, sin_o = orope.tables(pos.numpy(), inv.numpy())
    for a, b in ((cos_o, cos_t), (sin_o, sin_t)):
        d = np.abs(a.astype(np.int32) - b.astype(np.int32))
        assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_mrope_equal_axes_is_the_text_rope():
    """tests/test_text_rope.py:9-22: three equal position axes reduce MRoPE to plain RoPE."""
    inv = orope.inv_freq(128)
    c, _ = orope.tables(np.arange(12).reshape(3, 4), inv, dtype="f32")
    cos3 = np.stack([c, c, c])
    for sections, interleaved in (([24, 20, 20], False), ([16, 24, 24], False), ([24, 20, 20], True)):
        assert np.array_equal(orope.mrope_select(cos3, sections, interleaved), c)


def _axis_tables(width=128):
    """(3, 1, width) tables whose every entry names its own axis and dimension: axis a,
    dimension d holds 1000 a + d, so a selection shows which axis each dimension read."""
    d = np.arange(width, dtype=np.float64)
    return np.stack([1000.0 * a + d for a in range(3)])[:, None, :]


def test_mrope_sections_hand_computed():
    """[24, 20, 20], written out by hand.  Sectioned: dimensions 0-23 temporal, 24-43
    height, 44-63 width, the same again for 64-127.  Interleaved: frequencies cycle
    T, H, W from 0 to 59 (3 x 20), and the remaining 60-63 are temporal."""
    sel = orope.mrope_select(_axis_tables(), [24, 20, 20])[0]
    axes = (sel // 1000).astype(int)
    expected_half = [0] * 24 + [1] * 20 + [2] * 20
    assert axes.tolist() == expected_half + expected_half
    sel = orope.mrope_select(_axis_tables(), [24, 20, 20], interleaved=True)[0]
    axes = (sel // 1000).astype(int)
    expected_half = [0, 1, 2] * 20 + [0, 0, 0, 0]
    assert axes.tolist() == expected_half + expected_half
    assert np.array_equal(sel % 1000, np.arange(128))  # every dimension keeps its own column
    # sections that do not reach the end of the cycle: [32, 16, 16] interleaved gives
    # T H W for f < 48 and T from 48 to 63
    axes = (orope.mrope_select(_axis_tables(), [32, 16, 16], interleaved=True)[0] // 1000).astype(int)
    assert axes[:64].tolist() == [0, 1, 2] * 16 + [0] * 16


def test_mrope_matches_transformers_multimodal_rope():
    """Against the installed transformers' own multimodal RoPE on unequal axes: the
    interleaved layout of the Qwen3-Omni talker (Qwen3OmniMoeTalkerRotaryEmbedding's
    apply_interleaved_mrope, acting on the (3, ..., D/2) frequencies before the
    [f, f] concatenation) and the sectioned layout of Qwen2.5-Omni's
    apply_multimodal_rotary_pos_emb."""
    omni3 = pytest.importorskip('transformers.models.qwen3_omni_moe.modeling_qwen3_omni_moe')
    omni25 = pytest.importorskip('transformers.models.qwen2_5_omni.modeling_qwen2_5_omni')
    inv = torch.from_numpy(orope.inv_freq(128))
    gen = torch.Generator().manual_seed(3)
    pos = torch.randint(0, 4000, (3, 2, 5), generator=gen)          # distinct T, H, W positions
    freqs = (pos[..., None].double() * inv.double()).float()          # (3, B, S, 64)
    for sections in ([24, 20, 20], [16, 24, 24]):
        cat = torch.cat([freqs, freqs], dim=-1)
        ours = orope.mrope_select(cat.numpy(), sections, interleaved=True)
        theirs = omni3.Qwen3OmniMoeTalkerRotaryEmbedding.apply_interleaved_mrope(
            None, freqs.clone(), sections)
        assert np.array_equal(ours, torch.cat([theirs, theirs], dim=-1).numpy())
        # sectioned: their function applies the selected tables to q and k; with q = 1 on one
        # dimension and 0 elsewhere, q * cos + rotate_half(q) * sin reads back cos
        cos = torch.cos(cat)
        sin = torch.sin(cat)
        picked = orope.mrope_select(cos.numpy(), sections)
        for d in (0, 23, 24, 43, 44, 63, 64, 100, 127):
            unit = torch.zeros(2, 1, 5, 128, dtype=torch.float32)
            unit[..., d] = 1.0
            q_embed, _ = omni25.apply_multimodal_rotary_pos_emb(unit, unit, cos.float(), sin.float(),
                                                                list(sections))
            got = q_embed[:, 0, :, d].numpy()
            assert np.array_equal(got, picked[..., d].astype(np.float32)), (sections, d)


# ---- attention ---------------------------------------------------------------------------

def _sdpa(q, k, v, mask, scale):
    """torch CPU SDPA in float64 with KV heads repeated per query group."""
    group = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1)
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale)


@pytest.mark.parametrize("group,qlen", [(1, 1), (2, 1), (4, 1), (2, 2), (4, 2)])
def test_decode_attention_matches_sdpa(group, qlen):
    gen = torch.Generator().manual_seed(10 + group + qlen)
    batch, kv_heads, ctx, width = 5, 2, 40, 16
    q = torch.randn(batch, qlen, kv_heads * group, width, generator=gen, dtype=torch.float64)
    k = torch.randn(batch, kv_heads, ctx, width, generator=gen, dtype=torch.float64)
    v = torch.randn(batch, kv_heads, ctx, width, generator=gen, dtype=torch.float64)
    positions = torch.tensor([0, 1, 17, 38, 39])[:batch]
    positions = torch.maximum(positions, torch.tensor(qlen - 1))
    got = oatt.decode_attention(q.numpy(), k.numpy(), v.numpy(), positions.numpy(), 0.3)
    for b in range(batch):
        length = int(positions[b]) + 1
        # query s sits at position p_b - qlen + 1 + s and sees keys up to it
        allowed = torch.arange(length)[None, :] <= (length - qlen + torch.arange(qlen))[:, None]
        ref = _sdpa(q[b:b + 1].transpose(1, 2), k[b:b + 1, :, :length], v[b:b + 1, :, :length],
                    allowed[None, None], 0.3)
        assert np.allclose(got[b], ref[0].transpose(0, 1).numpy(), atol=1e-12)


@pytest.mark.parametrize("kind", ["additive", "bool"])
def test_decode_attention_masks_match_sdpa(kind):
    gen = torch.Generator().manual_seed(20)
    q = torch.randn(3, 2, 4, 8, generator=gen, dtype=torch.float64)
    k = torch.randn(3, 2, 24, 8, generator=gen, dtype=torch.float64)
    v = torch.randn(3, 2, 24, 8, generator=gen, dtype=torch.float64)
    positions = np.array([23, 23, 23])
    if kind == "bool":
        mask = torch.rand(3, 2, 24, generator=gen) > 0.3
        mask[..., 0] = True
    else:
        mask = torch.randn(3, 2, 24, generator=gen, dtype=torch.float64) * 4
    got = oatt.decode_attention(q.numpy(), k.numpy(), v.numpy(), positions, 0.5, mask=mask.numpy())
    ref = _sdpa(q.transpose(1, 2), k, v, mask[:, None], 0.5).transpose(1, 2)
    assert np.allclose(got, ref.numpy(), atol=1e-12)


def test_decode_attention_closed_forms():
    rng = np.random.default_rng(6)
    k = rng.standard_normal((1, 1, 8, 4))
    v = rng.standard_normal((1, 1, 8, 4))
    # one key: the output is that value row
    q = rng.standard_normal((1, 1, 2, 4))
    assert np.allclose(oatt.decode_attention(q, k, v, [0], 1.0)[0, 0], np.repeat(v[0, :, 0], 2, axis=0))
    # equal scores (q = 0): the mean of the visible value rows
    out = oatt.decode_attention(np.zeros((1, 1, 1, 4)), k, v, [5], 1.0)
    assert np.allclose(out[0, 0, 0], v[0, 0, :6].mean(axis=0))
    # one dominant score selects its row
    kd = np.zeros((1, 1, 8, 4))
    kd[0, 0, 3] = [1, 0, 0, 0]
    out = oatt.decode_attention(np.array([[[[1000.0, 0, 0, 0]]]]), kd, v, [7], 1.0)
    assert np.allclose(out[0, 0, 0], v[0, 0, 3])


def test_decode_attention_brute_force_loops():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((2, 1, 4, 3))
    k = rng.standard_normal((2, 2, 6, 3))
    v = rng.standard_normal((2, 2, 6, 3))
    positions = [2, 5]
    got = oatt.decode_attention(q, k, v, positions, 0.7)
    for b in range(2):
        for h in range(4):
            kh = h // 2
            scores = [sum(q[b, 0, h, d] * k[b, kh, j, d] for d in range(3)) * 0.7 for j in range(positions[b] + 1)]
            m = max(scores)
            w = [math.exp(s - m) for s in scores]
            total = sum(w)
            for d in range(3):
                ref = sum(w[j] * v[b, kh, j, d] for j in range(len(w))) / total
                assert abs(got[b, 0, h, d] - ref) < 1e-12


def test_trimmed_context_equals_full_arena_under_mask():
    """tests/test_slot_context.py:30-36: attending keys 0..pos of a trimmed view equals the
    full arena under the 0/-inf context mask."""
    rng = np.random.default_rng(42)
    q = rng.standard_normal((2, 1, 2, 8))
    k = rng.standard_normal((2, 2, 256, 8))
    v = rng.standard_normal((2, 2, 256, 8))
    positions = np.array([63, 17])
    mask = np.where(np.arange(256)[None, None, :] <= positions[:, None, None], 0.0, -np.inf)
    full = oatt.decode_attention(q, k, v, [255, 255], 8 ** -0.5, mask=mask)
    trimmed = oatt.decode_attention(q, k[:, :, :64], v[:, :, :64], positions, 8 ** -0.5)
    assert np.allclose(full, trimmed, atol=1e-12)


def test_prefill_attention_matches_causal_sdpa():
    gen = torch.Generator().manual_seed(30)
    lengths = [5, 1, 17, 0, 9]
    cu = np.concatenate([[0], np.cumsum(lengths)])
    q = torch.randn(int(cu[-1]), 4, 8, generator=gen, dtype=torch.float64)
    k = torch.randn(6, 2, 32, 8, generator=gen, dtype=torch.float64)
    v = torch.randn(6, 2, 32, 8, generator=gen, dtype=torch.float64)
    slots = np.array([5, 0, 2, 1, 3])
    got = oatt.prefill_attention(q.numpy(), k.numpy(), v.numpy(), cu, 0.4, slots=slots)
    for b, n in enumerate(lengths):
        if n == 0:
            continue
        s = int(slots[b])
        ref = _sdpa(q[cu[b]:cu[b + 1]].transpose(0, 1)[None], k[s:s + 1, :, :n], v[s:s + 1, :, :n],
                    None if n == 1 else torch.ones(n, n, dtype=torch.bool).tril(), 0.4)
        assert np.allclose(got[cu[b]:cu[b + 1]], ref[0].transpose(0, 1).numpy(), atol=1e-12)


# ---- KV writes and copies ----------------------------------------------------------------

def test_kv_write_matches_torch_scatter():
    """continuous.py:164-166 writes with Tensor.scatter_ along the context axis."""
    gen = torch.Generator().manual_seed(40)
    tk = torch.randn(6, 3, 20, 8, generator=gen)
    tv = torch.randn(6, 3, 20, 8, generator=gen)
    k = torch.randn(6, 3, 1, 8, generator=gen)
    v = torch.randn(6, 3, 1, 8, generator=gen)
    pos = torch.tensor([0, 19, 7, 7, 3, 12])
    index = pos.view(6, 1, 1, 1).expand(6, 3, 1, 8)
    ek, ev = tk.clone().scatter_(2, index, k), tv.clone().scatter_(2, index, v)
    gk, gv = okv.kv_write(tk.numpy().copy(), tv.numpy().copy(), k.numpy(), v.numpy(), pos.numpy())
    assert np.array_equal(gk, ek.numpy()) and np.array_equal(gv, ev.numpy())


def test_copy_packed_prefix_reference_fixtures():
    """tests/test_packed_kv.py:9-25: arange fixtures, strided source, expected by indexing."""
    target = torch.full((4, 5, 2, 7, 3), -7.0)
    source = torch.arange(4 * 3 * 2 * 5 * 6).view(4, 3, 2, 5, 6).float()[..., ::2]
    for row, slot, length in ((2, 3, 1), (0, 1, 5), (1, 4, 3)):
        expected = target.clone()
        for layer in range(4):
            expected[layer, slot, :, :length].copy_(source[layer, row, :, :length])
        got = okv.copy_packed_prefix(target.numpy().copy(), source.numpy(), slot, row=row, length=length)
        assert np.array_equal(got, expected.numpy())


def test_capacity_rule_and_grow():
    """continuous.py:353-363 as stated: unchanged below capacity, else the larger of double
    and the next power of two above the requirement; contents preserved, tail zero."""
    assert okv.grown_capacity(512, 511) == 512
    assert okv.grown_capacity(512, 512) == 1024
    assert okv.grown_capacity(512, 1500) == 2048
    assert okv.grown_capacity(1024, 4095) == 4096
    assert okv.grown_capacity(1024, 4096) == 8192
    for cap in (64, 512, 1000):
        for req in (0, cap - 1, cap, cap + 1, 3 * cap, 10 * cap):
            new = okv.grown_capacity(cap, req)
            assert new > req or req < cap
            assert new == cap or (new >= 2 * cap and new & (new - 1) == 0 or new == 2 * cap)
    planes = [np.arange(2 * 3 * 4 * 2).reshape(2, 3, 4, 2).astype(np.int16)]
    grown = okv.grow(planes, 8)
    assert np.array_equal(grown[0][:, :, :4], planes[0]) and not grown[0][:, :, 4:].any()


# ---- scheduler integer rules -------------------------------------------------------------

def test_decode_batch_size_reference_known_answers_and_invariants():
    """tests/test_batching.py:6-19."""
    assert osched.decode_batch_size(33, 64) == 64
    assert osched.decode_batch_size(33, 64, 8) == 40
    assert osched.decode_batch_size(17, 64, 8) == 24
    for slots in (1, 2, 4, 8, 16, 32, 64):
        for step in [0] + [x for x in (1, 2, 4, 8, 16, 32, 64) if x <= slots]:
            for active in range(1, slots + 1):
                batch = osched.decode_batch_size(active, slots, step)
                assert active <= batch <= slots
                if step and active > step:
                    assert batch % step == 0 and batch - active < step
                else:
                    assert batch & (batch - 1) == 0 and (batch == active or batch // 2 < active)


@pytest.mark.parametrize("active,slots,step", [(0, 64, 8), (65, 64, 8), (1, 3, 0), (1, 64, -1),
                                               (1, 64, 3), (1, 8, 16)])
def test_decode_batch_size_rejects_invalid_geometry(active, slots, step):
    with pytest.raises(ValueError):
        osched.decode_batch_size(active, slots, step)


def test_reference_scheduler_invariants_on_a_trace():
    """Slots stay dense (no gaps), every admitted request keeps its own position sequence,
    compaction moves the last slot into the freed one, capacity only grows and always
    exceeds every position in a decode."""
    trace = osched.make_trace(seed=3, iterations=120, mean_arrivals=1.5, lengths=(5, 40), cancel_rate=0.1)
    sched = osched.ReferenceScheduler(16, initial_capacity=64, decode_bucket_step=4, bucket_kv=True)
    records = osched.drive(sched, trace, 16)
    seen_capacity = 64
    expected_pos = {}
    for record, finished, ops in records:
        if record is None:
            continue
        assert record['capacity'] >= seen_capacity
        seen_capacity = record['capacity']
        count = len(record['slots'])
        assert record['batch'] == osched.decode_batch_size(count, 16, 4)
        assert max(record['positions'][:count]) < record['capacity']
        assert 64 <= record['context'] <= record['capacity'] or record['context'] == record['capacity']
        for slot, ident in enumerate(record['slots']):
            pos = record['positions'][slot]
            if ident in expected_pos:
                assert pos == expected_pos[ident]
            expected_pos[ident] = pos + 1
        for op in ops:
            if op[0] == 'move':
                assert op[1] > op[2]


# ---- RMSNorm (q_norm / k_norm) -----------------------------------------------------------

def _torch_rms_norm(x, weight, eps):
    """The module formula in torch (CPU): fp32 row statistic, bf16 round, bf16 weight."""
    y = x.float()
    y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)
    return weight * y.to(torch.bfloat16)


def test_rms_norm_matches_torch_module_formula():
    """Within one bf16 step of torch's CPU evaluation everywhere, and bit-equal for all but a
    sliver of elements (those next to a rounding tie, where the fp32 sum order decides)."""
    gen = torch.Generator().manual_seed(4)
    x = (torch.randn(4096, 128, generator=gen) * 3).bfloat16()
    w = (torch.rand(128, generator=gen) * 2 + 0.25).bfloat16()
    got = onorm.rms_norm_bf16(_torch_bits(x).reshape(4096, 128), _torch_bits(w), 1e-6)
    want = _torch_bits(_torch_rms_norm(x, w, 1e-6)).reshape(4096, 128)
    gv, wv = obf16.from_bits(got), obf16.from_bits(want)
    step = np.abs(wv) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(gv - wv) <= step)
    assert np.mean(got == want) > 0.995


def test_rms_norm_closed_forms():
    """A constant row normalises to sign * weight (up to eps); scaling the row by a power of
    two leaves the result unchanged; a zero row stays zero."""
    w = obf16.to_bits(np.linspace(0.5, 2.0, 128).astype(np.float32))
    row = obf16.to_bits(np.full((1, 128), -3.0, dtype=np.float32))
    out = obf16.from_bits(onorm.rms_norm_bf16(row, w, 0.0))
    assert np.array_equal(out, -obf16.from_bits(w)[None])
    rng = np.random.default_rng(5)
    x = obf16.to_bits(rng.standard_normal((64, 128)).astype(np.float32))
    x4 = obf16.to_bits(obf16.from_bits(x) * 4.0)
    assert np.array_equal(onorm.rms_norm_bf16(x, w, 0.0), onorm.rms_norm_bf16(x4, w, 0.0))
    zero = np.zeros((1, 128), dtype=np.uint16)
    assert np.all(obf16.from_bits(onorm.rms_norm_bf16(zero, w, 1e-6)) == 0)


# ---- the torch CPU path (the timed baseline) against the numpy oracle --------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_torch_path_matches_numpy_oracle_on_config1(dtype):
    """oracle/torch_path.decode_layer (the reference's eager RoPE, scatter_ write and SDPA
    under the 0 / finfo.min mask, the CPU baseline's arithmetic) and the numpy restatement
    (rope + kv_write + decode_attention) agree on the 4-request inputs, contexts
    {37, 120, 5, 256}: the arena after the write bit for bit, the outputs to 1e-5 in fp32
    and to the bf16 attention bar in bf16."""
    from oracle import torch_path
    from tests.golden.make_golden import CONFIG1_CONTEXTS, config1_inputs
    cache_k, cache_v, q, k, v = (t.to(dtype) for t in config1_inputs())
    positions = torch.tensor(CONFIG1_CONTEXTS, dtype=torch.int64)
    inv = torch.from_numpy(orope.inv_freq(128))
    angle = positions[:, None].float() * inv[None, :]
    emb = torch.cat([angle, angle], dim=-1)
    cos, sin = emb.cos().to(dtype)[:, None], emb.sin().to(dtype)[:, None]      # (B, 1, D)

    arena_k, arena_v = cache_k.clone(), cache_v.clone()
    out = torch_path.decode_layer(q, k, v, cos, sin, arena_k, arena_v, positions)

    if dtype == torch.float32:
        qr = orope.rope_f32(q.numpy(), cos.numpy()[:, :, None], sin.numpy()[:, :, None])
        kr = orope.rope_f32(k.numpy(), cos.numpy()[:, :, None], sin.numpy()[:, :, None])
        ok_, ov_ = cache_k.numpy().copy(), cache_v.numpy().copy()
        okv.kv_write(ok_, ov_, kr.transpose(0, 2, 1, 3), v.numpy().transpose(0, 2, 1, 3), positions.numpy())
        assert np.array_equal(arena_k.numpy(), ok_) and np.array_equal(arena_v.numpy(), ov_)
        ref = oatt.decode_attention(qr, ok_, ov_, positions.numpy(), 128 ** -0.5)
        assert np.abs(out.double().numpy() - ref).max() <= 1e-5
    else:
        qr = orope.rope_bf16(_torch_bits(q), _torch_bits(cos)[:, :, None], _torch_bits(sin)[:, :, None])
        kr = orope.rope_bf16(_torch_bits(k), _torch_bits(cos)[:, :, None], _torch_bits(sin)[:, :, None])
        ok_, ov_ = _torch_bits(cache_k).copy(), _torch_bits(cache_v).copy()
        okv.kv_write(ok_, ov_, kr.transpose(0, 2, 1, 3), _torch_bits(v).transpose(0, 2, 1, 3), positions.numpy())
        assert np.array_equal(_torch_bits(arena_k), ok_) and np.array_equal(_torch_bits(arena_v), ov_)
        ref = oatt.decode_attention(obf16.from_bits(qr), obf16.from_bits(ok_), obf16.from_bits(ov_),
                                    positions.numpy(), 128 ** -0.5)
        err = np.abs(out.double().numpy() - ref)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3
