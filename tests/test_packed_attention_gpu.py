"""The drop-in PackedAttention on talker- and predictor-shaped modules.

The modules are stand-ins with the attribute surface PackedAttention reads from
Qwen3TTSTalkerAttention / Qwen3TTSAttention (qwen_tts is not installed): q/k/v/o
projections, q/k RMSNorm, head_dim, layer_idx, scaling, rope_scaling.  o_proj is the
identity, so a layer's output is its attention output.  The expected values come from the
oracle applied to the same projected rows: exact RoPE, the scatter write (bit-exact) and
float64 attention (tolerance max-abs 2e-2, mean-abs 2e-3)."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import kv as okv
from oracle import rope as orope
from tests._util import assert_attention_close, bits

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


class RMSNorm(torch.nn.Module):
    def __init__(self, width):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(width, dtype=torch.bfloat16) * 1.5)

    def forward(self, x):
        y = x.float()
        y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + 1e-6)
        return self.weight * y.to(x.dtype)


class Config:
    _attn_implementation = 'sdpa'


class _Attention(torch.nn.Module):
    def __init__(self, layer_idx, hidden, seed):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.head_dim, self.layer_idx, self.scaling = D, layer_idx, D ** -0.5
        self.sliding_window, self.attention_dropout, self.is_causal = None, 0.0, True
        self.config = Config()
        self.rope_scaling = {'mrope_section': [24, 20, 20], 'interleaved': False}
        self.q_proj = torch.nn.Linear(hidden, HQ * D, bias=False, dtype=torch.bfloat16)
        self.k_proj = torch.nn.Linear(hidden, HKV * D, bias=False, dtype=torch.bfloat16)
        self.v_proj = torch.nn.Linear(hidden, HKV * D, bias=False, dtype=torch.bfloat16)
        self.o_proj = torch.nn.Linear(HQ * D, HQ * D, bias=False, dtype=torch.bfloat16)
        with torch.no_grad():
            for p in (self.q_proj, self.k_proj, self.v_proj):
                p.weight.copy_((torch.randn(p.weight.shape, generator=gen) * hidden ** -0.5).bfloat16())
            self.o_proj.weight.copy_(torch.eye(HQ * D, dtype=torch.bfloat16))
        self.q_norm, self.k_norm = RMSNorm(D), RMSNorm(D)


class Qwen3TTSTalkerAttention(_Attention):
    pass


class Qwen3TTSAttention(_Attention):
    pass


class _Layer(torch.nn.Module):
    def __init__(self, attn):
        super().__init__()
        self.self_attn = attn


class _Model(torch.nn.Module):
    def __init__(self, cls, layers, hidden):
        super().__init__()
        self.layers = torch.nn.ModuleList(_Layer(cls(i, hidden, 100 + i)) for i in range(layers))
        self.config = type('C', (), {'num_key_value_heads': HKV, 'head_dim': D, 'num_hidden_layers': layers})()
        self.weight = torch.nn.Parameter(torch.zeros(1, dtype=torch.bfloat16))


def _projected(module, hidden):
    """Rows exactly as PackedAttention.forward computes them (same fused weight and ops)."""
    proj = torch.nn.functional.linear(hidden, module.weight, module.bias)
    q, k, v = proj.split(module.sizes, dim=-1)
    shape = (*hidden.shape[:-1], -1, D)
    return module.reference.q_norm(q.reshape(shape)), module.reference.k_norm(k.reshape(shape)), v.reshape(shape)


def test_install_and_restore(pkg, device):
    model = _Model(Qwen3TTSTalkerAttention, 3, 256).to(device)
    originals = [layer.self_attn for layer in model.layers]
    replaced = pkg.install_packed_attention(model, native_gqa=True, text_only_rope=True, triton_talker_rope=True)
    assert len(replaced) == 3 and all(isinstance(l.self_attn, pkg.PackedAttention) for l in model.layers)
    pkg.restore_modules(replaced)
    assert [layer.self_attn for layer in model.layers] == originals
    with pytest.raises(ValueError):
        pkg.PackedAttention(originals[0], native_rope=True)            # talker needs equal axes
    with pytest.raises(ValueError):
        pkg.PackedAttention(originals[0], native_rope_scope='both')


@pytest.mark.parametrize("fused_path", [True, False])
def test_talker_decode_layer_through_slot_cache(pkg, device, fused_path):
    """One decode token per request over a SlotCache: bf16 takes the fused single launch;
    fp32 takes RoPE + cache update + the attention drop-in."""
    dtype = torch.bfloat16 if fused_path else torch.float32
    batch, hidden_size, capacity = 24, 256, 320
    model = _Model(Qwen3TTSTalkerAttention, 2, hidden_size).to(device).eval().to(dtype)
    pkg.install_packed_attention(model, native_gqa=True, text_only_rope=True, triton_talker_rope=True)
    module = model.layers[1].self_attn
    arena = pkg.SlotArena(model, 32, capacity, packed_kv=True)
    gen = torch.Generator().manual_seed(1)
    arena.packed.copy_(torch.randn(arena.packed.shape, generator=gen).to(dtype).to(device))
    contexts = torch.randint(0, capacity - 1, (batch,), generator=gen)
    positions = contexts.to(device)
    cache = pkg.SlotCache(arena, positions, capacity)
    hidden = torch.randn(batch, 1, hidden_size, generator=gen).to(dtype).to(device)
    cos, sin = pkg.rope_tables(positions[:, None], D, dtype=dtype)
    rope = (cos[None].expand(3, -1, -1, -1), sin[None].expand(3, -1, -1, -1))
    mask = torch.where(torch.arange(capacity, device=device)[None, :] <= positions[:, None], 0.0,
                       torch.finfo(dtype).min).to(dtype)[:, None, None, :]
    raw = (lambda t: bits(t)) if fused_path else (lambda t: t.detach().cpu().numpy())
    keys_before, values_before = raw(arena.keys[1]).copy(), raw(arena.values[1]).copy()
    q, k, v = _projected(module, hidden)
    out, _ = module(hidden, rope, mask, past_key_values=cache, cache_position=positions)
    torch.cuda.synchronize()

    if fused_path:
        cb, sb = bits(cos)[:, :, None, :], bits(sin)[:, :, None, :]
        q_rot = orope.rope_bf16(bits(q), cb, sb)
        k_rot = orope.rope_bf16(bits(k), cb, sb)
        to_f = obf16.from_bits
    else:
        cf, sf = cos.cpu().numpy()[:, :, None, :], sin.cpu().numpy()[:, :, None, :]
        q_rot = orope.rope_f32(q.detach().cpu().numpy(), cf, sf)
        k_rot = orope.rope_f32(k.detach().cpu().numpy(), cf, sf)
        to_f = np.asarray
    ek, ev = okv.kv_write(keys_before, values_before, k_rot.transpose(0, 2, 1, 3),
                          raw(v).transpose(0, 2, 1, 3), contexts.numpy())
    assert np.array_equal(raw(arena.keys[1]), ek) and np.array_equal(raw(arena.values[1]), ev)
    expected = oatt.decode_attention(to_f(q_rot), to_f(ek[:batch]), to_f(ev[:batch]), contexts.numpy(), D ** -0.5)
    got = out.detach().float().cpu().numpy().reshape(batch, 1, HQ, D)
    if fused_path:
        assert_attention_close(got, expected)
    else:
        assert_attention_close(got, expected, max_abs=1e-5, mean_abs=1e-6)


@pytest.mark.parametrize("width", [320, 200])
def test_slot_cache_step_honours_the_layer_mask(pkg, device, width):
    """The fused launch applies the mask the layer is given, as the reference's operator does
    (npu_attention.py:16-25): besides j <= pos[b], the mask here also hides every third key
    and the first key of odd requests, and with width 200 it covers a 200-key context view of
    the 320-row arena (SlotGraph's context_length, continuous.py:184-192).  The output must
    follow the oracle under that mask; without honouring it, it would not."""
    dtype = torch.bfloat16
    batch, hidden_size, capacity = 16, 256, 320
    model = _Model(Qwen3TTSTalkerAttention, 1, hidden_size).to(device).eval()
    pkg.install_packed_attention(model, native_gqa=True, text_only_rope=True, triton_talker_rope=True)
    module = model.layers[0].self_attn
    arena = pkg.SlotArena(model, batch, capacity, packed_kv=True)
    gen = torch.Generator().manual_seed(21)
    arena.packed.copy_(torch.randn(arena.packed.shape, generator=gen).to(dtype).to(device))
    contexts = torch.randint(2, width - 1, (batch,), generator=gen)
    positions = contexts.to(device)
    cache = pkg.SlotCache(arena, positions, width)
    hidden = torch.randn(batch, 1, hidden_size, generator=gen).to(dtype).to(device)
    cos, sin = pkg.rope_tables(positions[:, None], D, dtype=dtype)
    rope = (cos[None].expand(3, -1, -1, -1), sin[None].expand(3, -1, -1, -1))
    j = torch.arange(width)[None, :]
    allowed = (j <= contexts[:, None]) & ((j % 3 != 1) | (j == contexts[:, None]))
    allowed[1::2, 0] = False
    mask = torch.where(allowed, 0.0, torch.finfo(dtype).min).to(dtype)[:, None, None, :].to(device)
    keys_before, values_before = bits(arena.keys[0]).copy(), bits(arena.values[0]).copy()
    q, k, v = _projected(module, hidden)
    out, _ = module(hidden, rope, mask, past_key_values=cache, cache_position=positions)
    torch.cuda.synchronize()
    cb, sb = bits(cos)[:, :, None, :], bits(sin)[:, :, None, :]
    q_rot = orope.rope_bf16(bits(q), cb, sb)
    k_rot = orope.rope_bf16(bits(k), cb, sb)
    ek, ev = okv.kv_write(keys_before, values_before, k_rot.transpose(0, 2, 1, 3),
                          bits(v).transpose(0, 2, 1, 3), contexts.numpy())
    assert np.array_equal(bits(arena.keys[0]), ek) and np.array_equal(bits(arena.values[0]), ev)
    got = out.detach().float().cpu().numpy().reshape(batch, 1, HQ, D)
    expected = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(ek[:, :, :width]),
                                     obf16.from_bits(ev[:, :, :width]), contexts.numpy(), D ** -0.5,
                                     mask=allowed.numpy()[:, None, :])
    assert_attention_close(got, expected)
    unmasked = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(ek), obf16.from_bits(ev),
                                     contexts.numpy(), D ** -0.5)
    assert np.abs(got - unmasked).max() > 0.1  # the extra masked keys changed the result


@pytest.mark.parametrize("kind", ["causal", "none", "full"])
def test_predictor_first_step_two_queries_with_mask(pkg, device, monkeypatch, kind):
    """Code predictor step 0: two tokens, a PredictorCache writing positions [0, 2).  The 2x2
    causal 0/finfo.min mask (continuous.py:39-40) and no mask (two queries attend causally,
    npu_attention.py:17-18) take the fused two-token launch; any other mask (here all zeros:
    both queries see both keys) takes the unfused path with the mask applied as given."""
    import qwen3_tts_engine_amd.packed_attention as packed
    fused_calls = []
    original = packed.decode_step
    monkeypatch.setattr(packed, "decode_step", lambda *a, **k: fused_calls.append(1) or original(*a, **k))
    batch, hidden_size = 12, 256
    model = _Model(Qwen3TTSAttention, 1, hidden_size).to(device).eval()
    pkg.install_packed_attention(model, native_gqa=True)
    module = model.layers[0].self_attn
    gen = torch.Generator().manual_seed(2)
    hidden = torch.randn(batch, 2, hidden_size, generator=gen).bfloat16().to(device)
    cache = pkg.PredictorCache(model, hidden)
    pos = torch.arange(2, device=device)
    cos, sin = pkg.rope_tables(pos[None].expand(batch, 2).contiguous(), D)
    mask = torch.zeros(1, 1, 2, 2, device=device, dtype=torch.bfloat16)
    if kind == "causal":
        mask[..., 0, 1] = torch.finfo(torch.bfloat16).min
    q, k, v = _projected(module, hidden)
    out, _ = module(hidden, (cos, sin), None if kind == "none" else mask, past_key_values=cache,
                    cache_position=pos)
    torch.cuda.synchronize()
    assert len(fused_calls) == (0 if kind == "full" else 1)
    cb, sb = bits(cos)[:, :, None, :], bits(sin)[:, :, None, :]
    q_rot = obf16.from_bits(orope.rope_bf16(bits(q), cb, sb))
    k_rot = orope.rope_bf16(bits(k), cb, sb).transpose(0, 2, 1, 3)
    assert np.array_equal(bits(cache.keys[0][:, :, :2]), k_rot)
    assert np.array_equal(bits(cache.values[0][:, :, :2]), bits(v).transpose(0, 2, 1, 3))
    m = None if kind == "none" else np.broadcast_to(mask.float().cpu().numpy()[:, 0], (batch, 2, 2))
    expected = oatt.decode_attention(q_rot, obf16.from_bits(k_rot), f64v(v), [1] * batch, D ** -0.5, mask=m)
    assert_attention_close(out.detach().float().cpu().numpy().reshape(batch, 2, HQ, D), expected)


@pytest.mark.parametrize("step", [1, 7, 14])
def test_predictor_later_step_is_one_fused_launch(pkg, device, step):
    """Code predictor step s >= 1 (no mask): the new token is written at s + 1 and attends
    positions 0 ... s + 1 (predictor.py:19-24), taken by the fused launch with every
    position at s + 1.  Earlier positions hold random rotated keys from previous steps."""
    batch, hidden_size = 10, 256
    model = _Model(Qwen3TTSAttention, 2, hidden_size).to(device).eval()
    pkg.install_packed_attention(model, native_gqa=True)
    module = model.layers[1].self_attn
    gen = torch.Generator().manual_seed(20 + step)
    hidden = torch.randn(batch, 1, hidden_size, generator=gen).bfloat16().to(device)
    cache = pkg.PredictorCache(model, hidden)
    for plane in cache.keys + cache.values:
        plane.copy_(torch.randn(plane.shape, generator=gen).bfloat16().to(device))
    cache.step = step
    keys_before, values_before = bits(cache.keys[1]).copy(), bits(cache.values[1]).copy()
    pos = torch.full((batch, 1), step + 1, device=device, dtype=torch.int64)
    cos, sin = pkg.rope_tables(pos, D)
    q, k, v = _projected(module, hidden)
    out, _ = module(hidden, (cos, sin), None, past_key_values=cache, cache_position=pos[0])
    torch.cuda.synchronize()
    cb, sb = bits(cos)[:, :, None, :], bits(sin)[:, :, None, :]
    q_rot = obf16.from_bits(orope.rope_bf16(bits(q), cb, sb))
    k_rot = orope.rope_bf16(bits(k), cb, sb).transpose(0, 2, 1, 3)
    ek, ev = okv.kv_write(keys_before, values_before, k_rot, bits(v).transpose(0, 2, 1, 3),
                          np.full(batch, step + 1))
    assert np.array_equal(bits(cache.keys[1]), ek) and np.array_equal(bits(cache.values[1]), ev)
    expected = oatt.decode_attention(q_rot, obf16.from_bits(ek), obf16.from_bits(ev), [step + 1] * batch, D ** -0.5)
    assert_attention_close(out.detach().float().cpu().numpy().reshape(batch, 1, HQ, D), expected)


def f64v(v):
    return v.detach().float().cpu().numpy().transpose(0, 2, 1, 3).astype(np.float64)
