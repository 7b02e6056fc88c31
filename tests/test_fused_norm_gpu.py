"""q/k RMSNorm folded into the fused decode launch (decode_step with norm weights, and
PackedAttention(fused_qk_norm=True)).

The oracle chain is RMSNorm (oracle/norm.py, pinned against torch's module formula) ->
exact RoPE -> scatter write -> float64 attention.  A row's fp32 sum of squares depends on the
summation order, so a normalised element may land one bf16 step away from the oracle's next
to a rounding tie: arena keys are held to one step (relative 2^-7, then the RoPE of that
row) elementwise with at least 99% bit-equal, outputs to the attention bar.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import kv as okv
from oracle import norm as onorm
from oracle import rope as orope
from tests._talker import Talker
from tests._util import assert_attention_close, bits, f64

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


def _close_bf16(got_bits, want_bits, frac=0.99):
    g, w = obf16.from_bits(got_bits), obf16.from_bits(want_bits)
    scale = np.maximum(np.abs(w), np.abs(g)) * 2.0 ** -6 + 2.0 ** -20
    assert np.all(np.abs(g - w) <= scale), f"max diff {np.abs(g - w).max()}"
    assert np.mean(got_bits == want_bits) >= frac, f"bit-equal fraction {np.mean(got_bits == want_bits):.4f}"


@pytest.mark.parametrize("eps,grid", [(1e-6, None), (1e-2, None), (1e-6, "bundled"), (1e-2, "bundled")])
def test_decode_step_with_qk_norm_matches_oracle(pkg, device, eps, grid):
    gen = torch.Generator().manual_seed(7)
    batch, capacity = 48, 640
    contexts = torch.randint(0, capacity - 1, (batch,), generator=gen)
    k = torch.randn(batch, HKV, capacity, D, generator=gen).bfloat16().to(device)
    v = torch.randn(batch, HKV, capacity, D, generator=gen).bfloat16().to(device)
    qkv = (torch.randn(batch, 1, (HQ + 2 * HKV) * D, generator=gen) * 2).bfloat16().to(device)
    q = qkv[..., :HQ * D].view(batch, 1, HQ, D)
    kn = qkv[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D)
    vn = qkv[..., (HQ + HKV) * D:].view(batch, 1, HKV, D)
    qw = (torch.rand(D, generator=gen) + 0.5).bfloat16().to(device)
    kw = (torch.rand(D, generator=gen) + 0.5).bfloat16().to(device)
    positions = contexts.to(device)
    cos, sin = pkg.rope_tables(positions, D)
    k_before, v_before = bits(k).copy(), bits(v).copy()
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin, q_norm_weight=qw, k_norm_weight=kw,
                          norm_eps=eps, grid=grid)
    torch.cuda.synchronize()

    cb, sb = bits(cos)[:, None, None, :], bits(sin)[:, None, None, :]
    q_n = onorm.rms_norm_bf16(bits(q), bits(qw), eps)
    k_n = onorm.rms_norm_bf16(bits(kn), bits(kw), eps)
    q_rot = orope.rope_bf16(q_n, cb, sb)
    k_rot = orope.rope_bf16(k_n, cb, sb)
    ek, ev = okv.kv_write(k_before.copy(), v_before.copy(), k_rot.transpose(0, 2, 1, 3),
                          bits(vn).transpose(0, 2, 1, 3), contexts.numpy())
    got_k = bits(k)
    rows = np.arange(batch)
    # the written rows: within one bf16 step of the oracle; everything else untouched
    _close_bf16(got_k[rows, :, contexts.numpy()], ek[rows, :, contexts.numpy()])
    untouched = np.ones(got_k.shape, dtype=bool)
    untouched[rows, :, contexts.numpy()] = False
    assert np.array_equal(got_k[untouched], k_before[untouched])
    assert np.array_equal(bits(v), ev)
    expected = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(ek), obf16.from_bits(ev),
                                     contexts.numpy(), D ** -0.5)
    assert_attention_close(f64(out)[:, 0], expected[:, 0])


def test_packed_attention_fused_norm_matches_module_norms(pkg, device):
    """The same talker layer with the module's norms and with the norms fused: arena keys
    within one bf16 step (most bit-equal), outputs within the attention bar of each other."""
    batch, capacity = 32, 384
    gen = torch.Generator().manual_seed(8)
    contexts = torch.randint(0, capacity - 1, (batch,), generator=gen)
    hidden = torch.randn(batch, 1, 256, generator=gen).bfloat16().to(device)
    positions = contexts.to(device)
    cos, sin = pkg.rope_tables(positions[:, None], D)
    rope = (cos[None].expand(3, -1, -1, -1), sin[None].expand(3, -1, -1, -1))
    results = []
    for fused in (False, True):
        model = Talker(layers=1, hidden=256, seed=9).to(device).eval()
        with torch.no_grad():
            model.layers[0].self_attn.q_norm.weight.copy_(torch.linspace(0.5, 1.5, D).bfloat16())
            model.layers[0].self_attn.k_norm.weight.copy_(torch.linspace(1.5, 0.5, D).bfloat16())
        pkg.install_packed_attention(model, native_gqa=True, text_only_rope=True, triton_talker_rope=True,
                                     fused_qk_norm=fused)
        arena = pkg.SlotArena(model, batch, capacity, packed_kv=True)
        arena.packed.copy_(torch.randn(arena.packed.shape, generator=torch.Generator().manual_seed(10))
                           .bfloat16().to(device))
        cache = pkg.SlotCache(arena, positions, capacity)
        out, _ = model.layers[0].self_attn(hidden, rope, None, past_key_values=cache, cache_position=positions)
        torch.cuda.synchronize()
        results.append((bits(arena.keys[0]).copy(), out.detach().float().cpu().numpy()))
    (k0, o0), (k1, o1) = results
    rows = np.arange(batch)
    _close_bf16(k1[rows, :, contexts.numpy()], k0[rows, :, contexts.numpy()])
    assert_attention_close(o1, o0.astype(np.float64))
