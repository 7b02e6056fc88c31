"""The automatic decode grid at the shapes around its thresholds (24 requests, 64 requests,
512, 1024 and 4096 rows; see q3t_decode_grid): the automatic launch is bit-identical to the
same launch on the grid decode_grid_for names, and, against the float64 oracle, within the bar
for bf16 I/O with fp32 accumulation (max-abs <= 2e-2, mean-abs <= 2e-3).  Fused steps
(RoPE of the query and the new key, the paired write, attention) with uniform contexts."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import rope as orope
from tests._util import assert_attention_close, bits

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128
NAMED = {"bundled": dict(grid="bundled"), "balanced": dict(grid="balanced"), "chunked": dict(grid="chunked")}


@pytest.mark.parametrize("batch,capacity,expected", [
    (23, 1024, "chunked"), (24, 512, "bundled"), (63, 512, "bundled"), (64, 512, "chunked"),
    (64, 1023, "chunked"), (64, 1024, "bundled"), (16, 2048, "balanced"), (47, 4096, "balanced"),
    (48, 4096, "bundled")])
def test_automatic_grid_matches_its_named_grid_and_the_oracle(pkg, device, batch, capacity, expected):
    assert pkg.decode_grid_for(batch, 1, HQ, HKV, D, capacity) == expected
    gen = torch.Generator().manual_seed(batch * 7 + capacity)
    positions = torch.randint(0, capacity, (batch,), generator=gen)
    dg = torch.Generator(device=device).manual_seed(batch + capacity)
    keys = torch.randn(batch, HKV, capacity, D, generator=dg, device=device, dtype=torch.bfloat16)
    values = torch.randn_like(keys)
    qkv = torch.randn(batch, 1, (HQ + 2 * HKV) * D, generator=dg, device=device, dtype=torch.bfloat16)
    q = qkv[..., :HQ * D].view(batch, 1, HQ, D)
    k = qkv[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D)
    v = qkv[..., (HQ + HKV) * D:].view(batch, 1, HKV, D)
    dpos = positions.to(device)
    cos, sin = pkg.rope_tables(dpos, D)
    k_auto, v_auto = keys.clone(), values.clone()
    auto = pkg.decode_step(q, k, v, k_auto, v_auto, dpos, cos, sin)
    named = pkg.decode_step(q, k, v, keys, values, dpos, cos, sin, **NAMED[expected])
    torch.cuda.synchronize()
    assert torch.equal(auto, named)
    assert torch.equal(k_auto, keys) and torch.equal(v_auto, values)

    # the oracle: rotated rows written at the positions, then attention over keys 0 ... p_b
    cb, sb = bits(cos)[:, None, None, :], bits(sin)[:, None, None, :]
    q_rot = orope.rope_bf16(bits(q), cb, sb)
    arena_k = bits(keys).copy()
    arena_v = bits(values).copy()
    np.testing.assert_array_equal(arena_k[np.arange(batch), :, positions.numpy()],
                                  orope.rope_bf16(bits(k), cb, sb)[:, 0])
    np.testing.assert_array_equal(arena_v[np.arange(batch), :, positions.numpy()], bits(v)[:, 0])
    expected_out = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(arena_k),
                                         obf16.from_bits(arena_v), positions.numpy(), D ** -0.5)
    assert_attention_close(auto.float().cpu().numpy().astype(np.float64), expected_out)
