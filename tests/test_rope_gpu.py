"""RoPE on the GPU: bit-exact against the oracle (which is pinned to torch eager), over the
shapes of tools/probe_rotary_exact.py, and the cos/sin tables of the talker."""
import numpy as np
import pytest
import torch

from oracle import bf16 as obf16
from oracle import rope as orope
from tests._util import bits, from_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch", [1, 17, 64])
@pytest.mark.parametrize("length", [1, 2, 16, 64])
@pytest.mark.parametrize("heads,width", [(16, 128), (8, 128), (8, 64)])
def test_rotary_bf16_bit_exact(pkg, device, batch, length, heads, width):
    gen = torch.Generator().manual_seed(42)
    x = torch.randn(batch, length, heads, width, generator=gen).bfloat16()
    phase = torch.randn(batch, length, width // 2, generator=gen).repeat(1, 1, 2)
    cos, sin = phase.cos().bfloat16(), phase.sin().bfloat16()
    y = pkg.rotary(x.to(device), cos.to(device), sin.to(device))
    expected = orope.rope_bf16(bits(x), bits(cos)[:, :, None, :], bits(sin)[:, :, None, :])
    assert np.array_equal(bits(y), expected)


def test_rotary_bf16_special_values(pkg, device):
    """Ties, signed zeros, infinities and NaN go through the same per-op rounding."""
    vals = np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 3.0e38, -3.0e38, np.inf, -np.inf,
                     1e-40, 65504.0, 0.333984375], dtype=np.float32)
    gen = np.random.default_rng(0)
    x = obf16.to_bits(gen.choice(vals, size=(4, 3, 8, 128)).astype(np.float32))
    cos = obf16.to_bits(gen.choice(vals, size=(4, 3, 128)).astype(np.float32))
    sin = obf16.to_bits(gen.choice(vals, size=(4, 3, 128)).astype(np.float32))
    y = pkg.rotary(from_bits(x, device), from_bits(cos, device), from_bits(sin, device))
    expected = orope.rope_bf16(x, cos[:, :, None, :], sin[:, :, None, :])
    assert np.array_equal(bits(y), expected)


@pytest.mark.parametrize("width", [64, 128])
def test_rotary_fp32_exact(pkg, device, width):
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(5, 7, 16, width, generator=gen)
    phase = torch.randn(5, 7, width // 2, generator=gen).repeat(1, 1, 2)
    cos, sin = phase.cos(), phase.sin()
    y = pkg.rotary(x.to(device), cos.to(device), sin.to(device)).cpu().numpy()
    expected = orope.rope_f32(x.numpy(), cos.numpy()[:, :, None, :], sin.numpy()[:, :, None, :])
    assert np.array_equal(y.view(np.uint32), expected.view(np.uint32))


def test_rope_tables_talker_positions(pkg, device):
    """cos/sin rows for positions up to 4096 with theta 1e6: within one bf16 ulp of the
    float64-evaluated table (the device cosf/sinf differ from any CPU libm by <= 1 fp32 ulp)."""
    positions = torch.arange(0, 4097, dtype=torch.int64)
    inv = pkg.inverse_frequencies(128)
    cos, sin = pkg.rope_tables(positions.to(device), 128)
    ecos, esin = orope.tables(positions.numpy(), inv.numpy())
    for got, want in ((bits(cos), ecos), (bits(sin), esin)):
        diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
        # adjacent bf16 values differ by one in the bit pattern (same sign)
        assert diff.max() <= 1
        assert (diff == 0).mean() > 0.99
    assert np.array_equal(bits(cos)[:, :64], bits(cos)[:, 64:])
    f32cos, _ = pkg.rope_tables(positions.to(device), 128, dtype=torch.float32)
    ref32, _ = orope.tables(positions.numpy(), inv.numpy(), dtype="f32")
    assert np.abs(f32cos.cpu().numpy() - ref32).max() <= 2.5e-7


@pytest.mark.parametrize("length", [1, 64])
def test_rotary_graph_replays_track_inputs(pkg, device, length):
    """tools/probe_rotary_exact.py:41-61: q and k rotated by one captured graph; the inputs
    and the cos/sin rows are overwritten in place before each of three replays, and every
    replay must be bit-exact for the new inputs."""
    batch = 17
    gen = torch.Generator(device=device).manual_seed(43)
    q = torch.empty(batch, length, 16, 128, device=device, dtype=torch.bfloat16)
    k = torch.empty(batch, length, 8, 128, device=device, dtype=torch.bfloat16)
    cos = torch.empty(batch, length, 128, device=device, dtype=torch.bfloat16)
    sin = torch.empty_like(cos)

    def refill():
        for t in (q, k):
            t.copy_(torch.randn(t.shape, generator=gen, device=device))
        phase = torch.randn(batch, length, 64, generator=gen, device=device).repeat(1, 1, 2)
        cos.copy_(phase.cos())
        sin.copy_(phase.sin())

    refill()
    pkg.rotary(q, cos, sin), pkg.rotary(k, cos, sin)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outputs = (pkg.rotary(q, cos, sin), pkg.rotary(k, cos, sin))
    for _ in range(3):
        refill()
        graph.replay()
        torch.cuda.synchronize()
        c, s = bits(cos)[:, :, None, :], bits(sin)[:, :, None, :]
        for x, y in zip((q, k), outputs):
            assert np.array_equal(bits(y), orope.rope_bf16(bits(x), c, s))
