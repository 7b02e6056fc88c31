"""The allocation-free decode entry point (q3t_decode_attention_static) against the
workspace entry point (q3t_decode_attention), both through the C ABI: two calls in a row, the
second with a smaller input, each split over several workgroups so that the library's own
device array carries the partial states and counters.  Same kernels and the same grid, so
outputs and arena writes must be bit-identical."""
import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


def _inputs(batch, capacity, seed, device):
    gen = torch.Generator(device=device).manual_seed(seed)
    keys = torch.randn(batch, HKV, capacity, D, generator=gen, device=device, dtype=torch.bfloat16)
    values = torch.randn_like(keys)
    qkv = torch.randn(batch, 1, (HQ + 2 * HKV) * D, generator=gen, device=device, dtype=torch.bfloat16)
    positions = torch.randint(0, capacity, (batch,), generator=gen, device=device)
    return keys, values, qkv, positions


def _split(qkv, batch):
    q = qkv[..., :HQ * D].view(batch, 1, HQ, D)
    k = qkv[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D)
    v = qkv[..., (HQ + HKV) * D:].view(batch, 1, HKV, D)
    return q, k, v


@pytest.mark.parametrize("grid", [(-1, 4), (24, 0)])
def test_no_alloc_entry_point_matches_the_workspace_entry_point(pkg, device, grid):
    splits, max_chunks = grid
    # first call: the talker step shape (64 requests, 1024-row arena), fused RoPE + write
    keys, values, qkv, positions = _inputs(64, 1024, 90, device)
    q, k, v = _split(qkv, 64)
    cos, sin = pkg.rope_tables(positions, D)
    k2, v2 = keys.clone(), values.clone()
    expected = pkg.decode_step(q, k, v, keys, values, positions, cos, sin, splits=splits, max_chunks=max_chunks)
    got = pkg.decode_step(q, k, v, k2, v2, positions, cos, sin, splits=splits, max_chunks=max_chunks,
                          no_alloc=True)
    torch.cuda.synchronize()
    assert torch.equal(got, expected)
    assert torch.equal(k2, keys) and torch.equal(v2, values)
    # second call, smaller: 8 requests over a 300-row arena, attention only
    keys, values, qkv, positions = _inputs(8, 300, 91, device)
    q = qkv[..., :HQ * D].view(8, 1, HQ, D)
    expected = pkg.decode_attention(q, keys, values, positions, splits=splits, max_chunks=max_chunks)
    got = pkg.decode_attention(q, keys, values, positions, splits=splits, max_chunks=max_chunks, no_alloc=True)
    torch.cuda.synchronize()
    assert torch.equal(got, expected)


def test_no_alloc_rejects_calls_beyond_its_array(pkg, device):
    """1024 requests split in 16 chunks each need 68 MB of partial states: refused before
    any launch (the caller's output keeps its contents)."""
    batch, capacity = 1024, 1024
    keys = torch.zeros(batch, HKV, capacity, D, device=device, dtype=torch.bfloat16)
    q = torch.zeros(batch, 1, HQ, D, device=device, dtype=torch.bfloat16)
    positions = torch.full((batch,), capacity - 1, device=device, dtype=torch.int64)
    out = torch.full((batch, 1, HQ, D), 7.0, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.decode_attention(q, keys, keys, positions, splits=-1, max_chunks=16, out=out, no_alloc=True)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


@pytest.mark.parametrize("grid", [(-1, 4), (24, 0)])
def test_no_alloc_entry_point_under_graph_capture(pkg, device, grid):
    """Recorded in a graph (the callers the entry point is for) and replayed with the
    positions, the step's rows and the arena rewritten in place: every replay matches the
    workspace entry point run eagerly on the same inputs, bit for bit."""
    splits, max_chunks = grid
    keys, values, qkv, positions = _inputs(64, 1024, 92, device)
    q, k, v = _split(qkv, 64)
    cos, sin = pkg.rope_tables(positions, D)
    out = torch.empty(64, 1, HQ, D, device=device, dtype=torch.bfloat16)
    pkg.decode_step(q, k, v, keys, values, positions, cos, sin, splits=splits, max_chunks=max_chunks,
                    no_alloc=True, out=out)  # eager first call: the array's set-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph):  # as the package's graphs are captured
        pkg.decode_step(q, k, v, keys, values, positions, cos, sin, splits=splits, max_chunks=max_chunks,
                        no_alloc=True, out=out)
    gen = torch.Generator(device=device).manual_seed(93)
    for _ in range(3):
        positions.copy_(torch.randint(0, 1024, (64,), generator=gen, device=device))
        qkv.copy_(torch.randn(qkv.shape, generator=gen, device=device, dtype=torch.bfloat16))
        keys.copy_(torch.randn(keys.shape, generator=gen, device=device, dtype=torch.bfloat16))
        c, s = pkg.rope_tables(positions, D)
        cos.copy_(c)
        sin.copy_(s)
        k2, v2 = keys.clone(), values.clone()
        expected = pkg.decode_step(q, k, v, k2, v2, positions, cos, sin, splits=splits, max_chunks=max_chunks)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, expected)
        assert torch.equal(keys, k2) and torch.equal(values, v2)
