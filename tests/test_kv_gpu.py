"""KV arena writes and copies on the GPU: bit-exact against the oracle and the reference's
own fixtures (tests/test_packed_kv.py, tests/test_slot_context.py, tools/probe_paired_kv.py)."""
import numpy as np
import pytest
import torch

from oracle import kv as okv
from tests._util import bits

pytestmark = pytest.mark.gpu


def _qkv_views(batch, device, dtype=torch.bfloat16, seed=0, q_heads=16, kv_heads=8, width=128):
    """K/V as strided views of a fused QKV row, the layout the talker hands to the cache
    (row stride (Hq + 2*Hkv) * D, tools/probe_paired_kv.py:27-29)."""
    gen = torch.Generator().manual_seed(seed)
    packed = torch.randn(batch, 1, (q_heads + 2 * kv_heads) * width, generator=gen).to(dtype).to(device)
    k = packed[..., q_heads * width:(q_heads + kv_heads) * width].view(batch, 1, kv_heads, width).transpose(1, 2)
    v = packed[..., (q_heads + kv_heads) * width:].view(batch, 1, kv_heads, width).transpose(1, 2)
    return packed, k, v


@pytest.mark.parametrize("batch", [1, 8, 32, 64])
@pytest.mark.parametrize("capacity", [64, 512])
def test_paired_write_matches_scatter_on_strided_views(pkg, device, batch, capacity):
    _, k, v = _qkv_views(batch, device, seed=batch + capacity)
    gen = torch.Generator().manual_seed(1)
    tk = torch.randn(batch, 8, capacity, 128, generator=gen).bfloat16().to(device)
    tv = torch.randn(batch, 8, capacity, 128, generator=gen).bfloat16().to(device)
    positions = (torch.arange(batch) * 7 + capacity - 1) % capacity
    ek, ev = okv.kv_write(bits(tk).copy(), bits(tv).copy(), bits(k), bits(v), positions.numpy())
    pkg.write(k, v, tk, tv, positions.to(device), row_tiled=True)
    assert np.array_equal(bits(tk), ek) and np.array_equal(bits(tv), ev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_write_other_dtypes(pkg, device, dtype):
    _, k, v = _qkv_views(16, device, dtype=dtype, seed=3)
    tk = torch.zeros(16, 8, 100, 128, dtype=dtype, device=device)
    tv = torch.zeros_like(tk)
    positions = torch.arange(16) * 6
    ek, ev = okv.kv_write(tk.cpu().numpy().copy(), tv.cpu().numpy().copy(), k.cpu().numpy(),
                          v.cpu().numpy(), positions.numpy())
    pkg.write(k, v, tk, tv, positions.to(device))
    assert np.array_equal(tk.cpu().numpy(), ek) and np.array_equal(tv.cpu().numpy(), ev)


def test_out_of_arena_positions_are_skipped(pkg, device):
    _, k, v = _qkv_views(4, device, seed=4)
    tk = torch.zeros(4, 8, 32, 128, dtype=torch.bfloat16, device=device)
    tv = torch.zeros_like(tk)
    positions = torch.tensor([0, 31, 32, -1])
    ek, ev = okv.kv_write(bits(tk).copy(), bits(tv).copy(), bits(k), bits(v), positions.numpy())
    pkg.write(k, v, tk, tv, positions.to(device))
    assert np.array_equal(bits(tk), ek) and np.array_equal(bits(tv), ev)
    assert not bits(tk)[2:].any()


def test_multi_token_write_predictor_windows(pkg, device):
    """PredictorCache: step 0 writes [0, 2), step s writes s + 1 (predictor.py:19-24)."""
    gen = torch.Generator().manual_seed(5)
    tk = torch.zeros(64, 8, 16, 128, dtype=torch.bfloat16, device=device)
    tv = torch.zeros_like(tk)
    ek, ev = bits(tk).copy(), bits(tv).copy()
    for step in range(15):
        start = 0 if step == 0 else step + 1
        n = 2 if step == 0 else 1
        k = torch.randn(64, 8, n, 128, generator=gen).bfloat16().to(device)
        v = torch.randn(64, 8, n, 128, generator=gen).bfloat16().to(device)
        positions = torch.full((64,), start, dtype=torch.int64)
        okv.kv_write(ek, ev, bits(k), bits(v), positions.numpy())
        pkg.write_tokens(k, v, tk, tv, positions.to(device))
    assert np.array_equal(bits(tk), ek) and np.array_equal(bits(tv), ev)


def test_write_replays_in_a_graph_with_changed_inputs(pkg, device):
    """Frozen-argument check of tools/probe_paired_kv.py:52-57: change the inputs in place
    between replays of a captured write."""
    batch, capacity = 64, 512
    packed, k, v = _qkv_views(batch, device, seed=6)
    tk = torch.zeros(batch, 8, capacity, 128, dtype=torch.bfloat16, device=device)
    tv = torch.zeros_like(tk)
    positions = torch.zeros(batch, dtype=torch.int64, device=device)
    pkg.write(k, v, tk, tv, positions)  # eager warm-up
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pkg.write(k, v, tk, tv, positions)
    ek, ev = bits(tk).copy(), bits(tv).copy()
    gen = torch.Generator().manual_seed(7)
    for step in range(4):
        packed.copy_(torch.randn(packed.shape, generator=gen).bfloat16().to(device))
        new_pos = (torch.arange(batch) + capacity - 1 + step) % capacity
        positions.copy_(new_pos.to(device))
        graph.replay()
        torch.cuda.synchronize()
        okv.kv_write(ek, ev, bits(k), bits(v), new_pos.numpy())
        assert np.array_equal(bits(tk), ek) and np.array_equal(bits(tv), ev)


# --- copy_packed_prefix: the reference's own fixtures (tests/test_packed_kv.py) ---------

def _prefix_tensors(dtype, device):
    target = torch.full((4, 5, 2, 7, 3), -7, dtype=dtype)
    source = torch.arange(4 * 3 * 2 * 5 * 6).view(4, 3, 2, 5, 6).to(dtype)[..., ::2]
    return target.to(device), source.to(device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.int64])
def test_changed_strided_prefix_matches_closed_form(pkg, device, dtype):
    target, source = _prefix_tensors(dtype, device)
    for row, slot, length in ((2, 3, 1), (0, 1, 5), (1, 4, 3)):
        original = source.clone()
        expected = target.clone()
        for layer in range(target.shape[0]):
            expected[layer, slot, :, :length].copy_(source[layer, row, :, :length])
        pkg.copy_packed_prefix(target, source, slot, row=row, length=length)
        assert torch.equal(target, expected)
        assert torch.equal(source, original)
        source.add_(1)


def test_default_length_preserves_padded_tail(pkg, device):
    target, source = _prefix_tensors(torch.float32, device)
    expected = target.clone()
    expected[:, 0, :, :5].copy_(source[:, 0])
    pkg.copy_packed_prefix(target, source, 0)
    assert torch.equal(target, expected)


def test_strided_target_preserves_interleaved_storage(pkg, device):
    base = torch.full((4, 5, 2, 7, 6), -9.0, device=device)
    target = base[..., ::2]
    _, source = _prefix_tensors(torch.float32, device)
    expected = base.clone()
    expected[..., ::2][:, 2, :, :4].copy_(source[:, 1, :, :4])
    pkg.copy_packed_prefix(target, source, 2, row=1, length=4)
    assert torch.equal(base, expected)


def test_invalid_prefix_bounds_never_write(pkg, device):
    target, source = _prefix_tensors(torch.float32, device)
    saved = target.clone()
    for slot, row, length in ((-1, 0, 1), (5, 0, 1), (0, 3, 1), (0, -1, 1), (0, 0, 0), (0, 0, 6),
                              (True, 0, 1), (0, True, 1), (0, 0, True)):
        with pytest.raises(ValueError):
            pkg.copy_packed_prefix(target, source, slot, row=row, length=length)
    torch.cuda.synchronize()
    assert torch.equal(target, saved)


def test_packed_prefix_at_talker_shape(pkg, device):
    """A 16-row prefill cache (56, 16, 8, 512, 128) into a 64-slot arena, bit-exact."""
    gen = torch.Generator(device=device).manual_seed(8)
    source = torch.randn(56, 16, 8, 512, 128, generator=gen, device=device, dtype=torch.bfloat16)
    target = torch.randn(56, 64, 8, 1024, 128, generator=gen, device=device, dtype=torch.bfloat16)
    expected = target.clone()
    for slot, row, length in ((0, 3, 386), (63, 15, 84), (17, 0, 512)):
        expected[:, slot, :, :length] = source[:, row, :, :length]
        pkg.copy_packed_prefix(target, source, slot, row=row, length=length)
    assert torch.equal(target, expected)


# --- SlotArena: move / grow / load (continuous.py:97-132, 353-363) ---------------------

class _Config:
    num_key_value_heads = 8
    head_dim = 128
    num_hidden_layers = 3


class _Talker(torch.nn.Module):
    def __init__(self, layers=3):
        super().__init__()
        self.config = _Config()
        self.layers = torch.nn.ModuleList(torch.nn.Identity() for _ in range(layers))
        self.weight = torch.nn.Parameter(torch.zeros(1, dtype=torch.bfloat16))


@pytest.mark.parametrize("packed", [False, True])
def test_arena_move_and_grow(pkg, device, packed):
    from qwen3_tts_engine_amd.slots import SlotArena, grow_arena
    talker = _Talker().to(device)
    arena = SlotArena(talker, 8, 64, packed_kv=packed)
    gen = torch.Generator().manual_seed(9)
    for plane in arena.planes():
        plane.copy_(torch.randn(plane.shape, generator=gen).bfloat16().to(device))
    planes = [bits(p).copy() for p in arena.planes()]
    arena.move(7, 2)
    arena.move(3, 3)
    okv.move(planes, 7, 2)
    assert all(np.array_equal(bits(p), e) for p, e in zip(arena.planes(), planes))
    grown = grow_arena(arena, 64)
    assert grown.capacity == okv.grown_capacity(64, 64) == 128
    expected = okv.grow(planes, 128)
    assert all(np.array_equal(bits(p), e) for p, e in zip(grown.planes(), expected))
    assert grow_arena(grown, 100) is grown


def test_slot_cache_update_preserves_history(pkg, device):
    """tests/test_slot_context.py:11-31: exact scatter at positions and the returned views."""
    from qwen3_tts_engine_amd.slots import SlotCache

    class Arena:
        pass

    for valid_length in (False, True):
        for context, positions in ((64, [63, 17]), (128, [64, 127])):
            torch.manual_seed(42)
            keys, values = torch.randn(2, 2, 256, 8), torch.randn(2, 2, 256, 8)
            arena = Arena()
            arena.capacity = 256
            arena.keys, arena.values = [keys.clone().to(device)], [values.clone().to(device)]
            position = torch.tensor(positions)
            cache = SlotCache(arena, position.to(device), context, valid_length)
            new_keys, new_values = torch.randn(2, 2, 1, 8), torch.randn(2, 2, 1, 8)
            actual_k, actual_v = cache.update(new_keys.to(device), new_values.to(device), 0, {})
            for row, offset in enumerate(positions):
                keys[row, :, offset] = new_keys[row, :, 0]
                values[row, :, offset] = new_values[row, :, 0]
            assert torch.equal(arena.keys[0].cpu(), keys) and torch.equal(arena.values[0].cpu(), values)
            returned = 256 if valid_length else context
            assert actual_k.shape == (2, 2, returned, 8)
            if valid_length:
                assert actual_k.data_ptr() == arena.keys[0].data_ptr()
                assert cache.actual_seq_lengths_kv == [context, context]
