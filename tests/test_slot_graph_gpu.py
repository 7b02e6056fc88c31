"""SlotGraph: the talker decode step captured in one HIP graph through PackedAttention.

The graph (continuous.py:170-229 restated on HIP graphs) is checked against the same
``compute`` run eagerly on a twin arena: every replay's output and the whole arena after it
must be bit-identical, over several steps with padded rows (positions 0 past the active
count), with eager work on the stream between replays.  Capture must leave the arena rows at
position 0 of slots ``[:batch]`` as they were (the reference saves and restores them).  The
attention numerics themselves are pinned against the oracle in test_packed_attention_gpu.py
and test_decode_gpu.py.
"""
import numpy as np
import pytest
import torch

from tests._talker import Talker
from tests._util import bits

pytestmark = pytest.mark.gpu


def _model(pkg, device, layers=3, hidden=256):
    model = Talker(layers=layers, hidden=hidden, seed=3).to(device).eval()
    pkg.install_packed_attention(model, native_gqa=True, text_only_rope=True, triton_talker_rope=True)
    return model


def _arena(pkg, model, slots, capacity, seed):
    arena = pkg.SlotArena(model, slots, capacity, packed_kv=True)
    gen = torch.Generator().manual_seed(seed)
    arena.packed.copy_(torch.randn(arena.packed.shape, generator=gen).bfloat16().to(arena.packed.device))
    return arena


def test_replays_match_eager_compute_and_capture_restores_position_zero(pkg, device):
    slots, capacity, batch = 16, 192, 8
    model = _model(pkg, device)
    arena = _arena(pkg, model, slots, capacity, 4)
    twin_arena = pkg.SlotArena(model, slots, capacity, packed_kv=True)
    twin_arena.packed.copy_(arena.packed)
    row0 = bits(arena.packed[:, :batch, :, 0]).copy()

    graph = pkg.SlotGraph(arena, batch)
    graph.capture()
    torch.cuda.synchronize()
    assert np.array_equal(bits(arena.packed[:, :batch, :, 0]), row0)
    assert np.array_equal(bits(arena.packed), bits(twin_arena.packed))

    twin = pkg.SlotGraph(twin_arena, batch)
    gen = torch.Generator().manual_seed(5)
    for step, count in enumerate([8, 6, 8, 3, 8]):
        positions = torch.zeros(batch, dtype=torch.long)
        positions[:count] = torch.randint(0, capacity, (count,), generator=gen)
        inputs = torch.randn(batch, 1, model.config.hidden_size, generator=gen).bfloat16().to(device)
        rotary = positions.view(1, batch, 1).expand(3, batch, 1).to(device)
        positions = positions.to(device)
        out = graph.run(inputs, positions, rotary)
        scratch = torch.randn(4096, device=device).sum()  # unrelated eager work between replays
        with torch.inference_mode():
            twin.inputs.copy_(inputs)
            twin.positions.copy_(positions)
            twin.rotary.copy_(rotary)
            expected = twin.compute()
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
        assert np.array_equal(bits(out), bits(expected)), f"step {step}"
        assert np.array_equal(bits(arena.packed), bits(twin_arena.packed)), f"step {step}"
    graph.close()


def test_slot_graph_context_must_fit_the_arena(pkg, device):
    model = _model(pkg, device, layers=1)
    arena = pkg.SlotArena(model, 4, 64, packed_kv=True)
    with pytest.raises(ValueError):
        pkg.SlotGraph(arena, 4, context_length=65)
    with pytest.raises(ValueError):
        pkg.SlotGraph(arena, 4, context_length=0)
