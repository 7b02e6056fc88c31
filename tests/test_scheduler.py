"""The package's slot scheduler against the oracle's restatement of ContinuousModel's integer
state (continuous.py:353-363, 425-473, 541-657).

CPU: the mixed-traffic trace (128 slots, 200 iterations, Poisson arrivals with mean 2 per
iteration, prompts U{32..512}, retirement after U{200..2000} frames, capacity 512 growing
to 4096) must give bit-identical decode records, retirements and arena operations.
GPU: a small packed arena driven through a trace with prefix loads, decode writes at the
scheduled positions (padded rows included), compaction moves and regrowth stays
bit-identical to the same operations applied to numpy arrays."""
import numpy as np
import pytest
import torch

from oracle import kv as okv
from oracle import scheduler as osched
from tests._util import bits


class _Adapter:
    """Presents the package scheduler with the oracle's tick contract."""

    def __init__(self, scheduler):
        self.scheduler = scheduler

    @property
    def ops(self):
        return self.scheduler.ops

    def tick(self, submissions=(), cancelled=()):
        batch, done = self.scheduler.tick(submissions, cancelled)
        if batch is None:
            return None, done
        return {'batch': batch.batch, 'context': batch.context, 'positions': batch.positions,
                'slots': batch.identifiers, 'capacity': batch.capacity}, done


@pytest.mark.parametrize("step,bucket_kv,cancel_rate,lengths", [
    (0, False, 0.0, (200, 2000)), (8, True, 0.05, (200, 2000)), (16, True, 0.2, (200, 2000)),
    (0, True, 0.05, (2, 40)), (4, False, 0.0, (2, 40))])
def test_mixed_trace_integer_parity(pkg, step, bucket_kv, cancel_rate, lengths):
    """The long-limit traces reach a full arena and regrowth; the short-limit ones (frame
    limits 2 ... 40) make most requests retire by length, several in one tick."""
    from qwen3_tts_engine_amd.scheduler import SlotScheduler
    trace = osched.make_trace(seed=0, iterations=200, mean_arrivals=2.0, prompt=(32, 512),
                              lengths=lengths, cancel_rate=cancel_rate)
    ours = osched.drive(_Adapter(SlotScheduler(128, 512, step, bucket_kv)), trace, 128)
    ref = osched.drive(osched.ReferenceScheduler(128, 512, step, bucket_kv), trace, 128)
    assert len(ours) == len(ref) == 200
    for i, (a, b) in enumerate(zip(ours, ref)):
        assert a == b, f"iteration {i} differs"
    # the trace exercises the rules: growth past 512, a full arena, compaction on cancellation
    ops = [op for _, _, step_ops in ref for op in step_ops]
    assert any(op[0] == 'grow' for op in ops)
    if lengths[0] >= 200:
        assert max(r['capacity'] for r, _, _ in ref if r) >= 1024
        assert max(len(r['slots']) for r, _, _ in ref if r) == 128
    else:
        retired = sum(len(done) for _, done, _ in ref)
        assert retired > 300 and any(len(done) >= 2 for _, done, _ in ref)
        assert sum(op[0] == 'move' for op in ops) > 50
    if cancel_rate:
        assert any(op[0] == 'move' for op in ops)


def test_scheduler_rejects_invalid_geometry(pkg):
    from qwen3_tts_engine_amd.scheduler import SlotScheduler
    with pytest.raises(ValueError):
        SlotScheduler(48)
    with pytest.raises(ValueError):
        SlotScheduler(64, decode_bucket_step=3)
    s = SlotScheduler(4)
    s.admit([(0, 10, 50), (1, 10, 50), (2, 10, 50)])
    with pytest.raises(ValueError):
        s.admit([(3, 10, 50), (4, 10, 50)])
    assert len(s.states) == 3


@pytest.mark.gpu
@pytest.mark.parametrize("compact_prefix", [False, True])
def test_arena_follows_the_scheduler_bit_exact(pkg, device, compact_prefix):
    """The arena driven by the scheduler equals a numpy mirror of the reference's operations
    (full-row moves and regrowth copies).  With ``compact_prefix`` the moves copy only
    ``[:position + 1]`` and regrowth only the slots in use, so the comparison covers the rows
    every active request can still read: ``[:position]`` of each slot in use."""
    from qwen3_tts_engine_amd.scheduler import SlotScheduler
    from qwen3_tts_engine_amd.slots import SlotArena

    class Config:
        num_key_value_heads, head_dim, num_hidden_layers = 2, 16, 2

    class Talker(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = Config()
            self.layers = torch.nn.ModuleList([torch.nn.Identity(), torch.nn.Identity()])
            self.weight = torch.nn.Parameter(torch.zeros(1, dtype=torch.bfloat16))

    layers, slots, heads, width = 2, 8, 2, 16
    arena = SlotArena(Talker().to(device), slots, 16, packed_kv=True)
    sched = SlotScheduler(slots, 16, decode_bucket_step=4, bucket_kv=True, arena=arena,
                          compact_prefix=compact_prefix)
    mirror = np.zeros((2 * layers, slots, heads, 16, width), dtype=np.uint16)
    trace = osched.make_trace(seed=5, iterations=60, mean_arrivals=0.6, prompt=(3, 20), lengths=(4, 30),
                              cancel_rate=0.1)
    gen = torch.Generator().manual_seed(6)
    queue, active = [], []
    moves = 0
    for it, batch in enumerate(trace['arrivals']):
        queue.extend(batch)
        cancelled = [active[0]] if active and trace['cancels'][it] < trace['cancel_rate'] else []
        free = slots - (len(active) - len(cancelled))
        subs, queue = queue[:free], queue[free:]
        prefill = None
        if subs:
            longest = max(n for _, n, _ in subs)
            prefill = torch.randn(2 * layers, len(subs), heads, longest, width, generator=gen).bfloat16()
        # scheduler with device ops
        sched.ops = []
        sched.cancel(cancelled)
        sched.admit(subs, prefill.to(device) if prefill is not None else None)
        record = sched.decode_batch()
        moves += sum(op[0] == 'move' for op in sched.ops)
        # mirror the recorded operations on numpy
        for op in sched.ops:
            if op[0] == 'grow':
                grown = np.zeros(mirror.shape[:3] + (op[2],) + mirror.shape[4:], dtype=mirror.dtype)
                grown[:, :, :, :op[1]] = mirror
                mirror = grown
            elif op[0] == 'move':
                mirror[:, op[2]] = mirror[:, op[1]]
            elif op[0] == 'load':
                row = [i for i, (ident, _, _) in enumerate(subs) if ident == op[2]][0]
                mirror[:, op[1], :, :op[3]] = bits(prefill[:, row, :, :op[3]])
        if record is not None:
            positions = record.positions_tensor(device)
            for layer in range(layers):
                k = torch.randn(record.batch, heads, 1, width, generator=gen).bfloat16()
                v = torch.randn(record.batch, heads, 1, width, generator=gen).bfloat16()
                pkg.write(k.to(device), v.to(device), sched.arena.keys[layer][:record.batch],
                          sched.arena.values[layer][:record.batch], positions)
                okv.kv_write(mirror[layer], mirror[layers + layer], bits(k), bits(v), np.array(record.positions))
            sched.ops = []
            done = sched.advance()
            for op in sched.ops:
                assert op[0] == 'move'
                mirror[:, op[2]] = mirror[:, op[1]]
                moves += 1
        else:
            done = []
        torch.cuda.synchronize()
        if compact_prefix:
            got = bits(sched.arena.packed)
            for slot, state in enumerate(sched.states):
                n = state.position
                assert np.array_equal(got[:, slot, :, :n], mirror[:, slot, :, :n]), f"iteration {it} slot {slot}"
        else:
            assert np.array_equal(bits(sched.arena.packed), mirror), f"iteration {it}"
        active = [i for i in active if i not in cancelled and i not in done]
        active.extend(i for i, _, _ in subs if i not in done)
    assert sched.capacity > 16 and moves > 0


@pytest.mark.gpu
@pytest.mark.parametrize("packed", [True, False])
def test_prefix_move_and_active_regrowth(pkg, device, packed):
    """move(length=n) copies rows [:n] of every plane and leaves the destination's tail and
    every other slot untouched; grow_arena(active=n) carries slots [0, n) over unchanged."""
    from qwen3_tts_engine_amd.slots import SlotArena, grow_arena

    class Config:
        num_key_value_heads, head_dim, num_hidden_layers = 2, 16, 3

    class Talker(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = Config()
            self.layers = torch.nn.ModuleList([torch.nn.Identity() for _ in range(3)])
            self.weight = torch.nn.Parameter(torch.zeros(1, dtype=torch.bfloat16))

    arena = SlotArena(Talker().to(device), 6, 24, packed_kv=packed)
    gen = torch.Generator().manual_seed(9)
    for plane in arena.planes():
        plane.copy_(torch.randn(plane.shape, generator=gen).bfloat16().to(device))
    before = [bits(plane).copy() for plane in arena.planes()]
    arena.move(4, 1, length=7)
    torch.cuda.synchronize()
    for plane, old in zip(arena.planes(), before):
        expected = old.copy()
        expected[1, :, :7] = old[4, :, :7]
        assert np.array_equal(bits(plane), expected)
    arena.move(2, 0, length=100)  # clipped to the capacity: the whole row
    torch.cuda.synchronize()
    snapshot = [bits(plane).copy() for plane in arena.planes()]
    assert all(np.array_equal(p[0], p[2]) for p in snapshot)
    grown = grow_arena(arena, 30, active=3)
    torch.cuda.synchronize()
    assert grown.capacity == 48
    for plane, old in zip(grown.planes(), snapshot):
        assert np.array_equal(bits(plane)[:3, :, :24], old[:3])
