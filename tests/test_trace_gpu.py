"""The mixed continuous-batching trace on the HIP path, at talker shape.

The 128-slot, 200-iteration trace (seeded Poisson arrivals with mean 2, prompts U{32..512},
frame limits U{200..2000}, cancellations, decode bucket step 16 with bucket_kv: the third
setting of tests/golden/scheduler_trace.json), and the same trace with prompts up to 2000
tokens, drive SlotScheduler over a packed bf16 arena of 2 layers, 8 KV heads, head_dim 128,
starting at capacity 512 (continuous.py:353-363, 425-473, 541-657).  Every iteration runs the device side of a tick: prefix loads of the
admitted prompts from a seeded packed prefill cache (load_packed), compaction moves and
regrowth, then one fused decode step per layer (RoPE, the K/V write at the scheduled
positions, zero-position rows of the graph batch included, ragged GQA over keys
0 ... position).  A numpy mirror applies the same operations with the oracle (byte copies,
exact RoPE, the scatter write): the arena must equal it bit for bit at sampled iterations
and at the end, and the attention of sampled requests must match the float64 oracle."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import kv as okv
from oracle import rope as orope
from oracle import scheduler as osched
from tests._util import assert_attention_close, bits

pytestmark = pytest.mark.gpu

LAYERS, SLOTS, HQ, HKV, D = 2, 128, 16, 8, 128


class _Config:
    num_key_value_heads, head_dim, num_hidden_layers = HKV, D, LAYERS


class _Talker(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.config = _Config()
        self.layers = torch.nn.ModuleList([torch.nn.Identity() for _ in range(LAYERS)])
        self.weight = torch.nn.Parameter(torch.zeros(1, dtype=torch.bfloat16))


@pytest.mark.parametrize("prompt,grown", [((32, 512), 1024), ((32, 2000), 4096)])
def test_mixed_trace_on_the_hip_path(pkg, device, prompt, grown):
    """prompt (32, 512): the trace as specified (its positions stay below ~720 in 200
    iterations: one regrowth, 512 -> 1024).  prompt (32, 2000): the same trace with longer
    prompts, so that the capacity grows to 4096 and decode runs on the balanced grid
    (contexts of 2048 rows and more)."""
    from qwen3_tts_engine_amd.scheduler import SlotScheduler
    step, bucket_kv, cancel_rate = 16, True, 0.2
    trace = osched.make_trace(seed=0, iterations=200, mean_arrivals=2.0, prompt=prompt,
                              lengths=(200, 2000), cancel_rate=cancel_rate)
    arena = pkg.SlotArena(_Talker().to(device), SLOTS, 512, packed_kv=True)
    sched = SlotScheduler(SLOTS, 512, step, bucket_kv, arena=arena)
    reference = osched.ReferenceScheduler(SLOTS, 512, step, bucket_kv)
    mirror = np.zeros((2 * LAYERS, SLOTS, HKV, 512, D), dtype=np.uint16)
    gen = torch.Generator().manual_seed(50)
    queue, active = [], []
    checked_attention = 0
    samples = {0, 40, 80, 120, 160, 199}
    for it, arrivals in enumerate(trace['arrivals']):
        queue.extend(arrivals)
        cancelled = [active[0]] if active and trace['cancels'][it] < cancel_rate else []
        free = SLOTS - (len(active) - len(cancelled))
        subs, queue = queue[:free], queue[free:]
        prefill = None
        if subs:
            longest = max(n for _, n, _ in subs)
            prefill = torch.randn(2 * LAYERS, len(subs), HKV, longest, D, generator=gen).bfloat16()
        sched.ops = []
        sched.cancel(cancelled)
        sched.admit(subs, prefill.to(device) if prefill is not None else None)
        record = sched.decode_batch()
        # the integer state follows the reference's restatement
        ref_record, ref_done = reference.tick(subs, cancelled)
        mirror = _apply(mirror, sched.ops, subs, bits(prefill) if prefill is not None else None)
        done = []
        if record is not None:
            assert (record.batch, record.context, record.capacity) == (
                ref_record['batch'], ref_record['context'], ref_record['capacity'])
            assert record.positions == ref_record['positions'] and record.identifiers == ref_record['slots']
            positions = record.positions_tensor(device)
            cos, sin = pkg.rope_tables(positions, D)
            cb, sb = bits(cos)[:, None, None, :], bits(sin)[:, None, None, :]
            for layer in range(LAYERS):
                qkv = torch.randn(record.batch, 1, (HQ + 2 * HKV) * D, generator=gen).bfloat16()
                q = qkv[..., :HQ * D].view(record.batch, 1, HQ, D)
                k = qkv[..., HQ * D:(HQ + HKV) * D].view(record.batch, 1, HKV, D)
                v = qkv[..., (HQ + HKV) * D:].view(record.batch, 1, HKV, D)
                dq = qkv.to(device)
                out = pkg.decode_step(dq[..., :HQ * D].view(record.batch, 1, HQ, D),
                                      dq[..., HQ * D:(HQ + HKV) * D].view(record.batch, 1, HKV, D),
                                      dq[..., (HQ + HKV) * D:].view(record.batch, 1, HKV, D),
                                      sched.arena.keys[layer], sched.arena.values[layer], positions, cos, sin)
                k_rot = orope.rope_bf16(bits(k), cb, sb)
                okv.kv_write(mirror[layer], mirror[LAYERS + layer], k_rot.transpose(0, 2, 1, 3),
                             bits(v).transpose(0, 2, 1, 3), np.array(record.positions))
                if it in samples and layer == LAYERS - 1:
                    # attention of the longest, the shortest and a few other live requests
                    live = record.count
                    pos = np.array(record.positions[:live])
                    picks = sorted({int(np.argmax(pos)), int(np.argmin(pos)), 0, live - 1, live // 2})
                    q_rot = orope.rope_bf16(bits(q), cb, sb)
                    got = out.float().cpu().numpy()
                    for b in picks:
                        n = int(pos[b]) + 1
                        expected = oatt.decode_attention(
                            obf16.from_bits(q_rot[b:b + 1]), obf16.from_bits(mirror[layer][b:b + 1, :, :n]),
                            obf16.from_bits(mirror[LAYERS + layer][b:b + 1, :, :n]), [n - 1], D ** -0.5)
                        assert_attention_close(got[b:b + 1], expected)
                        checked_attention += 1
            sched.ops = []
            done = sched.advance()
            assert done == ref_done
            mirror = _apply(mirror, sched.ops, [], None)
        if it in samples:
            torch.cuda.synchronize()
            assert np.array_equal(bits(sched.arena.packed), mirror), f"iteration {it}"
            print(f"iteration {it}: capacity {sched.capacity}, {len(sched.states)} active, arena equal", flush=True)
        active = [i for i in active if i not in cancelled and i not in done]
        active.extend(i for i, _, _ in subs if i not in done)
    assert sched.capacity == grown and checked_attention >= 20


def _apply(mirror, ops, subs, prefill):
    """The arena operations of one scheduler phase on the numpy mirror: regrowth (the old
    rows copied, the rest zero, continuous.py:360-363), whole-slot moves (continuous.py:124-128)
    and prefix loads (packed_kv.py:21-31)."""
    for op in ops:
        if op[0] == 'grow':
            grown = np.zeros(mirror.shape[:3] + (op[2],) + mirror.shape[4:], dtype=mirror.dtype)
            grown[:, :, :, :op[1]] = mirror
            mirror = grown
        elif op[0] == 'move':
            mirror[:, op[2]] = mirror[:, op[1]]
        elif op[0] == 'load':
            row = [i for i, (ident, _, _) in enumerate(subs) if ident == op[2]][0]
            okv.copy_packed_prefix(mirror, prefill, op[1], row=row, length=op[3])
    return mirror
