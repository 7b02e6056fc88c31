"""Golden fixtures of the attention/KV hot path, written by the oracle from seeded CPU inputs.

Regenerate from the repository root with ``python -m tests.golden.make_golden``.  Every input
is re-created from its seed by the builders below (torch's CPU generator, numpy's PCG64), so a
fixture holds expected outputs plus the few table inputs that are not a seed draw.  The
oracle functions that produce them are themselves pinned by the reference's known answers,
closed forms and torch-eager checks (tests/test_oracle.py); the fixtures freeze those
results so that the package (tests/test_golden_gpu.py) and any later change of the oracle
(tests/test_golden.py) are compared with the same numbers.

Fixtures:
  rope_bf16.npz          cos/sin bf16 rows (theta 1e6, D 128) at edge positions and the
                         bit-exact rotate-half of a seeded bf16 input under those rows
                         (rotary_triton_ascend.py:19-24, continuous.py:193)
  config1_fp32.npz       4 requests, contexts {37, 120, 5, 256}, fp32: RoPE at c_b, the
                         paired write at c_b and attention over L_b = c_b + 1 keys
                         (continuous.py:152-166, 191-192; npu_attention.py:11-26)
  config2_talker64.npz   the 64-request ragged talker step (contexts U[64, 1024], seed 0,
                         sum 32,718): digests of the arena after the write and the
                         attention output of 8 of the requests
  prefill16.npz          the 16-prompt prefill (lengths randint(32, 513), seed 0, 4790
                         tokens): SHA-256 of the arena after the rotated K/V write and the
                         attention output of each prompt's last token (prefill_graph.py:31-50)
  scheduler_trace.json   the 128-slot, 200-iteration mixed trace under three scheduler
                         settings: per-iteration decode records and device operations
                         (continuous.py:353-363, 425-473, 541-657)
"""
import hashlib
import json
import sys
import zlib
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import attention as oatt  # noqa: E402
from oracle import bf16 as obf16  # noqa: E402
from oracle import kv as okv  # noqa: E402
from oracle import rope as orope  # noqa: E402
from oracle import scheduler as osched  # noqa: E402

HQ, HKV, D = 16, 8, 128
ROPE_POSITIONS = [0, 1, 5, 37, 120, 256, 1023, 4095, 30000]
CONFIG1_CONTEXTS = [37, 120, 5, 256]
CONFIG2_SELECTED = [0, 1, 2, 31, 32, 63]  # plus the shortest and longest request
SCHEDULER_SETTINGS = [(0, False, 0.0), (8, True, 0.05), (16, True, 0.2)]


def to_bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def sha256(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---- inputs -------------------------------------------------------------------------------

def rope_input():
    """bf16 x of shape (positions, 1, 8, 128), N(0, 4) so that large and small values occur."""
    gen = torch.Generator().manual_seed(7)
    return to_bits((torch.randn(len(ROPE_POSITIONS), 1, HKV, D, generator=gen) * 2).bfloat16())


def config1_inputs():
    """Cache (4, 8, 257, 128) fp32 with N(0,1) keys/values at rows < c_b, zeros elsewhere;
    q (4, 1, 16, 128), new k/v (4, 1, 8, 128); seed 0, drawn in this order."""
    batch, capacity = len(CONFIG1_CONTEXTS), 257
    gen = torch.Generator().manual_seed(0)
    cache_k = torch.zeros(batch, HKV, capacity, D)
    cache_v = torch.zeros(batch, HKV, capacity, D)
    for b, c in enumerate(CONFIG1_CONTEXTS):
        cache_k[b, :, :c] = torch.randn(HKV, c, D, generator=gen)
        cache_v[b, :, :c] = torch.randn(HKV, c, D, generator=gen)
    q = torch.randn(batch, 1, HQ, D, generator=gen)
    k = torch.randn(batch, 1, HKV, D, generator=gen)
    v = torch.randn(batch, 1, HKV, D, generator=gen)
    return cache_k, cache_v, q, k, v


def config2_inputs():
    """Seed 0: contexts randint(64, 1025, (64,)), then the arena keys and values
    (64, 8, 1024, 128) and the fused QKV rows (64, 1, 4096), all N(0,1) rounded to bf16."""
    gen = torch.Generator().manual_seed(0)
    contexts = torch.randint(64, 1025, (64,), generator=gen)
    keys = torch.randn(64, HKV, 1024, D, generator=gen).bfloat16()
    values = torch.randn(64, HKV, 1024, D, generator=gen).bfloat16()
    qkv = torch.randn(64, 1, (HQ + 2 * HKV) * D, generator=gen).bfloat16()
    return contexts, keys, values, qkv


PREFILL_SLOTS, PREFILL_CAPACITY = 16, 512


def prefill_inputs():
    """Seed 0: lengths randint(32, 513, (16,)), then q (T, 16, 128), k and v (T, 8, 128),
    N(0,1) rounded to bf16; request b fills slot b of a zeroed (16, 8, 512, 128) arena."""
    gen = torch.Generator().manual_seed(0)
    lengths = torch.randint(32, 513, (16,), generator=gen)
    total = int(lengths.sum())
    q = torch.randn(total, HQ, D, generator=gen).bfloat16()
    k = torch.randn(total, HKV, D, generator=gen).bfloat16()
    v = torch.randn(total, HKV, D, generator=gen).bfloat16()
    cu = np.concatenate([[0], np.cumsum(lengths.numpy())]).astype(np.int32)
    positions = np.concatenate([np.arange(int(n)) for n in lengths])
    return lengths.numpy(), cu, positions, q, k, v


def split_qkv(qkv):
    q = qkv[..., :HQ * D].view(-1, 1, HQ, D)
    k = qkv[..., HQ * D:(HQ + HKV) * D].view(-1, 1, HKV, D)
    v = qkv[..., (HQ + HKV) * D:].view(-1, 1, HKV, D)
    return q, k, v


def config2_selected(contexts):
    c = contexts.tolist()
    return sorted(set(CONFIG2_SELECTED) | {int(np.argmin(c)), int(np.argmax(c))})


def scheduler_trace(cancel_rate):
    return osched.make_trace(seed=0, iterations=200, mean_arrivals=2.0, prompt=(32, 512),
                             lengths=(200, 2000), cancel_rate=cancel_rate)


def compact_records(records):
    """Per iteration: [batch, context, capacity, active slots, sum of positions, crc32 of the
    slot identifiers, crc32 of the positions], the finished identifiers and the device ops."""
    out = []
    for record, finished, ops in records:
        if record is None:
            row = None
        else:
            slots = np.asarray(record['slots'], dtype=np.int64)
            positions = np.asarray(record['positions'], dtype=np.int64)
            row = [int(record['batch']), int(record['context']), int(record['capacity']), len(slots),
                   int(positions.sum()), zlib.crc32(slots.tobytes()), zlib.crc32(positions.tobytes())]
        out.append({'record': row, 'finished': [int(i) for i in finished],
                    'ops': [[op[0], *[int(x) for x in op[1:]]] for op in ops]})
    return out


# ---- expected outputs (oracle) ---------------------------------------------------------------

def expected_rope():
    inv = orope.inv_freq(D)
    cos, sin = orope.tables(ROPE_POSITIONS, inv)
    y = orope.rope_bf16(rope_input(), cos[:, None, None, :], sin[:, None, None, :])
    return {'positions': np.asarray(ROPE_POSITIONS, dtype=np.int64), 'cos': cos, 'sin': sin, 'y': y}


def expected_config1():
    cache_k, cache_v, q, k, v = config1_inputs()
    cos, sin = orope.tables(np.asarray(CONFIG1_CONTEXTS)[:, None], orope.inv_freq(D), dtype="f32")
    c4, s4 = cos[:, :, None, :], sin[:, :, None, :]
    q_rot = orope.rope_f32(q.numpy(), c4, s4)
    k_rot = orope.rope_f32(k.numpy(), c4, s4)
    ek, ev = okv.kv_write(cache_k.numpy().copy(), cache_v.numpy().copy(), k_rot.transpose(0, 2, 1, 3),
                          v.numpy().transpose(0, 2, 1, 3), CONFIG1_CONTEXTS)
    out = oatt.decode_attention(q_rot, ek, ev, CONFIG1_CONTEXTS, D ** -0.5)
    return {'contexts': np.asarray(CONFIG1_CONTEXTS, dtype=np.int64), 'cos': cos, 'sin': sin,
            'q_rot': q_rot, 'k_rot': k_rot, 'out': out}


def expected_config2():
    contexts, keys, values, qkv = config2_inputs()
    cos, sin = orope.tables(contexts.numpy(), orope.inv_freq(D))
    q, k, v = split_qkv(qkv)
    cb, sb = cos[:, None, None, :], sin[:, None, None, :]
    q_rot = orope.rope_bf16(to_bits(q), cb, sb)
    k_rot = orope.rope_bf16(to_bits(k), cb, sb)
    ak, av = okv.kv_write(to_bits(keys), to_bits(values), k_rot.transpose(0, 2, 1, 3),
                          to_bits(v).transpose(0, 2, 1, 3), contexts.numpy())
    selected = config2_selected(contexts)
    out = oatt.decode_attention(obf16.from_bits(q_rot[selected]), obf16.from_bits(ak[selected]),
                                obf16.from_bits(av[selected]), contexts.numpy()[selected], D ** -0.5)
    return {'contexts': contexts.numpy().astype(np.int64), 'cos': cos, 'sin': sin,
            'selected': np.asarray(selected, dtype=np.int64), 'out': out.astype(np.float32),
            'keys_sha256': np.asarray(sha256(ak)), 'values_sha256': np.asarray(sha256(av)),
            'q_rot_sha256': np.asarray(sha256(q_rot))}


def prefill_tables(positions):
    """bf16 cos/sin rows of the prefill tokens (the oracle tables, pinned by rope_bf16.npz)."""
    return orope.tables(positions, orope.inv_freq(D))


def expected_prefill():
    lengths, cu, positions, q, k, v = prefill_inputs()
    cos, sin = prefill_tables(positions)
    q_rot = orope.rope_bf16(to_bits(q), cos[:, None, :], sin[:, None, :])
    k_rot = orope.rope_bf16(to_bits(k), cos[:, None, :], sin[:, None, :])
    ak = np.zeros((PREFILL_SLOTS, HKV, PREFILL_CAPACITY, D), np.uint16)
    av = np.zeros_like(ak)
    vb = to_bits(v)
    for b, n in enumerate(lengths):
        t0 = int(cu[b])
        ak[b, :, :n] = k_rot[t0:t0 + n].transpose(1, 0, 2)
        av[b, :, :n] = vb[t0:t0 + n].transpose(1, 0, 2)
    out = oatt.prefill_attention(obf16.from_bits(q_rot), obf16.from_bits(ak), obf16.from_bits(av), cu, D ** -0.5)
    last = cu[1:] - 1
    return {'lengths': lengths.astype(np.int64), 'last_tokens': last.astype(np.int64),
            'out_last': out[last].astype(np.float32),
            'keys_sha256': np.asarray(sha256(ak)), 'values_sha256': np.asarray(sha256(av))}


def expected_scheduler():
    runs = []
    for step, bucket_kv, cancel_rate in SCHEDULER_SETTINGS:
        records = osched.drive(osched.ReferenceScheduler(128, 512, step, bucket_kv),
                               scheduler_trace(cancel_rate), 128)
        runs.append({'decode_bucket_step': step, 'bucket_kv': bucket_kv, 'cancel_rate': cancel_rate,
                     'iterations': compact_records(records)})
    return {'slots': 128, 'initial_capacity': 512, 'runs': runs}


def main():
    np.savez_compressed(HERE / 'rope_bf16.npz', **expected_rope())
    np.savez_compressed(HERE / 'config1_fp32.npz', **expected_config1())
    np.savez_compressed(HERE / 'config2_talker64.npz', **expected_config2())
    np.savez_compressed(HERE / 'prefill16.npz', **expected_prefill())
    (HERE / 'scheduler_trace.json').write_text(json.dumps(expected_scheduler(), separators=(',', ':')))
    for p in sorted(HERE.glob('*.*')):
        print(p.name, p.stat().st_size)


if __name__ == '__main__':
    main()
