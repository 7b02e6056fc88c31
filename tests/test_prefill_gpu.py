"""Varlen prefill on the GPU: the RoPE + arena-write prologue bit-exact against the oracle,
the causal GQA attention on MFMA tiles within the bf16 tolerance of the float64 oracle.

The prefill workload: 16 prompts with lengths torch.randint(32, 513, (16,)) under seed 0
(sum 4790), 16 query / 8 KV heads, head_dim 128, RoPE theta 1e6, rotated keys and values
written into arena slots, then causal attention over each prompt (PrefillGraph.compute,
prefill_graph.py:31-50, for the valid rows of each request)."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import rope as orope
from tests._util import assert_attention_close, bits, f64

pytestmark = pytest.mark.gpu


def _packed(lengths, q_heads, kv_heads, head_dim, seed):
    gen = torch.Generator().manual_seed(seed)
    total = int(sum(lengths))
    q = torch.randn(total, q_heads, head_dim, generator=gen).bfloat16()
    k = torch.randn(total, kv_heads, head_dim, generator=gen).bfloat16()
    v = torch.randn(total, kv_heads, head_dim, generator=gen).bfloat16()
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    positions = np.concatenate([np.arange(n) for n in lengths]) if total else np.zeros(0, np.int64)
    return q, k, v, cu, positions


def _tables(positions, head_dim):
    c, s = orope.tables(positions, orope.inv_freq(head_dim))
    return c, s


def test_prefill_workload_rope_write_and_attention(pkg, device):
    gen = torch.Generator().manual_seed(0)
    lengths = torch.randint(32, 513, (16,), generator=gen).tolist()
    assert sum(lengths) == 4790
    q_heads, kv_heads, head_dim, capacity, slots = 16, 8, 128, 512, 20
    q, k, v, cu, positions = _packed(lengths, q_heads, kv_heads, head_dim, 1)
    cos_b, sin_b = _tables(positions, head_dim)
    cos = torch.from_numpy(cos_b.view(np.int16)).view(torch.bfloat16).to(device)
    sin = torch.from_numpy(sin_b.view(np.int16)).view(torch.bfloat16).to(device)
    kv_slots = torch.randperm(slots, generator=torch.Generator().manual_seed(2))[:16]
    dg = torch.Generator(device=device).manual_seed(3)
    ak = torch.randn(slots, kv_heads, capacity, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    av = torch.randn(slots, kv_heads, capacity, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    before_k, before_v = bits(ak).copy(), bits(av).copy()
    dq, dk, dv, dcu = q.to(device), k.to(device), v.to(device), cu.to(device)
    q_rot = pkg.prefill_rope_write(dq, dk, dv, cos, sin, dcu, ak, av, kv_slots=kv_slots.to(device))
    out = pkg.prefill_attention(q_rot, ak, av, dcu, max(lengths), kv_slots=kv_slots.to(device))
    torch.cuda.synchronize()

    eq = orope.rope_bf16(bits(q), cos_b[:, None, :], sin_b[:, None, :])
    ek = orope.rope_bf16(bits(k), cos_b[:, None, :], sin_b[:, None, :])
    assert np.array_equal(bits(q_rot), eq)
    exp_k, exp_v = before_k.copy(), before_v.copy()
    vb = bits(v)
    for b, n in enumerate(lengths):
        s, t0 = int(kv_slots[b]), int(cu[b])
        exp_k[s, :, :n] = ek[t0:t0 + n].transpose(1, 0, 2)
        exp_v[s, :, :n] = vb[t0:t0 + n].transpose(1, 0, 2)
    assert np.array_equal(bits(ak), exp_k) and np.array_equal(bits(av), exp_v)
    expected = oatt.prefill_attention(obf16.from_bits(eq), obf16.from_bits(exp_k), obf16.from_bits(exp_v),
                                      cu.numpy(), head_dim ** -0.5, slots=kv_slots.numpy())
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("group", [1, 2, 4])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_prefill_rotates_queries_in_the_attention_kernel(pkg, device, group, head_dim):
    """prefill_step: the prologue writes only the keys and values, the attention kernel applies
    RoPE to the raw query rows as it loads them.  Same bits as the rotated-copy path (the
    rotation is the same bf16-exact arithmetic), and the query rows are left untouched."""
    lengths = [1, 15, 16, 17, 64, 65, 200, 333]
    kv_heads = 2
    q_heads = kv_heads * group
    q, k, v, cu, positions = _packed(lengths, q_heads, kv_heads, head_dim, 7 + group)
    cos_b, sin_b = _tables(positions, head_dim)
    cos = torch.from_numpy(cos_b.view(np.int16)).view(torch.bfloat16).to(device)
    sin = torch.from_numpy(sin_b.view(np.int16)).view(torch.bfloat16).to(device)
    dg = torch.Generator(device=device).manual_seed(8)
    ak = torch.randn(len(lengths), kv_heads, 384, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    av = torch.randn(len(lengths), kv_heads, 384, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    ak2, av2 = ak.clone(), av.clone()
    dq, dk, dv, dcu = q.to(device), k.to(device), v.to(device), cu.to(device)
    raw = bits(dq).copy()
    fused = pkg.prefill_step(dq, dk, dv, cos, sin, dcu, max(lengths), ak, av)
    q_rot = pkg.prefill_rope_write(dq, dk, dv, cos, sin, dcu, ak2, av2)
    chain = pkg.prefill_attention(q_rot, ak2, av2, dcu, max(lengths))
    torch.cuda.synchronize()
    assert np.array_equal(bits(dq), raw)
    assert torch.equal(ak, ak2) and torch.equal(av, av2)
    assert torch.equal(fused, chain)
    eq = orope.rope_bf16(bits(q), cos_b[:, None, :], sin_b[:, None, :])
    expected = oatt.prefill_attention(obf16.from_bits(eq), obf16.from_bits(bits(ak)), obf16.from_bits(bits(av)),
                                      cu.numpy(), head_dim ** -0.5)
    assert_attention_close(f64(fused), expected)


@pytest.mark.parametrize("group", [1, 2, 4])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_prefill_attention_tile_edges(pkg, device, group, head_dim):
    """Lengths on and around the 32-key and 64-query tile edges, an empty request and a
    single token; max_seqlen above the longest request."""
    lengths = [1, 0, 31, 32, 33, 64, 65, 127, 128, 129, 7]
    kv_heads = 2
    q_heads = kv_heads * group
    q, _, _, cu, _ = _packed(lengths, q_heads, kv_heads, head_dim, 10 + group)
    dg = torch.Generator(device=device).manual_seed(11)
    ak = torch.randn(len(lengths), kv_heads, 160, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    av = torch.randn(len(lengths), kv_heads, 160, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    out = torch.full((q.shape[0], q_heads, head_dim), float('nan'), device=device, dtype=torch.bfloat16)
    pkg.prefill_attention(q.to(device), ak, av, cu.to(device), 150, out=out)
    expected = oatt.prefill_attention(f64(q), f64(ak), f64(av), cu.numpy(), head_dim ** -0.5)
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("batch", [64, 80])
def test_prefill_many_requests(pkg, device, batch):
    """64 requests (the most the kernel numbers densely, longest blocks first) and 80 (the
    plain request-major numbering), with empty and one-token requests among them."""
    gen = torch.Generator().manual_seed(batch)
    lengths = torch.randint(0, 140, (batch,), generator=gen).tolist()
    lengths[3], lengths[10] = 0, 1
    kv_heads, q_heads, head_dim = 2, 4, 128
    q, _, _, cu, _ = _packed(lengths, q_heads, kv_heads, head_dim, 30)
    dg = torch.Generator(device=device).manual_seed(31)
    ak = torch.randn(batch, kv_heads, 144, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    av = torch.randn(batch, kv_heads, 144, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    out = torch.full((q.shape[0], q_heads, head_dim), float('nan'), device=device, dtype=torch.bfloat16)
    pkg.prefill_attention(q.to(device), ak, av, cu.to(device), max(lengths), out=out)
    expected = oatt.prefill_attention(f64(q), f64(ak), f64(av), cu.numpy(), head_dim ** -0.5)
    assert_attention_close(f64(out), expected)


def test_prefill_keys_past_capacity_do_not_exist(pkg, device):
    """A prompt longer than the arena: queries attend only keys below the capacity."""
    lengths, capacity = [40, 20], 32
    q, _, _, cu, _ = _packed(lengths, 4, 2, 64, 20)
    dg = torch.Generator(device=device).manual_seed(21)
    ak = torch.randn(2, 2, capacity, 64, generator=dg, device=device, dtype=torch.bfloat16)
    av = torch.randn(2, 2, capacity, 64, generator=dg, device=device, dtype=torch.bfloat16)
    out = pkg.prefill_attention(q.to(device), ak, av, cu.to(device), 40)
    k64, v64, q64 = f64(ak), f64(av), f64(q)
    expected = np.zeros_like(q64)
    for t in range(q.shape[0]):
        b = 0 if t < 40 else 1
        i = t if b == 0 else t - 40
        n = min(i, capacity - 1) + 1
        for hq in range(4):
            s = k64[b, hq // 2, :n] @ q64[t, hq] * 64 ** -0.5
            w = np.exp(s - s.max())
            expected[t, hq] = (w / w.sum()) @ v64[b, hq // 2, :n]
    assert_attention_close(f64(out), expected)


def test_prefill_step_replays_in_a_graph(pkg, device):
    lengths = [100, 37, 250]
    q, k, v, cu, positions = _packed(lengths, 16, 8, 128, 30)
    cos_b, sin_b = _tables(positions, 128)
    cos = torch.from_numpy(cos_b.view(np.int16)).view(torch.bfloat16).to(device)
    sin = torch.from_numpy(sin_b.view(np.int16)).view(torch.bfloat16).to(device)
    ak = torch.zeros(3, 8, 256, 128, device=device, dtype=torch.bfloat16)
    av = torch.zeros_like(ak)
    dq, dk, dv, dcu = q.to(device), k.to(device), v.to(device), cu.to(device)
    out = torch.empty(q.shape, device=device, dtype=torch.bfloat16)
    pkg.prefill_step(dq, dk, dv, cos, sin, dcu, 256, ak, av, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pkg.prefill_step(dq, dk, dv, cos, sin, dcu, 256, ak, av, out=out)
    gen = torch.Generator().manual_seed(31)
    for _ in range(3):
        dq.copy_(torch.randn(dq.shape, generator=gen).bfloat16().to(device))
        dk.copy_(torch.randn(dk.shape, generator=gen).bfloat16().to(device))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = pkg.prefill_step(dq, dk, dv, cos, sin, dcu, 256, ak, av)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)


def test_prefill_rejects_bad_arguments(pkg, device):
    q = torch.zeros(10, 16, 128, device=device, dtype=torch.bfloat16)
    ak = torch.zeros(2, 8, 64, 128, device=device, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32, device=device)
    with pytest.raises(ValueError):
        pkg.prefill_attention(q.float(), ak, ak, cu, 6)
    with pytest.raises(ValueError):
        pkg.prefill_attention(q, ak, ak, cu.long(), 6)
    with pytest.raises(ValueError):
        pkg.prefill_attention(q[:, :12], ak, ak, cu, 6)
    k = torch.zeros(10, 8, 128, device=device, dtype=torch.bfloat16)
    cos = torch.zeros(10, 128, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.prefill_rope_write(q, k, k, cos[:5], cos[:5], cu, ak, ak)
    with pytest.raises(ValueError):
        pkg.prefill_rope_write(q, k, k, cos, cos, cu, ak[:1], ak[:1])


def test_prefill_request_order_does_not_change_results(pkg, device):
    """tools/probe_prefill_graph.py:29-55 replays the same prompts in orders [0, 1, 2, 3] and
    [3, 0, 1, 2]: each prompt's arena rows and attention rows must not depend on where it
    sits in the packed batch (bit for bit), with every prompt keeping its slot."""
    lengths = [37, 200, 64, 129]
    q_heads, kv_heads, head_dim, capacity = 16, 8, 128, 256
    q, k, v, cu, positions = _packed(lengths, q_heads, kv_heads, head_dim, 11)
    cos_b, sin_b = _tables(positions, head_dim)
    cos = torch.from_numpy(cos_b.view(np.int16)).view(torch.bfloat16)
    sin = torch.from_numpy(sin_b.view(np.int16)).view(torch.bfloat16)
    rows = [slice(int(cu[b]), int(cu[b + 1])) for b in range(len(lengths))]
    results = []
    for order in ([0, 1, 2, 3], [3, 0, 1, 2]):
        pick = lambda t: torch.cat([t[rows[b]] for b in order]).to(device)
        ocu = torch.tensor(np.concatenate([[0], np.cumsum([lengths[b] for b in order])]),
                           dtype=torch.int32, device=device)
        ak = torch.zeros(4, kv_heads, capacity, head_dim, device=device, dtype=torch.bfloat16)
        av = torch.zeros_like(ak)
        out = pkg.prefill_step(pick(q), pick(k), pick(v), pick(cos), pick(sin), ocu, max(lengths), ak, av,
                               kv_slots=torch.tensor(order, device=device))
        torch.cuda.synchronize()
        starts = np.concatenate([[0], np.cumsum([lengths[b] for b in order])])
        per_prompt = {b: bits(out[int(starts[i]):int(starts[i + 1])]) for i, b in enumerate(order)}
        results.append((bits(ak), bits(av), per_prompt))
    (k0, v0, o0), (k1, v1, o1) = results
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    for b in range(len(lengths)):
        assert np.array_equal(o0[b], o1[b]), f"prompt {b}"
    expected = oatt.prefill_attention(obf16.from_bits(orope.rope_bf16(bits(q), cos_b[:, None, :], sin_b[:, None, :])),
                                      obf16.from_bits(k0), obf16.from_bits(v0), cu.numpy(), head_dim ** -0.5)
    got = np.concatenate([obf16.from_bits(o0[b]) for b in range(len(lengths))])
    assert_attention_close(got, expected)
