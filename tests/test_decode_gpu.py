"""Ragged GQA decode attention on the GPU against the float64 oracle.

Configs follow the build's workloads: config 1 (fp32 CPU-plumbing case, contexts
{37, 120, 5, 256}), config 2 (64-request ragged talker step, contexts U[64, 1024], seed 0),
and the code predictor's 16-slot cache (query length 2 at step 0).  Tolerance for bf16 I/O
with fp32 accumulation: max-abs <= 2e-2 and mean-abs <= 2e-3; fp32 I/O: 1e-5."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import kv as okv
from oracle import rope as orope
from tests._util import assert_attention_close, bits, f64, from_bits

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128

# (splits, max_chunks): the automatic grid, the chunked grid with several chunk counts and the
# balanced grid with several workgroup counts per KV head (1: one workgroup streams every
# request of a head in turn; 1000: shares of ~32 keys, most requests split in many parts)
GRIDS = [(0, 0), (-1, 0), (-1, 1), (-1, 3), (-1, 16), (-1, 1000), (1, 0), (7, 0), (128, 0), (1000, 0)]


def _arena(batch, capacity, dtype, device, seed, kv_heads=HKV, head_dim=D):
    gen = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(batch, kv_heads, capacity, head_dim, generator=gen, device=device, dtype=dtype)
    v = torch.randn(batch, kv_heads, capacity, head_dim, generator=gen, device=device, dtype=dtype)
    return k, v


def test_config1_fp32_write_rope_attention(pkg, device):
    """4 requests, contexts {37,120,5,256}, fp32: RoPE at position c_b, write at c_b,
    attend L_b = c_b + 1 keys."""
    contexts = [37, 120, 5, 256]
    batch, capacity = 4, 257
    gen = torch.Generator().manual_seed(0)
    cache_k = torch.zeros(batch, HKV, capacity, D)
    cache_v = torch.zeros(batch, HKV, capacity, D)
    for b, c in enumerate(contexts):
        cache_k[b, :, :c] = torch.randn(HKV, c, D, generator=gen)
        cache_v[b, :, :c] = torch.randn(HKV, c, D, generator=gen)
    q = torch.randn(batch, 1, HQ, D, generator=gen)
    k = torch.randn(batch, 1, HKV, D, generator=gen)
    v = torch.randn(batch, 1, HKV, D, generator=gen)
    positions = torch.tensor(contexts)
    inv = pkg.inverse_frequencies(D)
    cos, sin = pkg.rope_tables(positions.to(device)[:, None], D, dtype=torch.float32)
    q_rot = pkg.rotary(q.to(device), cos, sin)
    k_rot = pkg.rotary(k.to(device), cos, sin)
    dk, dv = cache_k.to(device), cache_v.to(device)
    pkg.write(k_rot.transpose(1, 2), v.to(device).transpose(1, 2), dk, dv, positions.to(device))
    out = pkg.decode_attention(q_rot, dk, dv, positions.to(device))
    # oracle chain
    ocos, osin = orope.tables(positions.numpy()[:, None], inv.numpy(), dtype="f32")
    np.testing.assert_allclose(cos.cpu().numpy(), ocos, atol=2.5e-7, rtol=0)
    c_np, s_np = cos.cpu().numpy()[:, :, None, :], sin.cpu().numpy()[:, :, None, :]
    eq = orope.rope_f32(q.numpy(), c_np, s_np)
    ek_rot = orope.rope_f32(k.numpy(), c_np, s_np)
    assert np.array_equal(q_rot.cpu().numpy(), eq) and np.array_equal(k_rot.cpu().numpy(), ek_rot)
    ek, ev = okv.kv_write(cache_k.numpy().copy(), cache_v.numpy().copy(),
                          ek_rot.transpose(0, 2, 1, 3), v.numpy().transpose(0, 2, 1, 3), contexts)
    assert np.array_equal(dk.cpu().numpy(), ek) and np.array_equal(dv.cpu().numpy(), ev)
    expected = oatt.decode_attention(eq, ek, ev, contexts, D ** -0.5)
    np.testing.assert_allclose(f64(out), expected, atol=1e-5, rtol=0)


def _config2(device, capacity=1024, seed=0):
    gen = torch.Generator().manual_seed(seed)
    contexts = torch.randint(64, 1025, (64,), generator=gen)
    k, v = _arena(64, capacity, torch.bfloat16, device, seed + 1)
    qkv = torch.randn(64, 1, (HQ + 2 * HKV) * D, generator=gen).bfloat16().to(device)
    q = qkv[..., :HQ * D].view(64, 1, HQ, D)
    kn = qkv[..., HQ * D:(HQ + HKV) * D].view(64, 1, HKV, D)
    vn = qkv[..., (HQ + HKV) * D:].view(64, 1, HKV, D)
    return contexts, k, v, q, kn, vn


def _expected_fused(contexts, k, v, q, kn, vn, cos, sin):
    cb, sb = bits(cos)[:, None, None, :], bits(sin)[:, None, None, :]
    q_rot = orope.rope_bf16(bits(q), cb, sb)
    k_rot = orope.rope_bf16(bits(kn), cb, sb)
    ak, av = okv.kv_write(bits(k).copy(), bits(v).copy(), k_rot.transpose(0, 2, 1, 3),
                          bits(vn).transpose(0, 2, 1, 3), contexts.numpy())
    out = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(ak), obf16.from_bits(av),
                                contexts.numpy(), D ** -0.5)
    return ak, av, out


@pytest.mark.parametrize("grid", ["bundled", "chunked", "balanced"])
def test_config2_fused_decode_step_on_each_named_grid(pkg, device, grid):
    """The headline step on each grid by name (the automatic choice for it is 'bundled')."""
    contexts, k, v, q, kn, vn = _config2(device, seed=11)
    positions = contexts.to(device)
    cos, sin = pkg.rope_tables(positions, D)
    expected_k, expected_v, expected = _expected_fused(contexts, k, v, q, kn, vn, cos, sin)
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin, grid=grid)
    assert np.array_equal(bits(k), expected_k) and np.array_equal(bits(v), expected_v)
    assert_attention_close(f64(out)[:, 0], expected[:, 0])


@pytest.mark.parametrize("group", [1, 2, 4])
@pytest.mark.parametrize("batch,capacity", [(6, 96), (64, 1024), (128, 640)])
@pytest.mark.parametrize("fused", [False, True])
def test_bundled_grid_edges(pkg, device, group, batch, capacity, fused):
    """The bundled grid (one workgroup per CU, requests ranked by length and bundled longest
    with shortest, K/V streamed through LDS, bf16 MFMA scores) against the oracle, with the
    edge lengths: position 0 (only the step's key), the last arena row, lengths on and around
    the 16- and 64-key boundaries of its tiles, repeated lengths (rank ties), invalid
    positions (zero rows, nothing written), and bundles left empty (6 requests over 256
    workgroups)."""
    gen = torch.Generator().manual_seed(80 + group + batch)
    kv_heads = HKV if group < 4 else 4
    q_heads = kv_heads * group
    contexts = torch.randint(0, capacity, (batch,), generator=gen)
    edge = torch.tensor([0, capacity - 1, 15, 16, 17, 63, 64, 65, 127, 128, 63, 63, -1, capacity])
    contexts[:min(batch, len(edge))] = edge[:min(batch, len(edge))]
    k, v = _arena(batch, capacity, torch.bfloat16, device, 81, kv_heads=kv_heads)
    q = torch.randn(batch, 1, q_heads, D, generator=gen).bfloat16().to(device)
    positions = contexts.to(device)
    valid = (contexts >= 0) & (contexts < capacity)
    if fused:
        kn = torch.randn(batch, 1, kv_heads, D, generator=gen).bfloat16().to(device)
        vn = torch.randn(batch, 1, kv_heads, D, generator=gen).bfloat16().to(device)
        cos, sin = pkg.rope_tables(positions.clamp(0, capacity - 1), D)
        before_k, before_v = bits(k).copy(), bits(v).copy()
        out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin, grid="bundled")
        cb, sb = bits(cos)[:, None, None, :], bits(sin)[:, None, None, :]
        q_rot = obf16.from_bits(orope.rope_bf16(bits(q), cb, sb))
        k_rot = orope.rope_bf16(bits(kn), cb, sb)
        ek, ev = before_k.copy(), before_v.copy()
        for b in np.flatnonzero(valid.numpy()):
            ek[b, :, contexts[b]] = k_rot[b, 0]
            ev[b, :, contexts[b]] = bits(vn)[b, 0]
        assert np.array_equal(bits(k), ek) and np.array_equal(bits(v), ev)
        keys, values, query = obf16.from_bits(ek), obf16.from_bits(ev), q_rot
    else:
        out = pkg.decode_attention(q, k, v, positions, grid="bundled")
        keys, values, query = f64(k), f64(v), f64(q)
    got = f64(out)
    assert not got[~valid.numpy()].any()
    idx = np.flatnonzero(valid.numpy())
    expected = oatt.decode_attention(query[idx], keys[idx], values[idx], contexts.numpy()[idx], D ** -0.5)
    assert_attention_close(got[idx], expected)
    # the same launch from the step's plan: each request is still scored whole by one
    # workgroup in the same order, so the outputs are bit-identical; and masked by
    # SlotGraph.compute's mask (0 up to each position, the most negative bf16 after): the same
    # arena rows, outputs in the bar
    plan = pkg.decode_plan(positions, capacity, q_heads, kv_heads)
    allowed = torch.arange(capacity, device=device)[None, :] <= positions[:, None]
    mask = torch.where(allowed, 0.0, torch.finfo(torch.bfloat16).min).to(torch.bfloat16)[:, None, None, :]
    if fused:
        k2, v2 = from_bits(before_k, device), from_bits(before_v, device)
        planned = pkg.decode_step(q, kn, vn, k2, v2, positions, cos, sin, grid="bundled", plan=plan)
        assert np.array_equal(bits(k2), bits(k)) and np.array_equal(bits(v2), bits(v))
        k3, v3 = from_bits(before_k, device), from_bits(before_v, device)
        masked = pkg.decode_step(q, kn, vn, k3, v3, positions, cos, sin, grid="bundled", plan=plan, mask=mask)
        assert np.array_equal(bits(k3), bits(k)) and np.array_equal(bits(v3), bits(v))
    else:
        planned = pkg.decode_attention(q, k, v, positions, grid="bundled", plan=plan)
        masked = pkg.decode_attention(q, k, v, positions, grid="bundled", plan=plan, mask=mask)
    assert torch.equal(planned, out)
    got = f64(masked)
    assert not got[~valid.numpy()].any()
    assert_attention_close(got[idx], expected)


PER_BUNDLE = 4


def plan_parts(plan):
    """Views of a plan tensor: its header (batch, M) and its table (M, 4, 2): four (request,
    length) pairs for each of the M bundles (workgroups) of a KV head."""
    return plan[:2], plan[2:].view(-1, PER_BUNDLE, 2)


def check_plan(plan, contexts, capacity, kv_heads):
    """The plan's contract: the header (batch, M) with M = max(ceil(256 / kv_heads),
    ceil(batch / 4)); every request of the batch listed once, with its length L = pos + 1
    (0 for a position outside the arena), (-1, 0) in unused slots; bundle m holding the
    requests of length ranks m, 2M-1-m, 2M+m, 4M-1-m, ranked longest first with ties by index
    (checked against a sort done here).  Returns the keys of each bundle."""
    header, table = (t.cpu().numpy() for t in plan_parts(plan))
    batch = len(contexts)
    bundles = max(-(-256 // kv_heads), -(-batch // PER_BUNDLE))
    assert list(header) == [batch, bundles] and table.shape == (bundles, PER_BUNDLE, 2)
    lengths = np.where((contexts >= 0) & (contexts < capacity), contexts + 1, 0)
    order = sorted(range(batch), key=lambda b: (-lengths[b], b))
    for m in range(bundles):
        for k, r in enumerate((m, 2 * bundles - 1 - m, 2 * bundles + m, 4 * bundles - 1 - m)):
            want = (order[r], lengths[order[r]]) if r < batch else (-1, 0)
            assert tuple(table[m, k]) == want, (m, k)
    return table[:, :, 1].sum(1)


@pytest.mark.parametrize("batch,capacity,group", [(1, 1024, 2), (6, 1024, 2), (64, 1024, 2), (100, 2048, 1),
                                                  (128, 1024, 4), (16, 4096, 3)])
def test_decode_plan_pairs_longest_with_shortest(pkg, device, batch, capacity, group):
    """The step's plan on the device: ties (a third of the requests share one length),
    invalid positions (negative, at or past the capacity: length 0), more requests than
    bundles (128 requests over 4 KV heads: four per bundle) and fewer (one request)."""
    gen = torch.Generator().manual_seed(900 + batch)
    contexts = torch.randint(-2, capacity + 2, (batch,), generator=gen)
    contexts[: batch // 3] = contexts[0]
    kv_heads = 8 if group < 4 else 4
    plan = pkg.decode_plan(contexts.to(device), capacity, kv_heads * group, kv_heads)
    assert tuple(plan.shape) == pkg.plan_shape(batch, kv_heads * group, kv_heads) and plan.dtype == torch.int32
    check_plan(plan, contexts.numpy(), capacity, kv_heads)
    with pytest.raises(ValueError):
        pkg.decode_plan(torch.zeros(129, dtype=torch.int64, device=device), capacity, 16, 8)
    with pytest.raises(ValueError):
        pkg.decode_plan(contexts.to(device), capacity, 40, 8)   # 5 query heads per KV head


def test_decode_plan_of_the_talker_step(pkg, device):
    """The headline step's plan: 32 bundles per head of two requests each, 936 to 1099 keys
    for a mean of 1024 (the seed-0 draw: 32,782 keys per head)."""
    contexts, *_ = _config2(device)
    plan = pkg.decode_plan(contexts.to(device), 1024, HQ, HKV)
    keys = check_plan(plan, contexts.numpy(), 1024, HKV)
    assert keys.sum() == 32782 and (plan_parts(plan)[1][:, 2:, 0] == -1).all().item()
    assert keys.min() == 936 and keys.max() == 1099


@pytest.mark.parametrize("masked", [False, True])
def test_decode_plan_of_other_positions_stays_in_bounds(pkg, device, masked):
    """A plan is only valid for the positions it was made from.  A stale one (made for other
    positions) or a malformed one (entries naming no request, lengths past the arena) gives
    other outputs but touches nothing outside the arguments: the fused step writes the new
    K/V rows at the rows the plan names (the last key of each request it lists) and nowhere
    else, and the output rows of requests it does not name stay as they were.  A plan of
    another batch is not used (the launch ranks the requests itself)."""
    contexts, k, v, q, kn, vn = _config2(device, seed=13)
    positions = contexts.to(device)
    cos, sin = pkg.rope_tables(positions, D)
    mask = None
    if masked:  # keys up to 1023 allowed: the positions and the plan's lengths decide
        mask = torch.zeros(64, 1, 1, 1024, device=device, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(14)
    stale_ctx = torch.randint(64, 1025, (64,), generator=gen)
    stale = pkg.decode_plan(stale_ctx.to(device), 1024, HQ, HKV)
    before_k, before_v = bits(k).copy(), bits(v).copy()
    pkg.decode_step(q, kn, vn, k, v, positions, cos, sin, grid="bundled", plan=stale, mask=mask)
    torch.cuda.synchronize()
    changed = np.argwhere((bits(k) != before_k).any(-1) | (bits(v) != before_v).any(-1))
    allowed = {(b, h, int(stale_ctx[b])) for b in range(64) for h in range(HKV)}
    assert changed.shape[0] > 0 and {tuple(int(x) for x in r) for r in changed} <= allowed
    bad = stale.clone()
    table = plan_parts(bad)[1].view(-1, 2)
    table[::3, 0] = 1000       # no such request: the slot attends nothing
    table[1::3, 1] = 5000      # more keys than the arena has: clamped
    named = set(int(b) for b in table[:, 0].cpu().tolist() if 0 <= b < 64)
    out = torch.full((64, 1, HQ, D), 7.0, device=device, dtype=torch.bfloat16)
    pkg.decode_attention(q, k, v, positions, grid="bundled", plan=bad, out=out, mask=mask)
    torch.cuda.synchronize()
    assert len(named) < 64
    for b in range(64):
        if b not in named:
            assert torch.all(out[b] == 7.0)
    other = pkg.decode_plan(positions[:60], 1024, HQ, HKV)  # 60 requests: the same plan shape
    out = pkg.decode_attention(q, k, v, positions, grid="bundled", plan=other, mask=mask)
    assert torch.equal(out, pkg.decode_attention(q, k, v, positions, grid="bundled", mask=mask))
    with pytest.raises(ValueError):
        pkg.decode_attention(q, k, v, positions, grid="bundled", plan=stale[:10], mask=mask)


def test_bundled_grid_is_deterministic_and_refuses_what_it_cannot_run(pkg, device):
    """Repeated launches are bit-identical, with and without the step's plan and a mask (a
    bool mask of the positions' own range gives the unmasked result bit for bit); asked for
    by name, the grid refuses a mask without unit key stride, two query tokens and fp32 rows
    (the automatic choice runs them on another grid)."""
    contexts, k, v, q, _, _ = _config2(device, seed=12)
    positions = contexts.to(device)
    first = pkg.decode_attention(q, k, v, positions, grid="bundled").clone()
    for _ in range(10):
        assert torch.equal(pkg.decode_attention(q, k, v, positions, grid="bundled"), first)
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), contexts.numpy(), D ** -0.5)
    assert_attention_close(f64(first), expected)
    plan = pkg.decode_plan(positions, 1024, HQ, HKV)
    assert torch.equal(pkg.decode_attention(q, k, v, positions, grid="bundled", plan=plan), first)
    mask = torch.zeros(64, 1, 1, 1024, device=device, dtype=torch.bfloat16)
    planned = pkg.decode_attention(q, k, v, positions, grid="bundled", plan=plan, mask=mask).clone()
    for _ in range(10):
        assert torch.equal(pkg.decode_attention(q, k, v, positions, grid="bundled", plan=plan, mask=mask), planned)
    assert_attention_close(f64(planned), expected)
    keep = torch.arange(1024, device=device)[None, None, None, :] <= positions[:, None, None, None]
    assert torch.equal(pkg.decode_attention(q, k, v, positions, mask=keep, grid="bundled"), first)
    wide = torch.arange(2048, device=device)[None, None, None, :] <= 2 * positions[:, None, None, None]
    with pytest.raises(ValueError, match="unsupported"):
        pkg.decode_attention(q, k, v, positions, mask=wide[..., ::2], grid="bundled")
    with pytest.raises(ValueError, match="unsupported"):
        pkg.decode_attention(q.float(), k.float(), v.float(), positions, grid="bundled")
    with pytest.raises(ValueError, match="unsupported"):
        pkg.decode_attention(torch.cat([q, q], 1), k, v, positions, grid="bundled")
    with pytest.raises(ValueError):
        pkg.decode_attention(q, k, v, positions, grid="striped")


@pytest.mark.parametrize("splits,max_chunks", GRIDS)
def test_config2_fused_decode_step(pkg, device, splits, max_chunks):
    """The headline step: RoPE + write + ragged GQA over 64 requests, seed 0 (sum c = 32718),
    on every grid."""
    contexts, k, v, q, kn, vn = _config2(device)
    assert int(contexts.sum()) == 32718
    positions = contexts.to(device)
    cos, sin = pkg.rope_tables(positions, D)
    expected_k, expected_v, expected = _expected_fused(contexts, k, v, q, kn, vn, cos, sin)
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin, max_chunks=max_chunks, splits=splits)
    assert np.array_equal(bits(k), expected_k) and np.array_equal(bits(v), expected_v)
    assert_attention_close(f64(out)[:, 0], expected[:, 0])


def _expected_fused_tokens(k, v, q, kn, vn, positions, cos, sin):
    """Oracle chain of a fused step of S tokens at positions p - S + 1 ... p: per-token RoPE of
    the query and key rows, the paired write, causal attention (query t sees keys <= p - S + 1 + t)."""
    tokens = q.shape[1]
    cb, sb = bits(cos)[:, :, None, :], bits(sin)[:, :, None, :]
    q_rot = orope.rope_bf16(bits(q), cb, sb)
    k_rot = orope.rope_bf16(bits(kn), cb, sb)
    ak, av = okv.kv_write(bits(k).copy(), bits(v).copy(), k_rot.transpose(0, 2, 1, 3),
                          bits(vn).transpose(0, 2, 1, 3), positions - tokens + 1)
    out = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(ak), obf16.from_bits(av),
                                positions, D ** -0.5)
    return ak, av, out


@pytest.mark.parametrize("group", [1, 2, 4])
@pytest.mark.parametrize("splits,max_chunks", [(0, 0), (-1, 1), (-1, 3), (1, 0), (5, 0), (64, 0)])
def test_fused_two_token_step(pkg, device, group, splits, max_chunks):
    """The code predictor's first step as one launch (continuous.py:37-40: two tokens, 2x2
    causal): RoPE of both tokens, the paired write at p - 1 and p, attention with query 0
    blind to key p.  Positions include chunk boundaries (the new key p - 1 in an earlier
    chunk than p) and the first two arena rows."""
    kv_heads, batch, capacity = 4, 9, 300
    q_heads = kv_heads * group
    k, v = _arena(batch, capacity, torch.bfloat16, device, 41 + group, kv_heads=kv_heads)
    gen = torch.Generator().manual_seed(40 + group + max_chunks + 7 * abs(splits))
    positions = torch.tensor([1, 2, 63, 64, 65, 128, 200, 298, 299])
    qkv = torch.randn(batch, 2, (q_heads + 2 * kv_heads) * D, generator=gen).bfloat16().to(device)
    q = qkv[..., :q_heads * D].view(batch, 2, q_heads, D)
    kn = qkv[..., q_heads * D:(q_heads + kv_heads) * D].view(batch, 2, kv_heads, D)
    vn = qkv[..., (q_heads + kv_heads) * D:].view(batch, 2, kv_heads, D)
    token_positions = torch.stack([positions - 1, positions], 1)
    cos, sin = pkg.rope_tables(token_positions.to(device), D)
    expected_k, expected_v, expected = _expected_fused_tokens(k, v, q, kn, vn, positions.numpy(), cos, sin)
    out = pkg.decode_step(q, kn, vn, k, v, positions.to(device), cos, sin, max_chunks=max_chunks,
                          splits=splits)
    assert np.array_equal(bits(k), expected_k) and np.array_equal(bits(v), expected_v)
    assert_attention_close(f64(out), expected)


def test_fused_two_token_predictor_first_step(pkg, device):
    """Batch 64, 8 KV heads, a fresh 16-position predictor cache: the first step writes rows
    0 and 1 and attends them causally; the unfused chain (rotary, write_tokens, two-query
    decode) gives the same cache and output."""
    batch = 64
    k = torch.zeros(batch, HKV, 16, D, device=device, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    gen = torch.Generator().manual_seed(44)
    rows = torch.randn(batch, 2, HQ + 2 * HKV, D, generator=gen).bfloat16().to(device)
    q, kn, vn = rows[:, :, :HQ], rows[:, :, HQ:HQ + HKV], rows[:, :, HQ + HKV:]
    positions = torch.ones(batch, dtype=torch.int64, device=device)
    cos, sin = pkg.rope_tables(torch.arange(2, device=device).expand(batch, 2).contiguous(), D)
    expected_k, expected_v, expected = _expected_fused_tokens(k, v, q, kn, vn, positions.cpu().numpy(), cos, sin)
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin)
    assert np.array_equal(bits(k), expected_k) and np.array_equal(bits(v), expected_v)
    assert_attention_close(f64(out), expected)
    k2, v2 = torch.zeros_like(k), torch.zeros_like(v)
    q_rot = pkg.rotary(q.contiguous(), cos, sin)
    k_rot = pkg.rotary(kn.contiguous(), cos, sin)
    pkg.write_tokens(k_rot.transpose(1, 2), vn.transpose(1, 2), k2, v2, torch.zeros_like(positions))
    chain = pkg.decode_attention(q_rot, k2, v2, positions)
    assert torch.equal(k, k2) and torch.equal(v, v2)
    assert (out.float() - chain.float()).abs().max().item() <= 1e-2


def test_fused_matches_unfused_chain(pkg, device):
    """rotary -> write -> decode_attention gives the same output as the fused launch."""
    contexts, k, v, q, kn, vn = _config2(device, seed=3)
    positions = contexts.to(device)
    cos, sin = pkg.rope_tables(positions, D)
    k2, v2 = k.clone(), v.clone()
    fused = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin)
    q_rot = pkg.rotary(q.contiguous(), cos[:, None], sin[:, None])
    k_rot = pkg.rotary(kn.contiguous(), cos[:, None], sin[:, None])
    pkg.write(k_rot.transpose(1, 2), vn.transpose(1, 2), k2, v2, positions)
    chain = pkg.decode_attention(q_rot, k2, v2, positions)
    assert torch.equal(k, k2) and torch.equal(v, v2)
    diff = (fused.float() - chain.float()).abs()
    assert diff.max().item() <= 1e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("group", [1, 2, 4])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("qlen", [1, 2])
def test_decode_shapes(pkg, device, dtype, group, head_dim, qlen):
    kv_heads, batch, capacity = 4, 9, 300
    gen = torch.Generator().manual_seed(group * 100 + head_dim + qlen)
    lengths = torch.tensor([1, 2, 3, 17, 64, 65, 128, 255, 300])[:batch]
    positions = lengths - 1
    if qlen == 2:
        positions = positions.clamp(min=1)
    k, v = _arena(batch, capacity, dtype, device, 11, kv_heads=kv_heads, head_dim=head_dim)
    q = torch.randn(batch, qlen, kv_heads * group, head_dim, generator=gen).to(dtype).to(device)
    out = pkg.decode_attention(q, k, v, positions.to(device))
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), positions.numpy(), head_dim ** -0.5)
    if dtype == torch.float32:
        np.testing.assert_allclose(f64(out), expected, atol=1e-5, rtol=0)
    else:
        assert_attention_close(f64(out), expected)


def test_poisoned_tail_is_never_read(pkg, device):
    """Keys beyond pos[b] hold stale or garbage data (tools/probe_attention_context.py:53-55):
    inf/NaN there must not leak into the output."""
    contexts, k, v, q, _, _ = _config2(device, seed=5)
    positions = contexts.to(device)
    mask = torch.arange(1024, device=device)[None, :] > positions[:, None]
    clean = pkg.decode_attention(q, k, v, positions).clone()
    k.masked_fill_(mask[:, None, :, None], float('inf'))
    v.masked_fill_(mask[:, None, :, None], float('nan'))
    poisoned = pkg.decode_attention(q, k, v, positions)
    assert torch.equal(clean, poisoned)


@pytest.mark.parametrize("kind", ["additive_bf16", "additive_f32", "bool"])
def test_mask_matches_sdpa_semantics(pkg, device, kind):
    """SlotGraph's additive mask (0 / finfo.min for j <= pos, continuous.py:191-192) over the
    whole arena equals the position-limited attention; an arbitrary mask follows SDPA."""
    batch, capacity = 8, 256
    k, v = _arena(batch, capacity, torch.bfloat16, device, 21)
    gen = torch.Generator().manual_seed(22)
    q = torch.randn(batch, 1, HQ, D, generator=gen).bfloat16().to(device)
    allowed = torch.rand(batch, 1, capacity, generator=gen) < 0.6
    allowed[:, :, 0] = True
    if kind == "bool":
        mask = allowed
    else:
        dtype = torch.bfloat16 if kind == "additive_bf16" else torch.float32
        mask = torch.where(allowed, 0.0, torch.finfo(dtype).min).to(dtype)
    full = torch.full((batch,), capacity - 1, dtype=torch.int64, device=device)
    out = pkg.decode_attention(q, k, v, full, mask=mask[:, None].to(device))
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), full.cpu().numpy(), D ** -0.5,
                                     mask=allowed.numpy())
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("kind", ["bool", "additive_bf16"])
def test_masked_full_arena_probe_shape(pkg, device, kind):
    """The reference's attention-context probe (tools/probe_attention_context.py:20-36): 64
    requests over a 512-row arena, positions (7 b) mod 512, the mask over all 512 keys; the
    launch reads more than 16 MB, so it takes the non-temporal loads."""
    batch, capacity = 64, 512
    k, v = _arena(batch, capacity, torch.bfloat16, device, 31)
    gen = torch.Generator().manual_seed(32)
    q = torch.randn(batch, 1, HQ, D, generator=gen).bfloat16().to(device)
    positions = (torch.arange(batch) * 7) % capacity
    allowed = torch.arange(capacity)[None, :] <= positions[:, None]
    if kind == "bool":
        mask = allowed
    else:
        mask = torch.where(allowed, 0.0, torch.finfo(torch.bfloat16).min).bfloat16()
    full = torch.full((batch,), capacity - 1, dtype=torch.int64, device=device)
    out = pkg.decode_attention(q, k, v, full, mask=mask[:, None, None].to(device))
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), positions.numpy(), D ** -0.5)
    assert_attention_close(f64(out), expected)


def test_trimmed_context_equals_masked_arena(pkg, device):
    """tests/test_slot_context.py:32-36: attention over the trimmed context equals
    attention over the full arena under the j <= pos mask."""
    batch, capacity = 2, 256
    k, v = _arena(batch, capacity, torch.float32, device, 42, kv_heads=2, head_dim=64)
    gen = torch.Generator().manual_seed(42)
    q = torch.randn(batch, 1, 2, 64, generator=gen).to(device)
    for context, pos in ((64, [63, 17]), (128, [64, 127])):
        positions = torch.tensor(pos, device=device)
        mask = torch.arange(capacity, device=device)[None, :] <= positions[:, None]
        full = pkg.decode_attention(q, k, v, torch.full_like(positions, capacity - 1),
                                    mask=mask[:, None, None])
        trimmed = pkg.decode_attention(q, k[:, :, :context], v[:, :, :context], positions)
        torch.testing.assert_close(trimmed, full, atol=1e-6, rtol=1e-6)


def test_predictor_windows_qlen2_then_single(pkg, device):
    """Code predictor: step 0 attends a 2x2 causal window, step s attends [:s + 2] of a
    16-slot cache (continuous.py:37-40, predictor.py:19-24); batch 64."""
    k, v = _arena(64, 16, torch.bfloat16, device, 31)
    gen = torch.Generator().manual_seed(32)
    for step in range(15):
        qlen = 2 if step == 0 else 1
        q = torch.randn(64, qlen, HQ, D, generator=gen).bfloat16().to(device)
        positions = torch.full((64,), step + 1, dtype=torch.int64, device=device)
        out = pkg.decode_attention(q, k, v, positions)
        expected = oatt.decode_attention(f64(q), f64(k), f64(v), positions.cpu().numpy(), D ** -0.5)
        assert_attention_close(f64(out), expected)
    # the reference's explicit 2x2 mask (finfo.min above the diagonal) gives the same result
    q = torch.randn(64, 2, HQ, D, generator=gen).bfloat16().to(device)
    mask = torch.zeros(1, 1, 2, 2, dtype=torch.bfloat16)
    mask[..., 0, 1] = torch.finfo(torch.bfloat16).min
    positions = torch.ones(64, dtype=torch.int64, device=device)
    with_mask = pkg.decode_attention(q, k[:, :, :2], v[:, :, :2], positions, mask=mask.to(device))
    implicit = pkg.decode_attention(q, k[:, :, :2], v[:, :, :2], positions)
    assert torch.equal(with_mask, implicit)


def test_invalid_positions_write_nothing_and_output_zero(pkg, device):
    batch, capacity = 4, 64
    k, v = _arena(batch, capacity, torch.bfloat16, device, 41)
    gen = torch.Generator().manual_seed(42)
    qkv = torch.randn(batch, 1, (HQ + 2 * HKV) * D, generator=gen).bfloat16().to(device)
    q = qkv[..., :HQ * D].view(batch, 1, HQ, D)
    kn = qkv[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D)
    vn = qkv[..., (HQ + HKV) * D:].view(batch, 1, HKV, D)
    positions = torch.tensor([5, 64, -1, 63], device=device)
    cos, sin = pkg.rope_tables(positions.clamp(min=0), D)
    before_k, before_v = k.clone(), v.clone()
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin)
    assert torch.equal(k[1:3], before_k[1:3]) and torch.equal(v[1:3], before_v[1:3])
    assert not out[1:3].any()
    assert out[0].abs().sum() > 0 and out[3].abs().sum() > 0


def test_graph_replay_with_changing_positions(pkg, device):
    """A captured fused step replayed while positions advance and inputs change in place
    (the SlotGraph.run pattern, continuous.py:218-224): every replay matches the oracle."""
    contexts, k, v, q, kn, vn = _config2(device, seed=7)
    qkv = q.as_strided((64, 1, (HQ + 2 * HKV) * D), (q.stride(0), q.stride(1), 1))
    positions = contexts.to(device).clone()
    cos, sin = pkg.rope_tables(positions, D)
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin)  # eager: sizes the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin)
    gen = torch.Generator().manual_seed(8)
    host_pos = contexts.clone()
    for replay in range(3):
        host_pos += 1
        positions.copy_(host_pos.to(device))
        c2, s2 = pkg.rope_tables(positions, D)
        cos.copy_(c2)
        sin.copy_(s2)
        qkv.copy_(torch.randn(qkv.shape, generator=gen).bfloat16().to(device))
        before_k, before_v = k.clone(), v.clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ek, ev, expected = _expected_fused(host_pos, before_k, before_v, q, kn, vn, cos, sin)
        assert np.array_equal(bits(k), ek) and np.array_equal(bits(v), ev)
        assert_attention_close(f64(out)[:, 0], expected[:, 0])


def test_attention_dropin_signature_and_errors(pkg, device):
    """npu_attention.attention's contract (npu_attention.py:11-26): BNSD in, BSND out,
    ValueError for training, dropout and sliding windows."""
    class Module:
        training = False
        sliding_window = None

    k, v = _arena(4, 64, torch.bfloat16, device, 51)
    gen = torch.Generator().manual_seed(52)
    q = torch.randn(4, HQ, 1, D, generator=gen).bfloat16().to(device)
    positions = torch.tensor([3, 10, 63, 0])
    allowed = torch.arange(64)[None, :] <= positions[:, None]
    mask = torch.where(allowed, 0.0, torch.finfo(torch.bfloat16).min).bfloat16()[:, None, None, :]
    out, weights = pkg.attention(Module(), q, k, v, mask.to(device), dropout=0.0, scaling=D ** -0.5,
                                 sliding_window=None)
    assert weights is None and out.shape == (4, 1, HQ, D) and out.is_contiguous()
    expected = oatt.decode_attention(f64(q.transpose(1, 2)), f64(k), f64(v), positions.numpy(), D ** -0.5)
    assert_attention_close(f64(out), expected)
    module = Module()
    module.training = True
    with pytest.raises(ValueError):
        pkg.attention(module, q, k, v, None)
    with pytest.raises(ValueError):
        pkg.attention(Module(), q, k, v, None, dropout=0.1)
    module = Module()
    module.sliding_window = 128
    with pytest.raises(ValueError):
        pkg.attention(module, q, k, v, None)


@pytest.mark.parametrize("batch,length", [(64, 64), (64, 256), (8, 512), (1, 128)])
def test_valid_length_dropin_with_poisoned_tail_and_replays(pkg, device, batch, length):
    """tools/probe_attention_context.py:20-60: 16/8 heads over a 512-row arena, positions
    (7 b) mod L, the mask over all 512 keys, with and without actual_seq_lengths_kv = [L]*B.
    Rows from L on are poisoned before every replay of the captured valid-length call; each
    replay must equal the same call made eagerly bit for bit, the eager full-mask call
    within the probe's own bar (assert_close atol = rtol = 0.02, :56; the two forms may
    split the keys differently, so their sums run in different orders), and the oracle."""
    class Module:
        training = False
        sliding_window = None

    gen = torch.Generator(device=device).manual_seed(60 + length)
    q = torch.randn(batch, HQ, 1, D, generator=gen, device=device, dtype=torch.bfloat16)
    k = torch.randn(batch, HKV, 512, D, generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    positions = (torch.arange(batch) * 7) % length
    allowed = torch.arange(512)[None, :] <= positions[:, None]
    mask = allowed[:, None, None, :].to(device)
    lengths = [length] * batch

    def valid():
        return pkg.attention(Module(), q, k, v, mask, scaling=D ** -0.5, actual_seq_lengths_kv=lengths)[0]

    expected = oatt.decode_attention(f64(q.transpose(1, 2)), f64(k), f64(v), positions.numpy(), D ** -0.5)
    assert_attention_close(f64(valid()), expected)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = valid()
    for replay in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device=device, dtype=torch.bfloat16))
        k[:, :, length:].fill_(100 * (replay + 1))
        v[:, :, length:].fill_(-100 * (replay + 1))
        graph.replay()
        eager = valid()
        full = pkg.attention(Module(), q, k, v, mask, scaling=D ** -0.5)[0]
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        torch.testing.assert_close(captured, full, atol=0.02, rtol=0.02)
    expected = oatt.decode_attention(f64(q.transpose(1, 2)), f64(k), f64(v), positions.numpy(), D ** -0.5)
    assert_attention_close(f64(captured), expected)


@pytest.mark.parametrize("batch,qlen,kvlen", [(1, 2, 2), (1, 1, 16), (4, 1, 512), (32, 1, 512)])
def test_mask_rewritten_between_replays_is_seen(pkg, device, batch, qlen, kvlen):
    """tools/probe_gqa_operator.py:31-58: one captured attention call with a boolean mask;
    before each replay the queries are redrawn and the mask is rewritten in place (a
    different key hidden from query 0), so frozen arguments would show."""
    class Module:
        training = False
        sliding_window = None

    gen = torch.Generator(device=device).manual_seed(80 + kvlen)
    q = torch.randn(batch, HQ, qlen, D, generator=gen, device=device, dtype=torch.bfloat16)
    k = torch.randn(batch, HKV, kvlen, D, generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    keep = torch.ones(batch, 1, qlen, kvlen, device=device, dtype=torch.bool)
    keep[..., 0, -1] = False

    def call():
        return pkg.attention(Module(), q, k, v, keep, scaling=D ** -0.5)[0]

    call()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = call()
    for replay in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device=device, dtype=torch.bfloat16))
        keep.fill_(True)
        keep[..., 0, -(replay % kvlen + 1)] = False
        graph.replay()
        eager = call()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        expected = oatt.decode_attention(f64(q.transpose(1, 2)), f64(k), f64(v), np.full(batch, kvlen - 1),
                                         D ** -0.5, mask=keep[:, 0].cpu().numpy())
        assert_attention_close(f64(captured), expected)


@pytest.mark.parametrize("length", [2, 3, 8, 16])
def test_predictor_padded_cache_equals_sliced(pkg, device, length):
    """tools/probe_predictor_padded_kv.py:20-60: head_dim 64 in a 16-row cache, two queries
    under the first step's mask at length 2 (query 0 sees key 0 only), one query otherwise;
    the padded call (actual_seq_lengths_kv, poisoned rows past the length) equals the call
    on the sliced cache, and both the oracle."""
    class Module:
        training = False
        sliding_window = None

    batch, head_dim = 64, 64
    qlen = 2 if length == 2 else 1
    gen = torch.Generator(device=device).manual_seed(70 + length)
    q = torch.randn(batch, HQ, qlen, head_dim, generator=gen, device=device, dtype=torch.bfloat16)
    k = torch.randn(batch, HKV, 16, head_dim, generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    k[:, :, length:].fill_(100)
    v[:, :, length:].fill_(-100)
    keep = torch.ones(1, 1, qlen, 16, dtype=torch.bool)
    if qlen == 2:
        keep[..., 0, 1:] = False
    keep = keep.to(device)
    scale = head_dim ** -0.5
    padded = pkg.attention(Module(), q, k, v, keep, scaling=scale, actual_seq_lengths_kv=[length] * batch)[0]
    sliced = pkg.attention(Module(), q, k[:, :, :length].contiguous(), v[:, :, :length].contiguous(),
                           keep[..., :length].contiguous(), scaling=scale)[0]
    torch.cuda.synchronize()
    assert torch.equal(padded, sliced)
    allowed = keep[0, 0, :, :length].cpu().numpy()[None].repeat(batch, 0)
    expected = oatt.decode_attention(f64(q.transpose(1, 2)), f64(k[:, :, :length]), f64(v[:, :, :length]),
                                     np.full(batch, length - 1), scale, mask=allowed)
    assert_attention_close(f64(padded), expected)


@pytest.mark.parametrize("kv_heads,splits,max_chunks", [(8, 0, 0), (4, -1, 5), (8, -1, 2), (4, 0, 0),
                                                      (8, 77, 0), (4, 1000, 0)])
def test_split_merge_is_deterministic_across_launches(pkg, device, kv_heads, splits, max_chunks):
    """Partial states cross workgroups (and, with 4 KV heads, XCDs) through the workspace;
    the merge runs in a fixed part order whichever part arrives last, so repeated launches
    are bit-identical and match the oracle."""
    gen = torch.Generator().manual_seed(60 + kv_heads)
    contexts = torch.randint(64, 1025, (64,), generator=gen)
    k, v = _arena(64, 1024, torch.bfloat16, device, 61, kv_heads=kv_heads)
    q = torch.randn(64, 1, kv_heads * 2, D, generator=gen).bfloat16().to(device)
    positions = contexts.to(device)
    first = pkg.decode_attention(q, k, v, positions, max_chunks=max_chunks, splits=splits).clone()
    for _ in range(20):
        again = pkg.decode_attention(q, k, v, positions, max_chunks=max_chunks, splits=splits)
        assert torch.equal(again, first)
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), contexts.numpy(), D ** -0.5)
    assert_attention_close(f64(first), expected)


def test_maximum_batch(pkg, device):
    """1024 requests (the largest batch), short contexts including position 0."""
    batch, capacity = 1024, 64
    gen = torch.Generator().manual_seed(70)
    contexts = torch.randint(0, capacity, (batch,), generator=gen)
    contexts[:3] = torch.tensor([0, 1, capacity - 1])
    k, v = _arena(batch, capacity, torch.bfloat16, device, 71)
    q = torch.randn(batch, 1, HQ, D, generator=gen).bfloat16().to(device)
    out = pkg.decode_attention(q, k, v, contexts.to(device))
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), contexts.numpy(), D ** -0.5)
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("splits,max_chunks", [(0, 0), (-1, 3), (3, 0), (50, 0)])
def test_long_context_multi_block_chunks(pkg, device, splits, max_chunks):
    """An 8192-key arena: with max_chunks 3 every chunk spans many 64-key blocks; with 3
    balanced workgroups per head every share spans several requests (one of them at
    position 0)."""
    capacity = 8192
    contexts = torch.tensor([8191, 3000, 64, 0])
    k, v = _arena(4, capacity, torch.bfloat16, device, 72)
    gen = torch.Generator().manual_seed(73)
    q = torch.randn(4, 1, HQ, D, generator=gen).bfloat16().to(device)
    out = pkg.decode_attention(q, k, v, contexts.to(device), max_chunks=max_chunks, splits=splits)
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), contexts.numpy(), D ** -0.5)
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("grid", [None, "bundled"])
def test_kv_offsets_address_any_layout(pkg, device, grid):
    """kv_offsets place each request's rows at an arbitrary element offset of one buffer
    (a request's keys at offset_b + h * stride_h + j * stride_t)."""
    batch, capacity = 6, 96
    gen = torch.Generator().manual_seed(74)
    flat_k = torch.randn(10 * HKV * capacity * D, generator=gen).bfloat16().to(device)
    flat_v = torch.randn(10 * HKV * capacity * D, generator=gen).bfloat16().to(device)
    slots = torch.tensor([9, 2, 5, 0, 7, 3])
    plane = HKV * capacity * D
    offsets = (slots * plane).to(device)
    keys = flat_k.view(10, HKV, capacity, D)
    values = flat_v.view(10, HKV, capacity, D)
    contexts = torch.tensor([95, 10, 40, 0, 63, 77])
    q = torch.randn(batch, 1, HQ, D, generator=gen).bfloat16().to(device)
    out = pkg.decode_attention(q, keys[:batch], values[:batch], contexts.to(device), kv_offsets=offsets, grid=grid)
    expected = oatt.decode_attention(f64(q), f64(keys[slots]), f64(values[slots]), contexts.numpy(), D ** -0.5)
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("grid", [None, "bundled"])
def test_fused_step_at_position_zero(pkg, device, grid):
    """A request at position 0 attends only its own new key: the output is the new value."""
    batch, capacity = 3, 32
    k, v = _arena(batch, capacity, torch.bfloat16, device, 75)
    gen = torch.Generator().manual_seed(76)
    qkv = torch.randn(batch, 1, (HQ + 2 * HKV) * D, generator=gen).bfloat16().to(device)
    q = qkv[..., :HQ * D].view(batch, 1, HQ, D)
    kn = qkv[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D)
    vn = qkv[..., (HQ + HKV) * D:].view(batch, 1, HKV, D)
    positions = torch.zeros(batch, dtype=torch.int64, device=device)
    cos, sin = pkg.rope_tables(positions, D)
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin, grid=grid)
    expected = vn.float().repeat_interleave(HQ // HKV, dim=2)
    assert torch.allclose(out.float(), expected, atol=1e-2, rtol=1e-2)
    assert torch.equal(v[:, :, 0], vn[:, 0])
