"""The bundled grid's masked launches against the float64 oracle: whole requests per
workgroup, each stage's mask words loaded with its K/V rows and added to the scores of keys
0 ... pos[b] (bf16 masks on a branch-free path, bool, fp16 and fp32 masks on the general one).

The reference's masked talker flow is covered at full size: SlotGraph.compute builds the
(B, 1, 1, ctx) mask 0 / finfo.min for keys j <= pos[b] every step and hands it to every layer
(continuous.py:188-197), whose operator adds it to the scores (npu_attention.py:16-25).
Tolerance for bf16 I/O with fp32 accumulation: max-abs <= 2e-2 and mean-abs <= 2e-3."""
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


def _inputs(batch, capacity, contexts, seed, device, kv_heads=HKV, group=2):
    gen = torch.Generator().manual_seed(seed)
    dgen = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(batch, kv_heads, capacity, D, generator=dgen, device=device, dtype=torch.bfloat16)
    v = torch.randn(batch, kv_heads, capacity, D, generator=dgen, device=device, dtype=torch.bfloat16)
    width = (kv_heads * group + 2 * kv_heads) * D
    qkv = torch.randn(batch, 1, width, generator=gen).bfloat16().to(device)
    q = qkv[..., :kv_heads * group * D].view(batch, 1, kv_heads * group, D)
    kn = qkv[..., kv_heads * group * D:(kv_heads * group + kv_heads) * D].view(batch, 1, kv_heads, D)
    vn = qkv[..., (kv_heads * group + kv_heads) * D:].view(batch, 1, kv_heads, D)
    return k, v, q, kn, vn


def _fused_oracle(k, v, q, kn, vn, contexts, cos, sin, mask=None):
    cb, sb = bits(cos)[:, None, None, :], bits(sin)[:, None, None, :]
    q_rot = orope.rope_bf16(bits(q), cb, sb)
    k_rot = orope.rope_bf16(bits(kn), cb, sb)
    ak, av = okv.kv_write(bits(k).copy(), bits(v).copy(), k_rot.transpose(0, 2, 1, 3),
                          bits(vn).transpose(0, 2, 1, 3), contexts)
    out = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(ak), obf16.from_bits(av),
                                contexts, D ** -0.5, mask=mask)
    return ak, av, out


def _slot_graph_mask(positions, width, dtype=torch.bfloat16):
    """SlotGraph.compute's mask (continuous.py:191-192): 0 for j <= pos[b], finfo.min after."""
    allowed = torch.arange(width, device=positions.device)[None, :] <= positions[:, None]
    return torch.where(allowed, 0.0, torch.finfo(dtype).min).to(dtype)[:, None, None, :]


@pytest.mark.parametrize("seed", [0, 5])
def test_reference_masked_talker_step_runs_on_the_bundled_grid(pkg, device, seed):
    """64 requests over a 1024-row arena, contexts U[64, 1024]: the fused step with the
    reference's per-step mask over the whole arena, on the bundled grid (the automatic choice
    for the masked call), matches the oracle, with and without the step's plan; the arena rows
    are bit-exact."""
    assert pkg.decode_grid_for(64, 1, HQ, HKV, D, 1024, masked=True) == "bundled"
    gen = torch.Generator().manual_seed(seed)
    contexts = torch.randint(64, 1025, (64,), generator=gen)
    k, v, q, kn, vn = _inputs(64, 1024, contexts, 100 + seed, device)
    positions = contexts.to(device)
    cos, sin = pkg.rope_tables(positions, D)
    mask = _slot_graph_mask(positions, 1024)
    ek, ev, expected = _fused_oracle(k, v, q, kn, vn, contexts.numpy(), cos, sin)
    plan = pkg.decode_plan(positions, 1024, HQ, HKV)
    k0, v0 = bits(k).copy(), bits(v).copy()
    out = pkg.decode_step(q, kn, vn, k, v, positions, cos, sin, mask=mask, plan=plan)
    assert np.array_equal(bits(k), ek) and np.array_equal(bits(v), ev)
    assert_attention_close(f64(out)[:, 0], expected[:, 0])
    k2, v2 = from_bits(k0, device), from_bits(v0, device)
    unplanned = pkg.decode_step(q, kn, vn, k2, v2, positions, cos, sin, mask=mask)
    assert torch.equal(unplanned, out) and torch.equal(k2, k) and torch.equal(v2, v)


@pytest.mark.parametrize("kind", ["bool", "additive_bf16", "additive_f16", "additive_f32"])
@pytest.mark.parametrize("batch,group,capacity", [(64, 2, 1024), (128, 1, 1024), (96, 4, 1024), (64, 2, 1023),
                                                  (37, 1, 333)])
def test_arbitrary_masks_on_the_bundled_grid(pkg, device, kind, batch, group, capacity):
    """Any additive or bool mask with unit key stride is added to the scores of keys
    0 ... pos[b] (SDPA's semantics within the positions' range), including finite additive
    terms; odd mask rows (1023 and 333 keys) put a request's 2-byte terms at odd element
    offsets, so the two halves of a mask word serve different keys."""
    kv_heads = HKV if group < 4 else 4
    gen = torch.Generator().manual_seed(200 + batch + group)
    contexts = torch.randint(0, capacity, (batch,), generator=gen)
    k, v, q, _, _ = _inputs(batch, capacity, contexts, 300 + batch, device, kv_heads=kv_heads, group=group)
    allowed = torch.rand(batch, 1, capacity, generator=gen) < 0.7
    allowed[torch.arange(batch), 0, contexts] = True   # every row sees its own last key
    if kind == "bool":
        mask, omask = allowed, allowed.numpy()
    else:
        dtype = {"additive_bf16": torch.bfloat16, "additive_f16": torch.float16, "additive_f32": torch.float32}[kind]
        terms = (-4.0 * torch.rand(batch, 1, capacity, generator=gen)).to(dtype)
        mask = torch.where(allowed, terms, torch.tensor(torch.finfo(dtype).min, dtype=dtype))
        omask = mask.float().numpy()
    positions = contexts.to(device)
    plan = pkg.decode_plan(positions, capacity, kv_heads * group, kv_heads)
    out = pkg.decode_attention(q, k, v, positions, mask=mask[:, None].to(device), plan=plan, grid="bundled")
    expected = oatt.decode_attention(f64(q), f64(k), f64(v), contexts.numpy(), D ** -0.5, mask=omask)
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("masked", [False, True])
def test_graph_replays_replan_changed_positions(pkg, device, masked):
    """The talker step as a graph: the plan launch and three fused layers captured once, the
    positions (and, masked, SlotGraph.compute's mask) rewritten in place between replays
    (requests growing, one retiring to an invalid position); every replay matches the oracle
    and writes exactly the new rows."""
    batch, capacity, layers = 64, 1024, 3
    gen = torch.Generator().manual_seed(600)
    contexts = torch.randint(64, 900, (batch,), generator=gen)
    positions = contexts.to(device)
    dgen = torch.Generator(device=device).manual_seed(601)
    arena = torch.randn(2 * layers, batch, HKV, capacity, D, generator=dgen, device=device, dtype=torch.bfloat16)
    qkv = torch.randn(layers, batch, 1, (HQ + 2 * HKV) * D, generator=dgen, device=device, dtype=torch.bfloat16)
    cos = torch.empty(batch, D, device=device, dtype=torch.bfloat16)
    sin = torch.empty_like(cos)
    out = torch.empty(layers, batch, 1, HQ, D, device=device, dtype=torch.bfloat16)
    plan_buf = torch.empty(pkg.plan_shape(batch, HQ, HKV), device=device, dtype=torch.int32)
    mask = _slot_graph_mask(positions, capacity) if masked else None

    def step():
        plan = pkg.decode_plan(positions, capacity, HQ, HKV, out=plan_buf)
        for layer in range(layers):
            r = qkv[layer]
            pkg.decode_step(r[..., :HQ * D].view(batch, 1, HQ, D), r[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D),
                            r[..., (HQ + HKV) * D:].view(batch, 1, HKV, D), arena[layer], arena[layers + layer],
                            positions, cos, sin, out=out[layer], plan=plan, mask=mask)

    c, s = pkg.rope_tables(positions.clamp(0, capacity - 1), D)
    cos.copy_(c)
    sin.copy_(s)
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for replay in range(3):
        contexts = contexts + 1
        if replay == 2:
            contexts[7] = -1
        positions.copy_(contexts.to(device))
        if masked:
            mask.copy_(_slot_graph_mask(positions, capacity))
        c, s = pkg.rope_tables(positions.clamp(0, capacity - 1), D)
        cos.copy_(c)
        sin.copy_(s)
        before = bits(arena).copy()
        graph.replay()
        torch.cuda.synchronize()
        valid = (contexts >= 0).numpy()
        for layer in range(layers):
            r = qkv[layer]
            q, kn, vn = r[..., :HQ * D].view(batch, 1, HQ, D), r[..., HQ * D:(HQ + HKV) * D].view(batch, 1, HKV, D), \
                r[..., (HQ + HKV) * D:].view(batch, 1, HKV, D)
            ks, vs = from_bits(before[layer]), from_bits(before[layers + layer])
            idx = np.flatnonzero(valid)
            ek, ev, expected = _fused_oracle(ks[idx], vs[idx], q[idx], kn[idx], vn[idx], contexts.numpy()[idx],
                                             cos[idx], sin[idx])
            assert np.array_equal(bits(arena[layer])[idx], ek) and np.array_equal(bits(arena[layers + layer])[idx], ev)
            assert np.array_equal(bits(arena[layer])[~valid], before[layer][~valid])
            got = f64(out[layer])
            assert_attention_close(got[idx][:, 0], expected[:, 0])
            assert not got[~valid].any()
