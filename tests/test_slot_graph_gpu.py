"""SlotGraph: the talker decode step captured in one HIP graph through PackedAttention.

The graph (the contract of continuous.py:172-230 on HIP graphs) is checked three ways:

* against the same ``compute`` run eagerly on a twin arena: every replay's output and the
  whole arena after it bit-identical, over several steps with padded rows (positions 0 past
  the active count), with eager work on the stream between replays; capture leaves the arena
  as it was;
* against an oracle of the whole step on the CPU (the stand-in talker's layers in CPU bf16
  torch ops, exact RoPE, the scatter write and float64 attention rounded to bf16, i.e. the
  arithmetic PackedAttention.forward asks for at the same rounding points): the output to
  max-abs 3e-2 / mean-abs 3e-3 (GEMM accumulation order and fp32 against float64 attention
  are the only differences), the arena bit-exact against the write of every layer's own
  projected rows, and every layer's attention output (the input of its o_proj) within the
  attention bar (max-abs 2e-2, mean-abs 2e-3) of float64 attention over that layer's own
  projected query rows and the arena;
* the mask: not built when every attention layer is wrapped.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import kv as okv
from oracle import rope as orope
from tests._talker import Talker
from tests._util import assert_attention_close, bits
from tests.test_decode_gpu import plan_parts

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


def test_replays_match_eager_compute_and_capture_writes_nothing(pkg, device):
    slots, capacity, batch = 16, 192, 8
    model = _model(pkg, device)
    arena = _arena(pkg, model, slots, capacity, 4)
    twin_arena = pkg.SlotArena(model, slots, capacity, packed_kv=True)
    twin_arena.packed.copy_(arena.packed)
    graph = pkg.SlotGraph(arena, batch)
    graph.capture()
    torch.cuda.synchronize()
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


def _cpu_step(talker, arena, inputs, positions, rotary):
    """The decode step on the CPU: per layer the input norm, the fused QKV projection, the
    q/k norms (the stand-in's own modules, CPU bf16), exact bf16 RoPE, the paired write at the
    positions into ``arena`` (bf16 bits, updated in place), float64 attention over keys
    0 ... position rounded to bf16, o_proj and the residual; then the final norm."""
    x = inputs.cpu()
    batch = x.shape[0]
    cos, sin = talker.rotary_emb(x, rotary.cpu())
    cb, sb = bits(cos[0])[:, :, None, :], bits(sin[0])[:, :, None, :]
    layers = len(talker.layers)
    for index, layer in enumerate(talker.layers):
        attn = layer.self_attn
        h = layer.input_layernorm(x)
        weight = torch.cat([attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight])
        q, k, v = torch.nn.functional.linear(h, weight).split(
            [attn.q_proj.out_features, attn.k_proj.out_features, attn.v_proj.out_features], dim=-1)
        q = attn.q_norm(q.reshape(batch, 1, -1, attn.head_dim))
        k = attn.k_norm(k.reshape(batch, 1, -1, attn.head_dim))
        v = v.reshape(batch, 1, -1, attn.head_dim)
        q_rot, k_rot = orope.rope_bf16(bits(q), cb, sb), orope.rope_bf16(bits(k), cb, sb)
        okv.kv_write(arena[index], arena[layers + index], k_rot.transpose(0, 2, 1, 3),
                     bits(v).transpose(0, 2, 1, 3), positions)
        out = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(arena[index][:batch]),
                                    obf16.from_bits(arena[layers + index][:batch]), positions,
                                    attn.scaling)
        attended = torch.from_numpy(out).to(torch.bfloat16).reshape(batch, 1, -1)
        x = x + attn.o_proj(attended)
    return talker.norm(x)


@pytest.mark.parametrize("shape", ["small", "talker", "talker_reference_mask"])
def test_graph_step_matches_the_oracle(pkg, device, shape):
    """small: 12 requests over 16 slots of a 256-row arena, 3 layers (the chunked grid).
    talker: 64 slots of a 1024-row arena, 2 layers (the bundled grid, each step's plan made by
    SlotCache.prepare).  talker_reference_mask: the same step as the reference's
    SlotGraph.compute runs it, the (B, 1, 1, ctx) 0 / finfo.min mask built every step and
    handed to every layer (continuous.py:188-197): the masked bundled launch."""
    slots, capacity, batch, layers, counts = {"small": (16, 256, 12, 3, [12, 9]),
                                              "talker": (64, 1024, 64, 2, [64, 40]),
                                              "talker_reference_mask": (64, 1024, 64, 2, [64, 40])}[shape]
    hidden = 512
    model = _model(pkg, device, layers=layers, hidden=hidden)
    cpu_talker = Talker(layers=layers, hidden=hidden, seed=3).eval()
    arena = _arena(pkg, model, slots, capacity, 14)
    mirror = bits(arena.packed).copy()                        # the oracle's arena
    twin_arena = pkg.SlotArena(model, slots, capacity, packed_kv=True)
    graph = pkg.SlotGraph(arena, batch)
    assert graph._mask(torch.bfloat16) is None                 # every layer is wrapped
    reference_mask = shape == "talker_reference_mask"
    if shape != "small":
        assert pkg.decode_grid_for(batch, 1, 16, 8, 128, capacity, masked=reference_mask) == 'bundled'
    graph._needs_mask = reference_mask
    graph.capture()
    twin = pkg.SlotGraph(twin_arena, batch)
    twin._needs_mask = reference_mask
    gen = torch.Generator().manual_seed(15)
    for step, count in enumerate(counts):
        positions = torch.zeros(batch, dtype=torch.long)
        positions[:count] = torch.randint(1, capacity, (count,), generator=gen)
        inputs = torch.randn(batch, 1, hidden, generator=gen).bfloat16()
        rotary = positions.view(1, batch, 1).expand(3, batch, 1)
        # the arena each layer must leave: its own projected rows (recorded on an eager twin,
        # bit-identical to the replay) rotated and written by the oracle
        twin_arena.packed.copy_(arena.packed)
        expected_arena = bits(arena.packed).copy()
        recorded, attended = [], []
        hooks = [layer.self_attn.register_forward_hook(
            lambda module, args, kwargs, out: recorded.append((module, kwargs['hidden_states'])),
            with_kwargs=True) for layer in model.layers]
        hooks += [layer.self_attn.reference.o_proj.register_forward_hook(
            lambda module, args, out: attended.append(args[0].detach().clone())) for layer in model.layers]
        with torch.inference_mode():
            twin.inputs.copy_(inputs.to(device))
            twin.positions.copy_(positions.to(device))
            twin.rotary.copy_(rotary.to(device))
            twin.compute()
        for hook in hooks:
            hook.remove()
        cos, sin = model.rotary_emb(inputs.to(device), rotary.to(device))
        cb, sb = bits(cos[0])[:, :, None, :], bits(sin[0])[:, :, None, :]
        queries = []
        for index, (module, h) in enumerate(recorded):
            proj = torch.nn.functional.linear(h, module.weight, module.bias)
            q, k, v = proj.split(module.sizes, dim=-1)
            head_dim = module.reference.head_dim
            queries.append(orope.rope_bf16(bits(module.reference.q_norm(q.reshape(batch, 1, -1, head_dim))), cb, sb))
            k = module.reference.k_norm(k.reshape(batch, 1, -1, head_dim))
            k_rot = orope.rope_bf16(bits(k), cb, sb)
            okv.kv_write(expected_arena[index], expected_arena[layers + index], k_rot.transpose(0, 2, 1, 3),
                         bits(v.reshape(batch, 1, -1, head_dim)).transpose(0, 2, 1, 3),
                         positions.numpy())
        # each layer's attention on the eager twin (bit-identical to the replay) against float64
        # attention over its own rotated query rows and the arena it wrote
        assert len(attended) == layers
        for index, (module, _) in enumerate(recorded):
            head_dim = module.reference.head_dim
            expected_attn = oatt.decode_attention(
                obf16.from_bits(queries[index]), obf16.from_bits(expected_arena[index][:batch]),
                obf16.from_bits(expected_arena[layers + index][:batch]), positions.numpy(), module.reference.scaling)
            got = attended[index].float().cpu().numpy().astype(np.float64).reshape(expected_attn.shape)
            assert_attention_close(got, expected_attn)
        out = graph.run(inputs.to(device), positions.to(device), rotary.to(device))
        torch.cuda.synchronize()
        assert np.array_equal(bits(arena.packed), expected_arena), f"step {step}"
        expected = _cpu_step(cpu_talker, mirror, inputs, positions.numpy(), rotary)
        err = (out.float().cpu() - expected.float()).abs()
        # 3e-2 absolute, widened by half a bf16 step of the value (one step is 2^-5 = 0.031 at
        # magnitudes 4-8, where GEMM accumulation order alone moves an output by one step)
        bound = 3e-2 + expected.float().abs() * 2.0 ** -8
        assert bool((err <= bound).all()) and err.mean().item() <= 3e-3, (step, err.max().item(), err.mean().item())
        mirror = bits(arena.packed).copy()                    # next step starts from the device arena
    graph.close()


def test_mask_is_built_only_for_unwrapped_layers(pkg, device):
    model = Talker(layers=2, hidden=256, seed=3).to(device).eval()
    arena = pkg.SlotArena(model, 4, 64, packed_kv=True)
    graph = pkg.SlotGraph(arena, 4, context_length=48)
    graph.positions.copy_(torch.tensor([0, 5, 47, 10], device=device))
    mask = graph._mask(torch.bfloat16)
    assert mask.shape == (4, 1, 1, 48)
    allowed = torch.arange(48, device=device)[None, :] <= graph.positions[:, None]
    assert torch.equal(mask[:, 0, 0] == 0, allowed)
    assert bool((mask[:, 0, 0][~allowed] == torch.finfo(torch.bfloat16).min).all())


def test_talker_step_on_the_bundled_grid_reads_the_step_plan(pkg, device):
    """At the talker's shape (64 slots of a 1024-row arena, 8 KV heads of 128: the bundled
    grid) SlotCache.prepare plans the step once (decode_plan) and every layer's launch reads
    the plan's bundles of whole requests: replays equal an eager twin whose cache holds no
    plan (each launch ranks and pairs the requests itself), output and arena bit-identical,
    and the bundles list every request once with its length."""
    slots, capacity, batch = 64, 1024, 64
    model = _model(pkg, device, layers=2)
    arena = _arena(pkg, model, slots, capacity, 24)
    twin_arena = pkg.SlotArena(model, slots, capacity, packed_kv=True)
    twin_arena.packed.copy_(arena.packed)
    assert pkg.decode_grid_for(batch, 1, 16, 8, 128, capacity) == 'bundled'
    graph = pkg.SlotGraph(arena, batch)
    graph.capture()
    twin = pkg.SlotGraph(twin_arena, batch)
    twin.cache.prepare = lambda: None                        # no plan: in-launch ranking
    gen = torch.Generator().manual_seed(25)
    for step, count in enumerate([64, 40]):
        positions = torch.zeros(batch, dtype=torch.long)
        positions[:count] = torch.randint(0, capacity, (count,), generator=gen)
        inputs = torch.randn(batch, 1, model.config.hidden_size, generator=gen).bfloat16().to(device)
        rotary = positions.view(1, batch, 1).expand(3, batch, 1).to(device)
        out = graph.run(inputs, positions.to(device), rotary)
        with torch.inference_mode():
            twin.inputs.copy_(inputs)
            twin.positions.copy_(positions.to(device))
            twin.rotary.copy_(rotary)
            expected = twin.compute()
        torch.cuda.synchronize()
        assert twin.cache.plan is None and graph.cache.plan is not None
        lengths = positions.numpy() + 1
        table = plan_parts(graph.cache.plan)[1].cpu().numpy().reshape(-1, 2)
        listed = table[table[:, 0] >= 0]
        np.testing.assert_array_equal(np.sort(listed[:, 0]), np.arange(batch))
        np.testing.assert_array_equal(listed[:, 1], lengths[listed[:, 0]])
        assert np.array_equal(bits(out), bits(expected)), f"step {step}"
        assert np.array_equal(bits(arena.packed), bits(twin_arena.packed)), f"step {step}"
    graph.close()


@pytest.mark.parametrize("capacity,batch,planned", [(1024, 64, True), (512, 64, False), (512, 32, True),
                                                     (256, 32, False)])
def test_prepare_plans_only_for_the_bundled_grid(pkg, device, capacity, batch, planned):
    """SlotCache.prepare runs the plan kernel only when the step's launches take the bundled
    grid (64 requests from 1024 rows, 24..63 from 512 rows); otherwise the cache holds no
    plan and no plan kernel runs."""
    model = _model(pkg, device, layers=1)
    arena = pkg.SlotArena(model, batch, capacity, packed_kv=True)
    positions = torch.randint(0, capacity, (batch,), generator=torch.Generator().manual_seed(3)).to(device)
    cache = pkg.SlotCache(arena, positions)
    cache.prepare()
    assert (pkg.decode_grid_for(batch, 1, 16, 8, 128, capacity) == 'bundled') == planned
    assert (cache.plan is not None) == planned

