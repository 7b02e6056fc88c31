"""The code predictor's attention chain at its own size, captured as one graph: 64 requests,
5 layers, 15 steps over a 16-position cache (PredictorCache, predictor.py:9-27, driven by
continuous.py:32-88).  Step 0 takes the two first tokens at positions 0 and 1 under the
2x2 causal rule; step s >= 1 takes one token at position s + 1 and attends keys 0 ... s + 1.
Every layer-step is one fused launch (RoPE of the query and key rows, the paired write,
attention), the 75 launches recorded and replayed as the benchmark times them.

Against the oracle chain (per-token RoPE, the paired write, causal attention) run step by
step on the CPU: every arena row each step writes is bit-exact, and every step's attention of
every layer is within the bar for bf16 I/O with fp32 accumulation (max-abs <= 2e-2,
mean-abs <= 2e-3)."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import kv as okv
from oracle import rope as orope
from tests._util import assert_attention_close, bits

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128
LAYERS, STEPS, BATCH, CAP = 5, 15, 64, 16


def test_predictor_chain_of_75_launches_matches_the_oracle(pkg, device):
    gen = torch.Generator(device=device).manual_seed(17)
    arena = torch.zeros(2 * LAYERS, BATCH, HKV, CAP, D, device=device, dtype=torch.bfloat16)
    rows = torch.randn(STEPS, LAYERS, BATCH, 2, HQ + 2 * HKV, D, generator=gen, device=device,
                       dtype=torch.bfloat16)
    positions = [torch.full((BATCH,), max(s + 1, 1), device=device, dtype=torch.int64) for s in range(STEPS)]
    token_positions = [torch.arange(2, device=device).expand(BATCH, 2).contiguous()] + \
                      [positions[s][:, None] for s in range(1, STEPS)]
    tables = [pkg.rope_tables(token_positions[s], D) for s in range(STEPS)]
    out = torch.empty(STEPS, LAYERS, BATCH, 2, HQ, D, device=device, dtype=torch.bfloat16)

    def chain():
        for s in range(STEPS):
            tokens = 2 if s == 0 else 1
            for layer in range(LAYERS):
                r = rows[s, layer, :, :tokens]
                pkg.decode_step(r[:, :, :HQ], r[:, :, HQ:HQ + HKV], r[:, :, HQ + HKV:], arena[layer],
                                arena[LAYERS + layer], positions[s], *tables[s], out=out[s, layer, :, :tokens])

    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    graph.replay()
    torch.cuda.synchronize()

    k_arena = np.zeros((LAYERS, BATCH, HKV, CAP, D), np.uint16)
    v_arena = np.zeros_like(k_arena)
    for s in range(STEPS):
        tokens = 2 if s == 0 else 1
        pos = np.full(BATCH, max(s + 1, 1))
        cos, sin = tables[s]
        cb, sb = bits(cos)[:, :, None, :], bits(sin)[:, :, None, :]
        for layer in range(LAYERS):
            r = bits(rows[s, layer, :, :tokens])
            q_rot = orope.rope_bf16(r[:, :, :HQ], cb, sb)
            k_rot = orope.rope_bf16(r[:, :, HQ:HQ + HKV], cb, sb)
            k_arena[layer], v_arena[layer] = okv.kv_write(k_arena[layer], v_arena[layer], k_rot.transpose(0, 2, 1, 3),
                                                          r[:, :, HQ + HKV:].transpose(0, 2, 1, 3), pos - tokens + 1)
            expected = oatt.decode_attention(obf16.from_bits(q_rot), obf16.from_bits(k_arena[layer]),
                                             obf16.from_bits(v_arena[layer]), pos, D ** -0.5)
            got = out[s, layer, :, :tokens].float().cpu().numpy().astype(np.float64)
            assert_attention_close(got, expected)
    # every row a step wrote (rows 0 ... 15, one step each), every layer, keys and values
    assert np.array_equal(bits(arena[:LAYERS]), k_arena)
    assert np.array_equal(bits(arena[LAYERS:]), v_arena)
