"""Padded prefill with explicit masks and per-row key counts, and the PrefillGraph flow.

Kernel level: the MFMA prefill with a mask (every key scored, the mask added to the scores)
and with kv_lens (causal over each row's first kv_lens keys) against the float64 oracle, on
every query row the mask defines, padding rows included.  The masks are PrefillGraph's
key-valid and causal form (prefill_graph.py:36-37: 0 where allowed, finfo.min elsewhere),
bool and fp32 variants, a broadcast mask and a sliding-window mask that is not causal-shaped.

Flow level: a stand-in talker (tests/_talker.py) with PackedAttention swapped in runs the
reference's padded prefill two ways: the reference's own flow (the additive mask and a
DynamicCache through PackedAttention's generic path: rotary, cache update, masked attention)
and this package's PrefillGraph (the packed cache written by the prologue kernel, row lengths
instead of a mask), captured and replayed on changing masks.  Both are compared with a CPU
float32 restatement of the same layers (torch ops and SDPA under the mask), on the valid rows."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from tests._talker import Talker
from tests._util import assert_attention_close, f64

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


def _padded_mask(lengths, padded, dtype):
    """(B, 1, Lp, Lp): key j visible to query i iff j < n_b and j <= i (prefill_graph.py:36-37)."""
    valid = torch.arange(padded)[None, :] < torch.tensor(lengths)[:, None]
    allowed = valid[:, None, :] & (torch.arange(padded)[None, :] <= torch.arange(padded)[:, None])[None]
    if dtype == torch.bool:
        return allowed[:, None]
    return torch.where(allowed, 0.0, torch.finfo(dtype).min).to(dtype)[:, None]


def _rows(batch, length, seed, device):
    gen = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(batch * length, HQ, D, generator=gen, device=device, dtype=torch.bfloat16)
    k = torch.randn(batch, HKV, length, D, generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    return q, k, v


def _expected(q, k, v, mask_bool, batch, queries):
    """Oracle: every query row under the bool mask (B, Lq, Lk)."""
    qb = f64(q).reshape(batch, queries, HQ, D)
    return oatt.decode_attention(qb, f64(k), f64(v), np.full(batch, k.shape[2] - 1), D ** -0.5,
                                 mask=mask_bool).reshape(batch * queries, HQ, D)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.bool])
def test_masked_prefill_padded_batch(pkg, device, dtype):
    lengths, padded = [128, 77, 1, 100], 128
    batch = len(lengths)
    q, k, v = _rows(batch, padded, 5, device)
    mask = _padded_mask(lengths, padded, dtype).to(device)
    cu = torch.arange(0, (batch + 1) * padded, padded, dtype=torch.int32, device=device)
    out = pkg.prefill_attention(q, k, v, cu, padded, mask=mask)
    expected = _expected(q, k, v, _padded_mask(lengths, padded, torch.bool)[:, 0].numpy(), batch, padded)
    assert_attention_close(f64(out), expected)


def test_key_counts_equal_the_padded_mask(pkg, device):
    """kv_lens gives PrefillGraph's key-valid and causal rule without a mask tensor: the same
    result as the masked kernel and the oracle, padding rows included."""
    lengths, padded = [256, 130, 64, 1, 255, 200, 17, 129], 256
    batch = len(lengths)
    q, k, v = _rows(batch, padded, 6, device)
    cu = torch.arange(0, (batch + 1) * padded, padded, dtype=torch.int32, device=device)
    kv_lens = torch.tensor(lengths, dtype=torch.int32, device=device)
    counted = pkg.prefill_attention(q, k, v, cu, padded, kv_lens=kv_lens)
    masked = pkg.prefill_attention(q, k, v, cu, padded, mask=_padded_mask(lengths, padded, torch.bfloat16).to(device))
    expected = _expected(q, k, v, _padded_mask(lengths, padded, torch.bool)[:, 0].numpy(), batch, padded)
    assert_attention_close(f64(counted), expected)
    assert_attention_close(f64(masked), expected)
    assert (counted.float() - masked.float()).abs().max().item() <= 2e-2


def test_masks_that_are_not_causal(pkg, device):
    """A broadcast (1, 1, Lq, Lk) fp16 sliding-window mask and more keys than queries: keys
    above the diagonal are scored when the mask allows them."""
    batch, queries, keys = 3, 96, 160
    gen = torch.Generator(device=device).manual_seed(7)
    q = torch.randn(batch * queries, HQ, D, generator=gen, device=device, dtype=torch.bfloat16)
    k = torch.randn(batch, HKV, keys, D, generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    i = torch.arange(queries)[:, None] + (keys - queries)
    j = torch.arange(keys)[None, :]
    window = (j <= i + 8) & (j > i - 40)                     # reaches 8 keys past the diagonal
    mask = torch.where(window, 0.0, float('-inf')).half()[None, None].to(device)
    cu = torch.arange(0, (batch + 1) * queries, queries, dtype=torch.int32, device=device)
    out = pkg.prefill_attention(q, k, v, cu, queries, mask=mask)
    expected = _expected(q, k, v, np.broadcast_to(window.numpy(), (batch, queries, keys)), batch, queries)
    assert_attention_close(f64(out), expected)


def test_attention_dropin_takes_the_prefill_mask(pkg, device):
    """npu_attention.attention's contract with several queries and an explicit mask (the call
    PrefillGraph.compute's layers make, prefill_graph.py:40-43): BNSD in, BSND out."""
    class Module:
        training, sliding_window, is_causal = False, None, True

    lengths, padded = [64, 33, 64, 5], 64
    batch = len(lengths)
    gen = torch.Generator(device=device).manual_seed(8)
    q = torch.randn(batch, padded, HQ, D, generator=gen, device=device, dtype=torch.bfloat16)
    k = torch.randn(batch, padded, HKV, D, generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    mask = _padded_mask(lengths, padded, torch.bfloat16).to(device)
    out, weights = pkg.attention(Module(), q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), mask,
                                 dropout=0.0, scaling=D ** -0.5, sliding_window=None)
    assert weights is None and out.shape == (batch, padded, HQ, D) and out.is_contiguous()
    expected = oatt.decode_attention(f64(q), f64(k.transpose(1, 2)), f64(v.transpose(1, 2)),
                                     np.full(batch, padded - 1), D ** -0.5,
                                     mask=_padded_mask(lengths, padded, torch.bool)[:, 0].numpy())
    assert_attention_close(f64(out), expected)


@pytest.mark.parametrize("with_mask", [False, True])
def test_attention_dropin_key_counts_at_any_query_length(pkg, device, with_mask):
    """The reference operator takes actual_seq_lengths_kv at every query length
    (npu_attention.py:20-24): with several queries the key counts bound every row, alone (the
    causal rule) or on top of a causal mask, which gives the padded batch's key-valid and
    causal mask (prefill_graph.py:36-37).  kv_positions, a decode bound, is refused there."""
    class Module:
        training, sliding_window, is_causal = False, None, True

    lengths, padded = [64, 33, 64, 5], 64
    batch = len(lengths)
    gen = torch.Generator(device=device).manual_seed(9)
    q = torch.randn(batch, padded, HQ, D, generator=gen, device=device, dtype=torch.bfloat16)
    k = torch.randn(batch, padded, HKV, D, generator=gen, device=device, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    mask = None
    if with_mask:  # causal only: the key counts come from actual_seq_lengths_kv
        mask = _padded_mask([padded] * batch, padded, torch.bfloat16).to(device)
    out, _ = pkg.attention(Module(), q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), mask,
                           scaling=D ** -0.5, actual_seq_lengths_kv=lengths)
    expected = oatt.decode_attention(f64(q), f64(k.transpose(1, 2)), f64(v.transpose(1, 2)),
                                     np.full(batch, padded - 1), D ** -0.5,
                                     mask=_padded_mask(lengths, padded, torch.bool)[:, 0].numpy())
    assert_attention_close(f64(out), expected)
    with pytest.raises(ValueError):
        pkg.attention(Module(), q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), mask,
                      kv_positions=torch.full((batch,), padded - 1, device=device))


# ---- the PrefillGraph flow on a stand-in talker --------------------------------------------

class _TalkerWithHead(torch.nn.Module):
    """talker.model (layers, rotary_emb, norm) and talker.codec_head, as PrefillGraph reads."""

    def __init__(self, layers, hidden, vocab=64):
        super().__init__()
        self.model = Talker(layers=layers, hidden=hidden, seed=3)
        self.config = type('C', (), {'hidden_size': hidden})()
        gen = torch.Generator().manual_seed(4)
        self.codec_head = torch.nn.Linear(hidden, vocab, bias=False, dtype=torch.bfloat16)
        with torch.no_grad():
            self.codec_head.weight.copy_((torch.randn(vocab, hidden, generator=gen) * hidden ** -0.5).bfloat16())


def _cpu_flow(talker_cpu, embeddings, mask):
    """The reference's padded prefill (prefill_graph.py:31-46) restated on the CPU in float32:
    positions cumsum(mask) - 1 (padding at 1), the key-valid and causal additive mask, each
    layer as input norm, projections, q/k norms, rotate-half RoPE, SDPA with KV heads repeated,
    o_proj and the residual; the final norm at each row's last valid token."""
    model = talker_cpu.model
    x = embeddings.float()
    batch, length, _ = x.shape
    ids = (mask.cumsum(-1) - 1).masked_fill(mask == 0, 1)
    cos, sin = model.rotary_emb(x, ids)
    cos, sin = cos.float()[:, None], sin.float()[:, None]
    allowed = mask[:, None, :].bool() & (torch.arange(length)[None, :] <= torch.arange(length)[:, None])[None]
    additive = torch.where(allowed, 0.0, float('-inf'))[:, None]

    def rope(t):
        half = t.shape[-1] // 2
        return t * cos + torch.cat((-t[..., half:], t[..., :half]), -1) * sin

    def norm(module, t):
        return module.weight.float() * (t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + module.eps))

    for layer in model.layers:
        attn = getattr(layer.self_attn, 'reference', layer.self_attn)
        h = norm(layer.input_layernorm, x)
        q = (h @ attn.q_proj.weight.float().T).view(batch, length, -1, D)
        k = (h @ attn.k_proj.weight.float().T).view(batch, length, -1, D)
        v = (h @ attn.v_proj.weight.float().T).view(batch, length, -1, D).transpose(1, 2)
        q = rope(norm(attn.q_norm, q).transpose(1, 2))
        k = rope(norm(attn.k_norm, k).transpose(1, 2))
        k = k.repeat_interleave(q.shape[1] // k.shape[1], 1)
        v = v.repeat_interleave(q.shape[1] // v.shape[1], 1)
        o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=additive, scale=attn.scaling)
        x = x + o.transpose(1, 2).reshape(batch, length, -1) @ attn.o_proj.weight.float().T
    rows = torch.arange(batch)
    return norm(model.norm, x)[rows, mask.sum(-1) - 1]


def test_prefill_graph_flow(pkg, device):
    from transformers.cache_utils import DynamicCache
    layers, hidden, padded = 2, 512, 128
    talker_cpu = _TalkerWithHead(layers, hidden).eval()
    talker = _TalkerWithHead(layers, hidden).to(device).eval()
    pkg.install_packed_attention(talker.model, native_gqa=True, text_only_rope=True)
    graph = pkg.PrefillGraph(talker, 4, padded, packed_kv=True)
    graph.capture()
    gen = torch.Generator().manual_seed(11)
    arena = pkg.SlotArena(talker.model, 8, 256, packed_kv=True)
    for replay, lengths in enumerate(([128, 77, 3], [64, 128, 1], [90, 91, 92])):
        embeddings = (torch.randn(3, padded, hidden, generator=gen) * 0.5).bfloat16()
        mask = (torch.arange(padded)[None, :] < torch.tensor(lengths)[:, None]).long()
        embeddings, mask = pkg.pad_prefill_batch(embeddings, mask, 4)
        hidden_out, logits, cache = graph.run(embeddings.to(device), mask.to(device))
        # the captured replay equals the eager forward of the same inputs
        eager_hidden, eager_logits, _ = graph.compute()
        torch.cuda.synchronize()
        assert torch.equal(hidden_out, eager_hidden) and torch.equal(logits, eager_logits), replay
        # the reference's own flow: additive mask and DynamicCache through PackedAttention
        dmask = mask.to(device)
        ids = (dmask.cumsum(-1) - 1).masked_fill(dmask == 0, 1)
        rotary = talker.model.rotary_emb(embeddings.to(device), ids[None].expand(3, -1, -1))
        allowed = dmask[:, None, :].bool() & (torch.arange(padded, device=device)[None, :]
                                              <= torch.arange(padded, device=device)[:, None])[None]
        additive = torch.where(allowed, 0.0, torch.finfo(torch.bfloat16).min).bfloat16()[:, None]
        dyn = DynamicCache()
        x = embeddings.to(device)
        for layer in talker.model.layers:
            x = layer(x, attention_mask=additive, position_ids=ids, past_key_values=dyn,
                      cache_position=torch.arange(padded, device=device), position_embeddings=rotary)[0]
        reference_hidden = talker.model.norm(x)[torch.arange(4, device=device), dmask.sum(-1) - 1]
        expected = _cpu_flow(talker_cpu, embeddings, mask)
        valid = slice(0, 3)  # the fourth row is pad_prefill_batch's dummy prompt
        # against the float32 CPU restatement: the bar of bf16 activations through two layers
        # (values of unit size after the final norm, several bf16 roundings: ~1% mean)
        for got in (hidden_out[:, 0], reference_hidden):
            err = (got[valid].float().cpu() - expected[valid]).abs()
            assert err.max().item() <= 8e-2 and err.mean().item() <= 1e-2, (replay, err.max().item())
        # the two GPU flows round at the same points and differ only in the attention kernel
        # (row lengths against the mask tensor): close to the attention bar
        err = (hidden_out[valid, 0].float() - reference_hidden[valid].float()).abs()
        assert err.max().item() <= 3e-2 and err.mean().item() <= 3e-3, (replay, err.max().item())
        # layer 0's keys and values are the same arithmetic in both flows (projections, norms,
        # exact RoPE): bit-identical on the valid rows
        for b, n in enumerate(lengths):
            assert torch.equal(cache.layers[0].keys[b, :, :n], dyn.layers[0].keys[b, :, :n])
            assert torch.equal(cache.layers[0].values[b, :, :n], dyn.layers[0].values[b, :, :n])
        # admission copies each prompt's rows into its arena slot bit for bit
        for b, n in enumerate(lengths):
            arena.load_packed(b, graph.packed_cache, row=b, length=n)
        torch.cuda.synchronize()
        for b, n in enumerate(lengths):
            assert torch.equal(arena.packed[:, b, :, :n], graph.packed_cache[:, b, :, :n])
    graph.close()


def test_bad_outputs_and_arenas_raise_before_any_launch(pkg, device):
    """A caller-supplied ``out`` of the wrong shape or dtype, or without unit-stride rows, or
    an arena with fewer slots than requests, raises ValueError and leaves every buffer
    untouched (strided outputs with unit-stride rows are accepted)."""
    batch = 4
    q = torch.zeros(batch, 1, HQ, D, device=device, dtype=torch.bfloat16)
    kn = torch.zeros(batch, 1, HKV, D, device=device, dtype=torch.bfloat16)
    arena = torch.zeros(batch, HKV, 64, D, device=device, dtype=torch.bfloat16)
    pos = torch.full((batch,), 5, device=device, dtype=torch.int64)
    cos, sin = pkg.rope_tables(pos, D)
    for bad in (torch.full((batch, 1, HQ, 2 * D), 3.0, device=device, dtype=torch.bfloat16)[..., ::2],
                torch.full((batch, 1, HQ, D), 3.0, device=device, dtype=torch.float32),
                torch.full((batch - 1, 1, HQ, D), 3.0, device=device, dtype=torch.bfloat16)):
        with pytest.raises(ValueError):
            pkg.decode_step(q, kn, kn, arena, arena.clone(), pos, cos, sin, out=bad)
        with pytest.raises(ValueError):
            pkg.decode_attention(q, arena, arena, pos, out=bad)
        assert bool((bad == 3.0).all())
    tokens = 3 * 40
    qp = torch.zeros(tokens, HQ, D, device=device, dtype=torch.bfloat16)
    cu = torch.arange(0, 4 * 40, 40, dtype=torch.int32, device=device)
    small = torch.zeros(2, HKV, 64, D, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.prefill_attention(qp, small, small, cu, 40)           # 3 requests, 2 slots
    wide = torch.full((tokens, HQ, 2 * D), 3.0, device=device, dtype=torch.bfloat16)
    for bad in (wide[..., ::2], torch.full((tokens - 1, HQ, D), 3.0, device=device, dtype=torch.bfloat16)):
        with pytest.raises(ValueError):
            pkg.prefill_attention(qp, arena, arena, cu, 40, out=bad)
    assert bool((wide == 3.0).all())
    with pytest.raises(ValueError):
        pkg.prefill_attention(qp, arena, arena, cu, 40, kv_lens=torch.zeros(3, device=device, dtype=torch.int64))
    with pytest.raises(ValueError):
        pkg.prefill_attention(qp, arena, arena, cu, 40, mask=torch.zeros(3, 1, 40, 63, device=device))
