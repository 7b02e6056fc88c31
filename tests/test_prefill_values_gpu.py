"""Prefill with the values read from the projection's rows: the prologue writes only the
rotated keys (``prefill_rope_write(value=None)``) and the attention launch reads each key's
value from the step's own value rows while its copy workgroups write those rows into the
arena (``prefill_attention(new_values=...)``).

Every case is compared bit for bit with the two-launch path that writes keys and values in
the prologue and attends the arena: the attention outputs (the same bf16 operands reach the
same products) and both arena planes (the copy is a byte copy at the token's position, rows
past the capacity untouched).  That path is itself checked against the float64 oracle in
test_prefill_gpu.py; here the new path is also held to the oracle on one case."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import bf16 as obf16
from oracle import rope as orope
from tests._util import assert_attention_close, bits, f64

pytestmark = pytest.mark.gpu


def _case(lengths, q_heads, kv_heads, head_dim, slots, capacity, seed, device):
    gen = torch.Generator().manual_seed(seed)
    total = int(sum(lengths))
    qkv = torch.randn(total, q_heads + 2 * kv_heads, head_dim, generator=gen).bfloat16().to(device)
    q, k, v = qkv[:, :q_heads], qkv[:, q_heads:q_heads + kv_heads], qkv[:, q_heads + kv_heads:]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    positions = np.concatenate([np.arange(n) for n in lengths])
    c, s = orope.tables(positions, orope.inv_freq(head_dim))
    cos = torch.from_numpy(c.view(np.int16)).view(torch.bfloat16).to(device)
    sin = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16).to(device)
    dg = torch.Generator(device=device).manual_seed(seed + 1)
    ak = torch.randn(slots, kv_heads, capacity, head_dim, generator=dg, device=device, dtype=torch.bfloat16)
    av = torch.randn_like(ak)
    return q, k, v, cu.to(device), cos, sin, ak, av


def _both(pkg, lengths, q_heads, kv_heads, head_dim, slots, capacity, seed, device, kv_slots=None, kv_lens=None):
    q, k, v, cu, cos, sin, ak, av = _case(lengths, q_heads, kv_heads, head_dim, slots, capacity, seed, device)
    ak2, av2 = ak.clone(), av.clone()
    longest = max(lengths)
    pkg.prefill_rope_write(q, k, None, cos, sin, cu, ak, av, kv_slots=kv_slots, rotate_query=False)
    got = pkg.prefill_attention(q, ak, av, cu, longest, kv_slots=kv_slots, cos=cos, sin=sin, kv_lens=kv_lens,
                                new_values=v)
    pkg.prefill_rope_write(q, k, v, cos, sin, cu, ak2, av2, kv_slots=kv_slots, rotate_query=False)
    expected = pkg.prefill_attention(q, ak2, av2, cu, longest, kv_slots=kv_slots, cos=cos, sin=sin, kv_lens=kv_lens)
    torch.cuda.synchronize()
    assert torch.equal(ak, ak2), "rotated keys"
    assert torch.equal(av, av2), "value rows copied by the attention launch"
    assert torch.equal(got, expected), "attention over the projection's value rows"
    return q, k, v, cu, cos, sin, ak, av, got


def test_prefill_workload_with_values_from_the_projection(pkg, device):
    """The 16-prompt prefill workload (lengths randint(32, 513) under seed 0, 16/8 heads,
    head_dim 128) in a 20-slot arena through kv_slots; also against the oracle."""
    lengths = torch.randint(32, 513, (16,), generator=torch.Generator().manual_seed(0)).tolist()
    kv_slots = torch.randperm(20, generator=torch.Generator().manual_seed(2))[:16].to(device)
    q, k, v, cu, cos, sin, ak, av, got = _both(pkg, lengths, 16, 8, 128, 20, 512, 3, device, kv_slots=kv_slots)
    c, s = bits(cos), bits(sin)
    eq = orope.rope_bf16(bits(q), c[:, None, :], s[:, None, :])
    expected = oatt.prefill_attention(obf16.from_bits(eq), obf16.from_bits(bits(ak)), obf16.from_bits(bits(av)),
                                      cu.cpu().numpy(), 128 ** -0.5, slots=kv_slots.cpu().numpy())
    assert_attention_close(f64(got), expected)


@pytest.mark.parametrize("group", [1, 2, 4])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_values_past_the_capacity_are_not_copied(pkg, device, group, head_dim):
    """Requests longer than the arena's 100 rows: keys and values past row 99 are neither
    written nor attended, as on the arena path; tile-edge lengths and a one-token request."""
    lengths = [1, 15, 16, 17, 64, 65, 99, 100, 101, 200, 333]
    _both(pkg, lengths, 2 * group, 2, head_dim, len(lengths), 100, 11 + group, device)


def test_more_than_64_requests(pkg, device):
    """70 requests: the copy workgroups find a token's request by a search of the row
    offsets instead of one ballot."""
    lengths = (torch.arange(70) * 7 % 61 + 1).tolist()
    kv_slots = torch.randperm(80, generator=torch.Generator().manual_seed(5))[:70].to(device)
    _both(pkg, lengths, 16, 8, 128, 80, 64, 21, device, kv_slots=kv_slots)


def test_right_padded_rows_with_key_counts(pkg, device):
    """A right-padded batch (PrefillGraph's layout): every row's tokens are written, the
    queries see only the first kv_lens[b] keys."""
    lengths = [96] * 6
    kv_lens = torch.tensor([96, 1, 40, 64, 65, 0], dtype=torch.int32, device=device)
    _both(pkg, lengths, 16, 8, 128, 6, 96, 31, device, kv_lens=kv_lens)


def test_keys_only_prologue_leaves_the_values(pkg, device):
    q, k, v, cu, cos, sin, ak, av = _case([5, 70, 33], 4, 2, 128, 3, 80, 41, device)
    before = av.clone()
    ak2, av2 = ak.clone(), av.clone()
    pkg.prefill_rope_write(q, k, None, cos, sin, cu, ak, av, rotate_query=False)
    pkg.prefill_rope_write(q, k, v, cos, sin, cu, ak2, av2, rotate_query=False)
    torch.cuda.synchronize()
    assert torch.equal(av, before)
    assert torch.equal(ak, ak2)


def test_values_from_the_projection_refuse_a_mask(pkg, device):
    q, k, v, cu, cos, sin, ak, av = _case([5, 7], 4, 2, 128, 2, 16, 51, device)
    mask = torch.zeros(2, 1, 7, 16, device=device, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.prefill_attention(q, ak, av, cu, 7, cos=cos, sin=sin, mask=mask, new_values=v)
    with pytest.raises(ValueError):  # value rows of another shape
        pkg.prefill_attention(q, ak, av, cu, 7, cos=cos, sin=sin, new_values=v[:, :1])
