"""The package's HIP path against the committed golden fixtures (tests/golden/).

The inputs are re-created from their seeds on the CPU and copied to the GPU; the RoPE tables
are the fixtures' own rows, so RoPE and the K/V write must match bit for bit; attention is
held to max-abs 2e-2 / mean-abs 2e-3 for bf16 I/O and 1e-5 for fp32 I/O."""
import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from tests._util import assert_attention_close, bits, f64, from_bits
from tests.golden import make_golden as mg

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_rope_golden(pkg, device):
    g = load("rope_bf16.npz")
    x = from_bits(mg.rope_input(), device)
    cos, sin = from_bits(g["cos"], device)[:, None], from_bits(g["sin"], device)[:, None]
    assert np.array_equal(bits(pkg.rotary(x, cos, sin)), g["y"])
    # device tables: within one bf16 step of the golden rows
    dcos, dsin = pkg.rope_tables(torch.from_numpy(g["positions"]).to(device), mg.D)
    for got, want in ((bits(dcos), g["cos"]), (bits(dsin), g["sin"])):
        assert np.abs(got.astype(np.int32) - want.astype(np.int32)).max() <= 1


def test_config1_golden(pkg, device):
    g = load("config1_fp32.npz")
    cache_k, cache_v, q, k, v = mg.config1_inputs()
    positions = torch.from_numpy(g["contexts"]).to(device)
    cos, sin = torch.from_numpy(g["cos"]).to(device), torch.from_numpy(g["sin"]).to(device)
    q_rot = pkg.rotary(q.to(device), cos, sin)
    k_rot = pkg.rotary(k.to(device), cos, sin)
    assert np.array_equal(q_rot.cpu().numpy().view(np.uint32), g["q_rot"].view(np.uint32))
    assert np.array_equal(k_rot.cpu().numpy().view(np.uint32), g["k_rot"].view(np.uint32))
    dk, dv = cache_k.to(device), cache_v.to(device)
    pkg.write(k_rot.transpose(1, 2), v.to(device).transpose(1, 2), dk, dv, positions)
    for b, c in enumerate(g["contexts"]):
        assert torch.equal(dk[b, :, c].cpu(), torch.from_numpy(g["k_rot"][b, 0]))
    out = pkg.decode_attention(q_rot, dk, dv, positions)
    np.testing.assert_allclose(f64(out), g["out"], atol=1e-5, rtol=0)


@pytest.mark.parametrize("splits,max_chunks", [(0, 0), (-1, 4), (300, 0)])
def test_config2_golden_fused_step(pkg, device, splits, max_chunks):
    g = load("config2_talker64.npz")
    contexts, keys, values, qkv = mg.config2_inputs()
    assert np.array_equal(contexts.numpy(), g["contexts"])
    dk, dv, dqkv = keys.to(device), values.to(device), qkv.to(device)
    del keys, values
    q, k, v = mg.split_qkv(dqkv)
    positions = contexts.to(device)
    cos, sin = from_bits(g["cos"], device), from_bits(g["sin"], device)
    out = pkg.decode_step(q, k, v, dk, dv, positions, cos, sin, max_chunks=max_chunks, splits=splits)
    torch.cuda.synchronize()
    assert hashlib.sha256(bits(dk).tobytes()).hexdigest() == str(g["keys_sha256"])
    assert hashlib.sha256(bits(dv).tobytes()).hexdigest() == str(g["values_sha256"])
    selected = torch.from_numpy(g["selected"]).to(device)
    assert_attention_close(f64(out.index_select(0, selected)), g["out"].astype(np.float64))


def test_prefill_golden(pkg, device):
    """The 16-prompt prefill through prefill_step (keys/values prologue, attention rotating the
    raw queries): the arena bit-exact, each prompt's last-token output within the bf16 bar."""
    g = load("prefill16.npz")
    lengths, cu, positions, q, k, v = mg.prefill_inputs()
    assert np.array_equal(lengths, g["lengths"])
    cos_b, sin_b = mg.prefill_tables(positions)
    cos, sin = from_bits(cos_b, device), from_bits(sin_b, device)
    ak = torch.zeros(mg.PREFILL_SLOTS, mg.HKV, mg.PREFILL_CAPACITY, mg.D, device=device, dtype=torch.bfloat16)
    av = torch.zeros_like(ak)
    dcu = torch.from_numpy(cu).to(device)
    out = pkg.prefill_step(q.to(device), k.to(device), v.to(device), cos, sin, dcu, int(lengths.max()), ak, av)
    torch.cuda.synchronize()
    assert hashlib.sha256(bits(ak).tobytes()).hexdigest() == str(g["keys_sha256"])
    assert hashlib.sha256(bits(av).tobytes()).hexdigest() == str(g["values_sha256"])
    last = torch.from_numpy(g["last_tokens"]).to(device)
    assert_attention_close(f64(out.index_select(0, last)), g["out_last"].astype(np.float64))
