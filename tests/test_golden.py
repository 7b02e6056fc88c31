"""The committed golden fixtures (tests/golden/) on the CPU: the oracle still reproduces every
one of them, the fixtures agree with closed forms where one exists, and the package's host
scheduler reproduces the golden 128-slot trace record for record."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import bf16 as obf16
from tests.golden import make_golden as mg

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_rope_golden_reproduced_and_closed_forms():
    g = load("rope_bf16.npz")
    now = mg.expected_rope()
    for key in ("positions", "cos", "sin", "y"):
        assert np.array_equal(g[key], now[key]), key
    # position 0: cos 1, sin 0, so RoPE is the identity; |cos| and |sin| never exceed 1
    assert np.all(g["cos"][0] == 0x3F80) and np.all(g["sin"][0] == 0)
    assert np.array_equal(g["y"][0], mg.rope_input()[0])
    c, s = obf16.from_bits(g["cos"]), obf16.from_bits(g["sin"])
    assert np.all(np.abs(c) <= 1) and np.all(np.abs(s) <= 1)
    assert np.array_equal(g["cos"][:, :64], g["cos"][:, 64:])


def test_config1_golden_reproduced():
    g = load("config1_fp32.npz")
    now = mg.expected_config1()
    for key in ("contexts", "cos", "sin", "q_rot", "k_rot"):
        assert np.array_equal(g[key], now[key]), key
    np.testing.assert_allclose(g["out"], now["out"], atol=1e-12, rtol=0)
    # the attention output is a convex combination of value rows: inside their range
    assert np.all(np.abs(g["out"]) < 5)


def test_config2_golden_reproduced():
    g = load("config2_talker64.npz")
    now = mg.expected_config2()
    assert int(g["contexts"].sum()) == 32718
    for key in ("contexts", "cos", "sin", "selected"):
        assert np.array_equal(g[key], now[key]), key
    for key in ("keys_sha256", "values_sha256", "q_rot_sha256"):
        assert str(g[key]) == str(now[key]), key
    np.testing.assert_allclose(g["out"], now["out"], atol=1e-6, rtol=0)


def test_prefill_golden_reproduced():
    g = load("prefill16.npz")
    now = mg.expected_prefill()
    assert int(g["lengths"].sum()) == 4790
    for key in ("lengths", "last_tokens"):
        assert np.array_equal(g[key], now[key]), key
    for key in ("keys_sha256", "values_sha256"):
        assert str(g[key]) == str(now[key]), key
    np.testing.assert_allclose(g["out_last"], now["out_last"], atol=1e-6, rtol=0)


@pytest.mark.parametrize("run", range(len(mg.SCHEDULER_SETTINGS)))
def test_scheduler_golden_reproduced_by_oracle_and_package(pkg, run):
    from qwen3_tts_engine_amd.scheduler import SlotScheduler
    from tests.test_scheduler import _Adapter
    from oracle import scheduler as osched

    golden = json.loads((GOLDEN / "scheduler_trace.json").read_text())
    spec = golden["runs"][run]
    step, bucket_kv, rate = spec["decode_bucket_step"], spec["bucket_kv"], spec["cancel_rate"]
    trace = mg.scheduler_trace(rate)
    ref = mg.compact_records(osched.drive(osched.ReferenceScheduler(128, 512, step, bucket_kv), trace, 128))
    ours = mg.compact_records(osched.drive(_Adapter(SlotScheduler(128, 512, step, bucket_kv)), trace, 128))
    assert len(spec["iterations"]) == 200
    for i, (want, a, b) in enumerate(zip(spec["iterations"], ref, ours)):
        assert a == want, f"oracle differs from the golden trace at iteration {i}"
        assert b == want, f"package differs from the golden trace at iteration {i}"
