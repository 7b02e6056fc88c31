"""The decode workspaces: split launches merge partial states through a caller-side buffer
whose counters must be zero between launches (q3t_decode_attention's `workspace`).

* Each stream has its own buffer, so split launches on two streams may run at once.
* Each graph capture has its own buffer, zeroed by a reset kernel recorded in that graph, so
  graphs may be replayed in any order, including one replayed before any other has run.
* reset_workspaces re-zeroes the counters after a launch that stopped part-way (planted
  here from the host) and leaves the next launch correct.

Split launches merge their parts in part order, so every output here is compared
bit-for-bit with the same launch run eagerly, one at a time, on the default stream; that
launch is itself checked against the float64 oracle."""
import sys

import pytest
import torch

from oracle import attention as oatt
from tests._util import assert_attention_close, f64

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128
SPLITS = {"chunked": dict(splits=-1, max_chunks=8), "balanced": dict(splits=24)}


def _problem(batch, capacity, seed, device):
    gen = torch.Generator(device=device).manual_seed(seed)
    keys = torch.randn(batch, HKV, capacity, D, generator=gen, device=device, dtype=torch.bfloat16)
    values = torch.randn_like(keys)
    query = torch.randn(batch, 1, HQ, D, generator=gen, device=device, dtype=torch.bfloat16)
    positions = torch.randint(0, capacity, (batch,), generator=gen, device=device)
    return query, keys, values, positions


def _oracle(query, keys, values, positions):
    return oatt.decode_attention(f64(query), f64(keys), f64(values), positions.cpu().numpy(), D ** -0.5)


def test_split_launches_overlap_on_two_streams(pkg, device):
    """Chunked launches on one stream and balanced launches on another, issued alternately
    without synchronisation, each stream with its own workspace."""
    a = _problem(64, 1024, 1, device)
    b = _problem(48, 2048, 2, device)
    expected_a = pkg.decode_attention(*a, **SPLITS["chunked"])
    expected_b = pkg.decode_attention(*b, **SPLITS["balanced"])
    assert_attention_close(f64(expected_a), _oracle(*a))
    assert_attention_close(f64(expected_b), _oracle(*b))
    reps = 12
    out_a = torch.empty((reps,) + tuple(expected_a.shape), device=device, dtype=torch.bfloat16)
    out_b = torch.empty((reps,) + tuple(expected_b.shape), device=device, dtype=torch.bfloat16)
    s1, s2 = torch.cuda.Stream(device), torch.cuda.Stream(device)  # default priority
    s1.wait_stream(torch.cuda.current_stream(device))
    s2.wait_stream(torch.cuda.current_stream(device))
    for i in range(reps):
        with torch.cuda.stream(s1):
            pkg.decode_attention(*a, out=out_a[i], **SPLITS["chunked"])
        with torch.cuda.stream(s2):
            pkg.decode_attention(*b, out=out_b[i], **SPLITS["balanced"])
    torch.cuda.synchronize(device)
    for i in range(reps):
        assert torch.equal(out_a[i], expected_a) and torch.equal(out_b[i], expected_b)


def _captured(pkg, grid, problem, out):
    # captured in inference mode, as the package's graphs are (torch keeps its generator
    # state for graphs as tensors of the mode the first capture ran in)
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph):
        pkg.decode_attention(*problem, out=out, **SPLITS[grid])
    return graph


def test_graphs_replay_in_any_order(pkg, device):
    """Two graphs of split launches captured one after the other and replayed second first,
    then alternately with their inputs rewritten in place between replays; a third graph
    holds a masked bundled launch with the step's plan."""
    a = _problem(64, 1024, 3, device)
    b = _problem(48, 2048, 4, device)
    out_a = torch.empty(64, 1, HQ, D, device=device, dtype=torch.bfloat16)
    out_b = torch.empty(48, 1, HQ, D, device=device, dtype=torch.bfloat16)
    torch.cuda.synchronize(device)
    graph_a = _captured(pkg, "chunked", a, out_a)
    graph_b = _captured(pkg, "balanced", b, out_b)

    qc, kc, vc, pc = _problem(64, 1024, 5, device)
    plan = pkg.decode_plan(pc, 1024, HQ, HKV)
    allowed = torch.arange(1024, device=device)[None, :] <= pc[:, None]
    mask = torch.where(allowed, 0.0, torch.finfo(torch.bfloat16).min).to(torch.bfloat16)[:, None, None, :]
    out_c = torch.empty(64, 1, HQ, D, device=device, dtype=torch.bfloat16)
    torch.cuda.synchronize(device)
    graph_c = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(graph_c):
        pkg.decode_attention(qc, kc, vc, pc, out=out_c, mask=mask, plan=plan, grid="bundled")

    gen = torch.Generator(device=device).manual_seed(6)
    for order in (["b", "a", "c"], ["c", "a", "b"], ["a", "b", "c"]):
        for name in order:
            problem, graph, out, grid = {"a": (a, graph_a, out_a, "chunked"), "b": (b, graph_b, out_b, "balanced"),
                                         "c": (None, graph_c, out_c, None)}[name]
            if name == "c":
                graph.replay()
                expected = pkg.decode_attention(qc, kc, vc, pc, mask=mask, plan=plan, grid="bundled")
                torch.cuda.synchronize(device)
                assert torch.equal(out, expected)
                continue
            query, keys, values, positions = problem
            query.copy_(torch.randn(query.shape, generator=gen, device=device, dtype=torch.bfloat16))
            positions.copy_(torch.randint(0, keys.shape[2], positions.shape, generator=gen, device=device))
            graph.replay()
            expected = pkg.decode_attention(*problem, **SPLITS[grid])
            torch.cuda.synchronize(device)
            assert torch.equal(out, expected)
    assert_attention_close(f64(out_a), _oracle(*a))
    assert_attention_close(f64(out_b), _oracle(*b))


@pytest.mark.parametrize("grid", ["chunked", "balanced"])
def test_reset_after_a_launch_that_stopped_part_way(pkg, device, grid):
    """A call refused for its arguments launches nothing and leaves the counters as they were;
    counters left non-zero by a launch that stopped part-way (planted from the host) are
    cleared by reset_workspaces, after which the next split launch is exact again."""
    problem = _problem(64, 1024, 7, device)
    expected = pkg.decode_attention(*problem, **SPLITS[grid])
    query, keys, values, positions = problem
    with pytest.raises(ValueError):
        pkg.decode_attention(query, keys, values, positions.int(), **SPLITS[grid])
    assert torch.equal(pkg.decode_attention(*problem, **SPLITS[grid]), expected)
    stream = torch.cuda.current_stream(device).cuda_stream
    module = sys.modules[pkg.__name__ + ".attention"]
    buffer = module.workspace(device, 1, stream)         # this stream's eager workspace
    buffer[:1 << 18].fill_(1)                            # its counter region, all non-zero
    pkg.reset_workspaces(device)
    out = pkg.decode_attention(*problem, **SPLITS[grid])
    torch.cuda.synchronize(device)
    assert torch.equal(out, expected)
    assert not bool(buffer[:1 << 18].any())
    assert_attention_close(f64(out), _oracle(*problem))
