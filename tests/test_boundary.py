"""The C-ABI boundary without a GPU: the library loads, exports every symbol the header
declares, its structs match ctypes field for field, and host validation raises ValueError
before anything is launched (the reference's error convention, tests/test_packed_kv.py:45-81)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qwen3tts_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = re.findall(r"\b(q3t_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.library()
    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert set(names) == set(pkg._lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_status_strings_and_version(pkg):
    lib = pkg.library()
    assert lib.q3t_abi_version() == 8
    assert lib.q3t_status_string(0) == b"success"
    assert lib.q3t_status_string(-1) == b"invalid argument"
    assert lib.q3t_status_string(-3) == b"workspace missing or too small"


def _c_layout(struct_name, fields, tmp_path):
    src = tmp_path / "layout.c"
    lines = [f'#include "{HEADER}"', "#include <stdio.h>", "#include <stddef.h>", "int main(void) {",
             f'  printf("%zu\\n", sizeof({struct_name}));']
    lines += [f'  printf("%zu\\n", offsetof({struct_name}, {f}));' for f in fields]
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", str(src), "-o", str(exe)], check=True)
    return [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]


@pytest.mark.parametrize("name,cls", [("q3t_decode_args", "DecodeArgs"), ("q3t_prefill_args", "PrefillArgs"),
                                      ("q3t_prefill_rope_write_args", "PrefillRopeWriteArgs")])
def test_struct_layouts_match_the_header(pkg, tmp_path, name, cls):
    struct = getattr(pkg._lib, cls)
    fields = [f for f, _ in struct._fields_]
    c = _c_layout(name, fields, tmp_path)
    assert c[0] == ctypes.sizeof(struct)
    assert c[1:] == [getattr(struct, f).offset for f in fields]


def test_rejected_calls_return_negative_status_without_a_gpu(pkg):
    lib = pkg.library()
    zero = pkg._lib.i64x3((0, 0, 0))
    assert lib.q3t_kv_write(None, None, None, None, None, 1, 1, 1, 1, 2, zero, zero, zero, 1, None) == -1
    assert lib.q3t_rotary(None, None, None, None, 1, 1, 128, 0, None) == -1
    assert lib.q3t_decode_attention(None, None) == -1
    args = pkg._lib.DecodeArgs()
    args.batch, args.query_len, args.q_heads, args.kv_heads, args.head_dim, args.ctx = 1, 1, 16, 8, 96, 8
    args.query = args.keys = args.values = args.positions = args.out = 16
    args.dtype = 0
    assert lib.q3t_decode_attention(args, None) == -2   # head_dim 96 not compiled
    args.head_dim = 128
    assert lib.q3t_decode_attention(args, None) == -3   # no workspace
    args.max_chunks = 1025
    assert lib.q3t_decode_attention(args, None) == -1   # more chunks than supported
    args.max_chunks, args.splits = 0, 32769
    assert lib.q3t_decode_attention(args, None) == -1   # more splits than supported
    args.splits, args.grid = 0, 4
    assert lib.q3t_decode_attention(args, None) == -1   # no such grid
    args.grid, args.query_len = 3, 2
    assert lib.q3t_decode_attention(args, None) == -2   # two query tokens: not on the bundled grid
    args.grid, args.query_len = 0, 1
    assert lib.q3t_decode_reset_workspace(None, 1 << 20, None) == -3
    assert lib.q3t_decode_plan(None, 4, 1024, 16, 8, 16, None) == -1      # no positions
    assert lib.q3t_decode_plan(16, 129, 1024, 16, 8, 16, None) == -1      # more requests than a plan covers
    assert lib.q3t_decode_plan(16, 4, 0, 16, 8, 16, None) == -1           # no arena rows
    assert lib.q3t_decode_plan(16, 4, (1 << 20) + 1, 16, 8, 16, None) == -1
    assert lib.q3t_decode_plan(16, 4, 1024, 40, 8, 16, None) == -1        # 5 query heads per KV head
    assert lib.q3t_decode_plan(16, 4, 1024, 16, 8, 8, None) == -1         # plan not 16-byte aligned
    assert lib.q3t_decode_plan(None, 0, 1024, 16, 8, None, None) == 0     # an empty batch launches nothing
    # the plan's size: (batch, M) and four (b, L) pairs of 4-byte ints for each of the M
    # bundles of a KV head: M = 32 for 8 KV heads (one workgroup per CU), more when a batch
    # needs more than 4 requests per bundle
    def size(bundles):
        return 8 + bundles * 4 * 8
    assert lib.q3t_decode_plan_bytes(64, 16, 8) == size(32)
    assert lib.q3t_decode_plan_bytes(128, 16, 16) == size(32)
    assert lib.q3t_decode_plan_bytes(128, 64, 64) == size(32)
    assert lib.q3t_decode_plan_bytes(128, 4, 4) == size(64)
    assert lib.q3t_decode_plan_bytes(64, 40, 8) == -1
    # the allocation-free entry point refuses, before touching any device, a call whose split
    # states would not fit its fixed 8 MiB array (1024 requests x 8 heads x 16 chunks)
    big = pkg._lib.DecodeArgs()
    big.batch, big.query_len, big.q_heads, big.kv_heads, big.head_dim, big.ctx = 1024, 1, 16, 8, 128, 1024
    big.query = big.keys = big.values = big.positions = big.out = 16
    big.splits, big.max_chunks = -1, 16
    assert lib.q3t_decode_attention_static(big, None) == -3


def _ws(lib, pkg, batch, qlen, ctx, max_chunks=0, splits=0, fused=0, masked=False, dtype=0, grid=0):
    a = pkg._lib.DecodeArgs()
    a.batch, a.query_len, a.q_heads, a.kv_heads, a.head_dim, a.ctx = batch, qlen, 16, 8, 128, ctx
    a.dtype, a.fused, a.max_chunks, a.splits, a.grid = dtype, fused, max_chunks, splits, grid
    a.mask = 16 if masked else None
    return lib.q3t_decode_workspace_bytes(a)


def test_decode_workspace_sizes(pkg):
    """256 KiB of counters, then one (G * query_len) x (head_dim + 2) fp32 state per part.
    Chunked grid: ctx 1024 is 16 blocks of 64 keys, chunks capped by max_chunks, by default
    at ceil(512 / (batch * kv_heads)).  Balanced grid: two state slots per workgroup, by
    default 256 / kv_heads workgroups per head.  Bundled grid: no workspace at all.  Automatic
    choice: bundled for bf16 single-token launches of 24..63 requests (192..511 (request, KV
    head) items) from 512 rows, of 64..128 requests from 1024 rows, and of 48 or more from 4096
    rows; balanced otherwise from 2048 rows, chunked otherwise."""
    lib = pkg.library()
    counters = 65536 * 4
    state = 2 * 130 * 4
    assert _ws(lib, pkg, 64, 1, 1024) == 0                                           # bundled
    assert _ws(lib, pkg, 128, 1, 2047) == 0                                          # bundled
    assert _ws(lib, pkg, 129, 1, 1024) == counters + 129 * 8 * 1 * state             # chunked
    assert _ws(lib, pkg, 63, 1, 1024) == 0                                           # bundled
    assert _ws(lib, pkg, 24, 1, 512) == 0                                            # bundled
    assert _ws(lib, pkg, 23, 1, 1024) == counters + 23 * 8 * 3 * state               # chunked
    assert _ws(lib, pkg, 64, 1, 1023) == counters + 64 * 8 * 1 * state               # chunked
    assert _ws(lib, pkg, 63, 1, 511) == counters + 63 * 8 * 2 * state                # chunked
    assert _ws(lib, pkg, 64, 1, 1024, dtype=2) == counters + 64 * 8 * 1 * state      # fp32: chunked
    assert _ws(lib, pkg, 64, 1, 1024, masked=True) == counters + 64 * 8 * 1 * state  # mask: chunked
    assert _ws(lib, pkg, 64, 1, 1024, grid=1) == counters + 64 * 8 * 1 * state       # named chunked
    assert _ws(lib, pkg, 64, 1, 1024, grid=2) == counters + 8 * 32 * 2 * state       # named balanced
    assert _ws(lib, pkg, 8, 1, 64, grid=3) == 0                                      # named bundled
    assert _ws(lib, pkg, 64, 2, 1024, grid=3) == counters  # sized; the launch refuses the grid
    assert _ws(lib, pkg, 64, 1, 1024, grid=4) == -1       # no such grid
    assert _ws(lib, pkg, 64, 1, 4096) == 0                                           # bundled
    assert _ws(lib, pkg, 47, 1, 4096) == counters + 8 * 32 * 2 * state              # balanced
    assert _ws(lib, pkg, 64, 1, 1024, splits=7) == counters + 8 * 7 * 2 * state
    assert _ws(lib, pkg, 64, 1, 4096, splits=-1) == counters + 64 * 8 * 1 * state    # chunked
    assert _ws(lib, pkg, 64, 1, 1024, splits=-1) == counters + 64 * 8 * 1 * state    # chunked
    assert _ws(lib, pkg, 8, 1, 1024) == counters + 8 * 8 * 8 * state
    assert _ws(lib, pkg, 2, 1, 1024) == counters + 2 * 8 * 16 * state
    assert _ws(lib, pkg, 64, 2, 1024, max_chunks=4) == counters + 64 * 8 * 4 * 2 * state
    assert _ws(lib, pkg, 64, 1, 16) == counters + 64 * 8 * 1 * state
    assert _ws(lib, pkg, 64, 1, 16, fused=1, masked=True) == counters + 64 * 8 * 1 * state
    assert _ws(lib, pkg, 64, 1, 1024, max_chunks=1025) == -1
    assert _ws(lib, pkg, 64, 1, 1024, splits=32769) == -1


def test_decode_grid_choice(pkg):
    """The library's grid choice, without a GPU: the talker step (64 requests, 1024-row arena)
    runs bundled, also with the reference's mask, and so do 24..63 requests from 512 rows;
    64 or more requests over 512..1023 rows, short arenas and small batches run chunked, few
    requests over long arenas balanced; splits still selects balanced (> 0) or chunked (< 0)
    under the automatic choice."""
    decode_grid_for = pkg.decode_grid_for
    assert decode_grid_for(64, 1, 16, 8, 128, 1024) == "bundled"
    assert decode_grid_for(128, 1, 16, 8, 128, 1500) == "bundled"
    assert decode_grid_for(64, 1, 16, 8, 128, 4096) == "bundled"
    assert decode_grid_for(47, 1, 16, 8, 128, 4096) == "balanced"
    assert decode_grid_for(16, 1, 16, 8, 128, 2048) == "balanced"
    assert decode_grid_for(64, 1, 16, 8, 128, 16) == "chunked"
    assert decode_grid_for(128, 1, 16, 8, 128, 511) == "chunked"
    assert decode_grid_for(32, 1, 16, 8, 128, 1024) == "bundled"
    assert decode_grid_for(24, 1, 16, 8, 128, 512) == "bundled"
    assert decode_grid_for(63, 1, 16, 8, 128, 512, masked=True) == "bundled"
    assert decode_grid_for(23, 1, 16, 8, 128, 1024) == "chunked"
    assert decode_grid_for(64, 1, 16, 8, 128, 512) == "chunked"
    assert decode_grid_for(128, 1, 16, 8, 128, 1023) == "chunked"
    assert decode_grid_for(128, 1, 16, 8, 128, 3000) == "bundled"
    assert decode_grid_for(64, 2, 16, 8, 128, 1024) == "chunked"
    assert decode_grid_for(64, 1, 16, 8, 128, 1024, masked=True) == "bundled"
    assert decode_grid_for(64, 1, 16, 8, 128, 1024, torch.float32) == "chunked"
    assert decode_grid_for(64, 1, 16, 8, 128, 1024, splits=-1) == "chunked"
    assert decode_grid_for(64, 1, 16, 8, 128, 1024, splits=9) == "balanced"
    assert decode_grid_for(4, 1, 16, 8, 128, 16, grid="bundled") == "bundled"
    assert decode_grid_for(64, 1, 16, 8, 128, 1024, grid="chunked") == "chunked"
    with pytest.raises(ValueError):
        decode_grid_for(64, 2, 16, 8, 128, 1024, grid="bundled")
    with pytest.raises(ValueError):
        decode_grid_for(64, 1, 64, 8, 128, 1024, grid="bundled")   # 8 query heads per KV head


def test_wrappers_reject_cpu_tensors(pkg):
    k = torch.zeros(2, 8, 1, 128, dtype=torch.bfloat16)
    t = torch.zeros(2, 8, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.write(k, k, t, t.clone(), torch.zeros(2, dtype=torch.int64))
    with pytest.raises(ValueError):
        pkg.rotary(torch.zeros(1, 1, 8, 128, dtype=torch.bfloat16), torch.zeros(1, 1, 128, dtype=torch.bfloat16),
                   torch.zeros(1, 1, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        pkg.decode_attention(torch.zeros(2, 1, 16, 128, dtype=torch.bfloat16), t, t,
                             torch.zeros(2, dtype=torch.int64))


def test_kv_write_validation_mirrors_reference(pkg):
    """kv_triton_ascend.write's shape/dtype/position checks (kv_triton_ascend.py:41-53)."""
    k = torch.zeros(2, 8, 1, 128, dtype=torch.bfloat16)
    t = torch.zeros(2, 8, 16, 128, dtype=torch.bfloat16)
    pos = torch.zeros(2, dtype=torch.int64)
    for bad in [(k[:, :, :0], k, t, t, pos), (k, k, t[:1], t[:1], pos), (k, k, t, t, pos.int()),
                (k, k, t, t, pos[:1]), (k, k.float(), t, t, pos), (k, k, t[..., ::2], t[..., ::2], pos)]:
        with pytest.raises(ValueError):
            pkg.write(*bad)


def test_packed_prefix_rejects_before_any_write(pkg):
    """tests/test_packed_kv.py:45-81 run on CPU tensors: every invalid call raises."""
    target = torch.full((4, 5, 2, 7, 3), -7.0)
    source = torch.arange(4 * 3 * 2 * 5 * 6).view(4, 3, 2, 5, 6).float()[..., ::2]
    saved = target.clone()
    for slot, row, length in ((-1, 0, 1), (5, 0, 1), (0, 3, 1), (0, -1, 1), (0, 0, 0), (0, 0, 6),
                              (True, 0, 1), (0, True, 1), (0, 0, True)):
        with pytest.raises(ValueError):
            pkg.copy_packed_prefix(target, source, slot, row=row, length=length)
    for bad in (source[:3], source[:, :, :1], source[..., :2], source.double(), source[0], source[:, :0],
                target, torch.empty_like(source, device="meta")):
        with pytest.raises(ValueError):
            pkg.copy_packed_prefix(target, bad, 0, length=1)
    assert torch.equal(target, saved)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus above 1 exits with a message before touching a GPU."""
    import sys
    done = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=300, cwd=ROOT)
    assert done.returncode == 2
    assert "one GPU" in done.stderr and done.stdout == ""
