"""Grouped-query attention on the GPU: decode (split-K), fused decode step, drop-in dispatch.

* ``decode_attention`` - ragged GQA over a slot arena: request b attends keys
  0 ... positions[b] of its slot (the mask ``j <= pos[b]`` of SlotGraph.compute,
  qwen3_tts_engine/continuous.py:191-192), optionally under an SDPA-style mask.
* ``decode_step`` - one launch doing RoPE of q and the new key, the paired K/V write at
  positions[b] and the attention (PackedAttention.forward's decode path,
  qwen3_tts_engine/packed_attention.py:46-84).
* ``attention`` - drop-in for ``npu_attention.attention``
  (qwen3_tts_engine/npu_attention.py:11-26): same signature, errors and output layout.
* ``prefill_attention`` - varlen causal attention over cu_seqlens on bf16 MFMA tiles.
"""
from __future__ import annotations

import torch

from . import _lib

_WORKSPACES: dict = {}
_RETIRED: list = []


def workspace(device: torch.device, nbytes: int, stream: int | None = None) -> torch.Tensor:
    """Split-softmax workspace of one stream of ``device``, or of one graph capture, its
    counters zeroed.

    Kernels leave the counters zeroed, so one buffer serves every sequential launch on its
    stream; launches on different streams get different buffers, so they may overlap.  Eager
    launches share the stream's buffer, zeroed by the library's reset kernel when it is
    created.  A launch being captured gets the buffer of its capture instead (keyed by the
    capture id), created in the graph's memory pool and zeroed by a reset kernel recorded in
    that graph ahead of its first use, so every replay starts from zeroed counters and no two
    graphs share a buffer (they may be replayed in any order, also on different streams; one
    graph's replays must not overlap each other).  A buffer that grows during a capture keeps
    the old one alive with the process (the graph's earlier launches use it); an eager buffer
    replaced by a larger one is released at once."""
    stream = _lib.stream_handle(device) if stream is None else stream
    capturing = torch.cuda.is_current_stream_capturing()
    key = (device, stream, _lib.capture_id(stream) if capturing else 0)
    current = _WORKSPACES.get(key)
    if current is None or current.numel() < nbytes:
        buffer = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        status = _lib.library().q3t_decode_reset_workspace(buffer.data_ptr(), buffer.numel(), stream)
        _lib.check(status, 'decode workspace')
        if current is not None and key[2]:
            _RETIRED.append(current)
        _WORKSPACES[key] = current = buffer
    return current


def reset_workspaces(device: torch.device | None = None) -> None:
    """Re-zero the counters of every decode workspace (of ``device``, or of all devices),
    on each workspace's own stream: after a launch that failed part-way, counters may be
    left non-zero and would mislead the next launch that splits a request."""
    lib = _lib.library()
    for (dev, stream, _), ws in list(_WORKSPACES.items()):
        if device is not None and dev != torch.device(device):
            continue
        with torch.cuda.device(dev):
            status = lib.q3t_decode_reset_workspace(ws.data_ptr(), ws.numel(), stream)
        _lib.check(status, 'decode workspace reset')


def _mask_view(mask, batch, query_len, ctx):
    """SDPA-style mask broadcastable to (batch, 1, query_len, ctx) -> (batch, query_len, ctx)."""
    if mask.ndim == 4:
        if mask.shape[1] != 1:
            raise ValueError('per-head attention masks are not supported')
        mask = mask[:, 0]
    elif mask.ndim == 2:
        mask = mask[None]
    if mask.ndim != 3 or mask.shape[-1] != ctx:
        raise ValueError('attention mask must end in the key dimension')
    if mask.dtype not in _lib.DTYPE_CODES:
        raise ValueError('attention mask must be bool, bf16, fp16 or fp32')
    return mask.expand(batch, query_len, ctx)


def _run_decode(args: _lib.DecodeArgs, device: torch.device, what: str, no_alloc: bool = False) -> None:
    lib = _lib.library()
    with torch.cuda.device(device):
        stream = _lib.stream_handle(device)
        if no_alloc:
            status = lib.q3t_decode_attention_static(args, stream)
        else:
            need = lib.q3t_decode_workspace_bytes(args)
            if need < 0:
                raise ValueError(f'{what}: invalid sizes')
            if need > 0:  # the bundled grid needs none
                ws = workspace(device, need, stream)
                args.workspace = ws.data_ptr()
                args.workspace_bytes = ws.numel()
            status = lib.q3t_decode_attention(args, stream)
    _lib.check(status, what)


def _check_out(out, shape, dtype, device, what):
    """A caller-supplied output: the exact shape and dtype, unit-stride rows, on the device."""
    if (tuple(out.shape) != tuple(shape) or out.dtype != dtype or out.device != device
            or out.stride(-1) != 1):
        raise ValueError(f'{what}: out must be a {tuple(shape)} {dtype} tensor on {device} '
                         'with unit-stride rows')


GRIDS = {None: 0, 'auto': 0, 'chunked': 1, 'balanced': 2, 'bundled': 3}


def _grid_code(grid):
    if grid not in GRIDS:
        raise ValueError(f"grid must be one of {sorted(k for k in GRIDS if k)} or None")
    return GRIDS[grid]


def decode_grid_for(batch, query_len, q_heads, kv_heads, head_dim, ctx, dtype=torch.bfloat16, *,
                    masked=False, splits=0, grid=None):
    """Name of the grid a decode call of these sizes runs on ('bundled', 'balanced' or
    'chunked'), as the library chooses it (q3t_decode_grid); ValueError when a named grid does
    not take such a call.  ``masked``: a contiguous (batch, 1, ctx) bf16 mask, as
    SlotGraph.compute builds it."""
    a = _lib.DecodeArgs()
    a.batch, a.query_len, a.q_heads, a.kv_heads, a.head_dim, a.ctx = batch, query_len, q_heads, kv_heads, head_dim, ctx
    a.dtype = _lib.DTYPE_CODES[dtype]
    a.k_stride_b = a.v_stride_b = kv_heads * ctx * head_dim
    a.k_stride_h = a.v_stride_h = ctx * head_dim
    a.k_stride_t = a.v_stride_t = head_dim
    if masked:
        a.mask, a.mask_dtype = 16, _lib.Q3T_BF16
        a.mask_stride_b, a.mask_stride_s, a.mask_stride_t = ctx, ctx, 1
    a.splits, a.grid = int(splits), _grid_code(grid)
    code = _lib.library().q3t_decode_grid(a)
    if code < 0:
        _lib.check(code, 'decode grid')
    return {v: k for k, v in GRIDS.items() if k not in (None, 'auto')}[code]


PLAN_MAX_BATCH = 128  # requests a decode plan covers (the bundled grid's limit)


def plan_shape(batch, q_heads, kv_heads):
    """Shape of the int32 plan ``decode_plan`` writes for a launch of these sizes: one
    dimension holding (batch, M) and four (request, length) pairs for each of the M bundles
    (workgroups) of a KV head (q3t_decode_plan); None when no plan covers the shape."""
    nbytes = _lib.library().q3t_decode_plan_bytes(int(batch), int(q_heads), int(kv_heads))
    if nbytes <= 0:
        return None
    return (nbytes // 4,)


def decode_plan(positions, capacity, q_heads, kv_heads, *, out=None):
    """The bundled grid's plan of a step, made once for the step's positions and passed as
    ``plan=`` to every layer's ``decode_step`` / ``decode_attention`` of that step (the layers
    of a talker step all attend the same lengths, SlotGraph.compute, continuous.py:188-198).
    positions (B,) int64 with B <= 128, capacity: the arena's rows (a position at or past it
    attends nothing), q_heads / kv_heads: the attention's heads (q_heads / kv_heads <= 4).
    The requests are ranked by length and bundled, whole, one bundle per workgroup of each KV
    head, the i-th longest with the i-th shortest.  Returns an int32 ``plan_shape`` tensor.
    One small kernel on the current stream (it can be captured); the plan stays valid while
    ``positions`` are unchanged: a plan of other positions gives wrong outputs."""
    if positions.ndim != 1 or positions.dtype != torch.int64:
        raise ValueError('positions must be an int64 (batch,) tensor')
    batch = positions.shape[0]
    if batch > PLAN_MAX_BATCH:
        raise ValueError(f'a decode plan covers at most {PLAN_MAX_BATCH} requests')
    if not 1 <= int(capacity) <= 1 << 20:
        raise ValueError('capacity must be in [1, 2^20]')
    shape = plan_shape(batch, q_heads, kv_heads)
    if shape is None:
        raise ValueError('a decode plan needs q_heads a multiple of kv_heads, at most 4 per KV head')
    device = _lib.require_gpu(positions)
    if not positions.is_contiguous():
        positions = positions.contiguous()
    if out is None:
        out = torch.empty(shape, device=device, dtype=torch.int32)
    else:
        _check_out(out, shape, torch.int32, device, 'decode plan')
        if not out.is_contiguous():
            raise ValueError('decode plan: out must be contiguous')
    with torch.cuda.device(device):
        status = _lib.library().q3t_decode_plan(positions.data_ptr(), batch, int(capacity), int(q_heads),
                                                int(kv_heads), out.data_ptr(), _lib.stream_handle(device))
    _lib.check(status, 'decode plan')
    return out


def _set_plan(a, plan, device):
    if plan is None:
        return
    shape = plan_shape(a.batch, a.q_heads, a.kv_heads)
    if (shape is None or tuple(plan.shape) != shape or plan.dtype != torch.int32 or not plan.is_contiguous()
            or plan.device != device):
        raise ValueError(f'plan must be the contiguous int32 {shape} tensor of decode_plan on {device}')
    a.plan = plan.data_ptr()


def decode_attention(query, keys, values, positions, *, scale=None, mask=None, kv_offsets=None,
                     out=None, max_chunks=0, splits=0, grid=None, no_alloc=False, plan=None):
    """query (B, S, Hq, D) BSND; keys/values (B, Hkv, ctx, D) views of the arena (or, with
    ``kv_offsets``, any base tensor whose request rows start at those element offsets);
    positions (B,) int64: the last query position of each request.  ``grid`` picks the
    kernel grid: 'bundled' (one workgroup per CU streaming through LDS onto bf16 MFMA tiles: whole
    requests in length-balanced bundles, bundled by ``plan`` when given; a mask with unit key
    stride; one query token, head_dim 128, up to 128 requests), 'balanced'
    (equal shares of each head's keys over ``splits`` workgroups per head, 0: 256 in all),
    'chunked' (chunks of 64-key blocks per request, at most ``max_chunks``, 0: enough for
    ~512 workgroups) or None for the library's choice, in which ``splits`` > 0 / < 0 still
    selects balanced / chunked.  ``no_alloc`` runs the library's allocation-free entry point, which keeps
    its split states in a fixed per-GPU device array instead of a workspace (calls that
    overlap in time on one GPU then race).  ``plan``: ``decode_plan(positions, ctx, q_heads,
    kv_heads)`` of these positions, read by the bundled grid (other grids ignore it).
    Returns (B, S, Hq, D)."""
    if query.ndim != 4 or keys.ndim != 4 or values.shape != keys.shape:
        raise ValueError('expected BSND query and BNSD key/value views')
    batch, qlen, q_heads, head_dim = query.shape
    kv_heads, ctx = keys.shape[1], keys.shape[2]
    if kv_offsets is None and keys.shape[0] < batch:
        raise ValueError('key/value views must cover every request')
    if keys.shape[3] != head_dim or q_heads % kv_heads:
        raise ValueError('head_dim mismatch or q_heads not a multiple of kv_heads')
    if query.dtype not in (torch.bfloat16, torch.float32) or keys.dtype != query.dtype or values.dtype != query.dtype:
        raise ValueError('decode attention supports bf16 or fp32 tensors of one dtype')
    if positions.shape != (batch,) or positions.dtype != torch.int64:
        raise ValueError('positions must be an int64 (batch,) tensor')
    if query.stride(3) != 1 or keys.stride(3) != 1 or values.stride(3) != 1:
        raise ValueError('rows must be unit-stride along head_dim')
    tensors = [query, keys, values, positions] + ([kv_offsets] if kv_offsets is not None else [])
    device = _lib.require_gpu(*tensors)
    if out is None:
        out = torch.empty(batch, qlen, q_heads, head_dim, device=device, dtype=query.dtype)
    else:
        _check_out(out, (batch, qlen, q_heads, head_dim), query.dtype, device, 'decode attention')
    a = _lib.DecodeArgs()
    a.batch, a.query_len, a.q_heads, a.kv_heads, a.head_dim = batch, qlen, q_heads, kv_heads, head_dim
    a.ctx = ctx
    a.dtype = _lib.DTYPE_CODES[query.dtype]
    a.scale = head_dim ** -0.5 if scale is None else float(scale)
    a.fused = 0
    a.query = query.data_ptr()
    a.q_stride_b, a.q_stride_s, a.q_stride_h = query.stride()[:3]
    a.keys, a.values = keys.data_ptr(), values.data_ptr()
    a.k_stride_b, a.k_stride_h, a.k_stride_t = keys.stride()[:3]
    a.v_stride_b, a.v_stride_h, a.v_stride_t = values.stride()[:3]
    if kv_offsets is not None:
        if kv_offsets.shape != (batch,) or kv_offsets.dtype != torch.int64:
            raise ValueError('kv_offsets must be an int64 (batch,) tensor')
        a.kv_offsets = kv_offsets.data_ptr()
    a.positions = positions.data_ptr()
    if mask is not None:
        m = _mask_view(mask.to(device), batch, qlen, ctx)
        a.mask = m.data_ptr()
        a.mask_dtype = _lib.DTYPE_CODES[m.dtype]
        a.mask_stride_b, a.mask_stride_s, a.mask_stride_t = m.stride()
    a.out = out.data_ptr()
    a.o_stride_b, a.o_stride_s, a.o_stride_h = out.stride()[:3]
    a.max_chunks = int(max_chunks)
    a.splits = int(splits)
    a.grid = _grid_code(grid)
    _set_plan(a, plan, device)
    _run_decode(a, device, 'decode attention', no_alloc)
    return out


def decode_step(query, new_key, new_value, key_arena, value_arena, positions, cos, sin, *,
                scale=None, out=None, max_chunks=0, splits=0, grid=None, q_norm_weight=None,
                k_norm_weight=None, norm_eps=1e-6, mask=None, no_alloc=False, plan=None):
    """Fused decode step of a layer for one token, or two (the code predictor's first step).

    query (B, S, Hq, D), new_key/new_value (B, S, Hkv, D) with S in {1, 2}: un-rotated bf16
    rows (views of the fused QKV projection are fine); key_arena/value_arena (slots >= B, Hkv,
    C, D) contiguous; positions (B,) int64, the position of the step's last token; cos/sin
    (B, S, D), or (B, D) for one token, bf16.  Writes the rotated keys and the values at
    positions[b] - S + 1 ... positions[b] and returns the attention output (B, S, Hq, D); with
    two tokens the first does not attend the second (2x2 causal, continuous.py:39-40).

    With ``q_norm_weight`` / ``k_norm_weight`` (bf16 (D,)) the query / key rows are first
    RMS-normalised in the kernel (the module's q_norm / k_norm, eps ``norm_eps``): raw
    projection rows go in and no separate norm kernels run.  The fp32 row sums follow the
    kernel's order, so a result can differ from another implementation's in the last bf16 bit.

    ``mask`` (SDPA-style, broadcastable to (B, 1, S, C)) is added to the scores of the keys
    0 ... positions[b], as the reference's operator applies the mask it is given; without it
    request b attends exactly those keys (the ``j <= pos[b]`` mask of SlotGraph.compute).
    ``grid`` / ``splits`` / ``max_chunks`` choose the grid, ``no_alloc`` the
    allocation-free entry point and ``plan`` the step's plan, as in ``decode_attention``."""
    if (query.ndim != 4 or query.shape[1] not in (1, 2) or new_key.ndim != 4
            or new_key.shape[1] != query.shape[1]):
        raise ValueError('fused decode expects one- or two-token BSND rows')
    batch, tokens, q_heads, head_dim = query.shape
    if new_value.shape != new_key.shape or new_key.shape[0] != batch or new_key.shape[3] != head_dim:
        raise ValueError('new key/value rows must match the query batch and head_dim')
    kv_heads = new_key.shape[2]
    if (key_arena.ndim != 4 or key_arena.shape != value_arena.shape or key_arena.shape[0] < batch
            or key_arena.shape[1] != kv_heads or key_arena.shape[3] != head_dim
            or not key_arena.is_contiguous() or not value_arena.is_contiguous()):
        raise ValueError('arena planes must be contiguous (slots, kv_heads, capacity, head_dim)')
    if head_dim != 128 or q_heads % kv_heads:
        raise ValueError('fused decode supports head_dim 128 with q_heads a multiple of kv_heads')
    tensors = (query, new_key, new_value, key_arena, value_arena, cos, sin)
    if any(t.dtype != torch.bfloat16 for t in tensors):
        raise ValueError('fused decode is bf16-only (exact RoPE rounding contract)')
    if positions.shape != (batch,) or positions.dtype != torch.int64:
        raise ValueError('positions must be an int64 (batch,) tensor')
    cos3 = cos[:, None] if cos.ndim == 2 else cos
    sin3 = sin[:, None] if sin.ndim == 2 else sin
    if (cos3.shape != (batch, tokens, head_dim) or sin3.shape != cos3.shape or cos3.stride(2) != 1
            or sin3.stride() != cos3.stride()):
        raise ValueError('cos/sin must be (B, S, head_dim) rows')
    if any(t.stride(3) != 1 for t in (query, new_key, new_value)):
        raise ValueError('rows must be unit-stride along head_dim')
    device = _lib.require_gpu(*tensors, positions)
    if out is None:
        out = torch.empty(batch, tokens, q_heads, head_dim, device=device, dtype=query.dtype)
    else:
        _check_out(out, (batch, tokens, q_heads, head_dim), query.dtype, device, 'fused decode step')
    a = _lib.DecodeArgs()
    a.batch, a.query_len, a.q_heads, a.kv_heads, a.head_dim = batch, tokens, q_heads, kv_heads, head_dim
    a.ctx = key_arena.shape[2]
    a.dtype = _lib.Q3T_BF16
    a.scale = head_dim ** -0.5 if scale is None else float(scale)
    a.fused = 1
    a.query = query.data_ptr()
    a.q_stride_b, a.q_stride_s, a.q_stride_h = query.stride()[:3]
    a.keys, a.values = key_arena.data_ptr(), value_arena.data_ptr()
    a.k_stride_b, a.k_stride_h, a.k_stride_t = key_arena.stride()[:3]
    a.v_stride_b, a.v_stride_h, a.v_stride_t = value_arena.stride()[:3]
    a.positions = positions.data_ptr()
    a.out = out.data_ptr()
    a.o_stride_b, a.o_stride_s, a.o_stride_h = out.stride()[:3]
    a.new_key, a.new_value = new_key.data_ptr(), new_value.data_ptr()
    a.nk_stride_b, a.nk_stride_s, a.nk_stride_h = new_key.stride()[:3]
    a.nv_stride_b, a.nv_stride_s, a.nv_stride_h = new_value.stride()[:3]
    a.cos, a.sin = cos3.data_ptr(), sin3.data_ptr()
    a.cs_stride_b, a.cs_stride_s = cos3.stride(0), cos3.stride(1)
    a.max_chunks = int(max_chunks)
    a.splits = int(splits)
    a.grid = _grid_code(grid)
    if mask is not None:
        # the mask covers keys 0 ... width-1 (SlotGraph's context view, continuous.py:184-192)
        width = mask.shape[-1]
        if not 1 <= width <= a.ctx:
            raise ValueError('the mask is wider than the arena')
        a.ctx = width
        m = _mask_view(mask.to(device), batch, tokens, a.ctx)
        a.mask = m.data_ptr()
        a.mask_dtype = _lib.DTYPE_CODES[m.dtype]
        a.mask_stride_b, a.mask_stride_s, a.mask_stride_t = m.stride()
    for name, weight in (('q_norm_weight', q_norm_weight), ('k_norm_weight', k_norm_weight)):
        if weight is None:
            continue
        if weight.shape != (head_dim,) or weight.dtype != torch.bfloat16 or not weight.is_contiguous():
            raise ValueError(f'{name} must be a contiguous bf16 ({head_dim},) tensor')
        _lib.require_gpu(weight)
        setattr(a, name, weight.data_ptr())
    a.norm_eps = float(norm_eps)
    _set_plan(a, plan, device)
    _run_decode(a, device, 'fused decode step', no_alloc)
    return out


_UNIFORM_CU: dict = {}


def _uniform_cu(batch, length, device):
    """Row offsets 0, L, 2L, ... of a (batch, length) padded batch as int32 cu_seqlens, kept
    per shape so that captured graphs keep using the same tensor."""
    key = (batch, length, device)
    cu = _UNIFORM_CU.get(key)
    if cu is None:
        cu = _UNIFORM_CU[key] = torch.arange(0, (batch + 1) * length, length, device=device,
                                             dtype=torch.int32)
    return cu


_LENGTH_POSITIONS: dict = {}


def _length_positions(lengths, device, counts=False):
    """Device positions n - 1 (int64), or with ``counts`` the key counts n (int32), for a list
    of key counts, cached: captured graphs keep using the same tensor, and no host copy
    happens during capture."""
    key = (tuple(int(n) for n in lengths), device, counts)
    cached = _LENGTH_POSITIONS.get(key)
    if cached is None:
        if torch.cuda.is_current_stream_capturing():
            raise ValueError('actual_seq_lengths_kv must be seen once before graph capture')
        if counts:
            cached = torch.tensor(key[0], device=device, dtype=torch.int32)
        else:
            cached = torch.tensor([n - 1 for n in key[0]], device=device, dtype=torch.int64)
        _LENGTH_POSITIONS[key] = cached
    return cached


def attention(module, query, key, value, attention_mask, **kwargs):
    """Drop-in for the reference's native GQA call: query (B, Hq, S, D), key/value
    (B, Hkv, ctx, D) BNSD; returns ((B, S, Hq, D) contiguous, None).

    ``kv_positions`` (a device int64 (B,) tensor, as kept by SlotCache) limits request b to
    keys 0 ... kv_positions[b] (one or two queries: decode); ``actual_seq_lengths_kv`` (list
    of ints) limits it to that many keys at any query length; the mask, if any, is applied on
    top, as the reference's operator does (npu_attention.py:16-25)."""
    if module.training or kwargs.get('dropout', 0.0) != 0.0:
        raise ValueError('Native GQA is inference-only')
    if getattr(module, 'sliding_window', None) is not None:
        raise ValueError('Native GQA sliding-window masks are not implemented')
    batch, _, qlen, head_dim = query.shape
    ctx = key.shape[2]
    scale = kwargs.get('scaling', head_dim ** -0.5)
    positions = kwargs.get('kv_positions')
    lengths = kwargs.get('actual_seq_lengths_kv')
    device = query.device
    mask = attention_mask
    if positions is None:
        if lengths is not None:
            positions = _length_positions(lengths, device)
        else:
            positions = torch.full((batch,), ctx - 1, device=device, dtype=torch.int64)
        if mask is None and 1 < qlen <= 2 and getattr(module, 'is_causal', True):
            # the reference operator's default for several queries: query i sees keys 0 ... i
            mask = torch.ones(qlen, ctx, device=device, dtype=torch.bool).tril()
    if qlen <= 2:
        out = decode_attention(query.transpose(1, 2), key, value, positions, scale=scale, mask=mask)
        return out, None
    if kwargs.get('kv_positions') is not None:
        raise ValueError('kv_positions bounds one or two queries per request; for more, pass '
                         'actual_seq_lengths_kv or a mask')
    if mask is None and not getattr(module, 'is_causal', True):
        raise ValueError('non-causal prefill without a mask is not supported')
    # several queries per request on the MFMA kernel: without a mask, causal with request b's
    # queries at positions 0 ... qlen-1 (and keys below actual_seq_lengths_kv[b]); with one
    # (PrefillGraph's key-valid and causal mask, prefill_graph.py:36-37, or any other) every
    # key is scored and the mask decides, the key counts folded into it
    kv_lens = None
    if lengths is not None:
        if len(lengths) != batch:
            raise ValueError('actual_seq_lengths_kv needs one key count per request')
        if mask is None:
            kv_lens = _length_positions(lengths, device, counts=True)
        else:
            beyond = (torch.arange(ctx, device=device)[None, :]
                      >= _length_positions(lengths, device, counts=True)[:, None])[:, None, None, :]
            view = mask if mask.ndim == 4 else mask.view((1,) * (4 - mask.ndim) + tuple(mask.shape))
            if view.dtype == torch.bool:
                mask = view & ~beyond
            else:
                mask = view.masked_fill(beyond, torch.finfo(view.dtype).min)
    cu = _uniform_cu(batch, qlen, device)
    q = query.transpose(1, 2).reshape(batch * qlen, query.shape[1], head_dim)
    out = prefill_attention(q, key, value, cu, qlen, scale=scale, mask=mask, kv_lens=kv_lens)
    return out.view(batch, qlen, query.shape[1], head_dim), None


def prefill_attention(query, keys, values, cu_seqlens, max_seqlen, *, scale=None, kv_slots=None,
                      out=None, cos=None, sin=None, kv_lens=None, mask=None, new_values=None):
    """Varlen causal GQA: query (T, Hq, D) packed by cu_seqlens (B+1, int32); keys/values
    (slots, Hkv, capacity, D) arena views holding each request's keys at positions
    0 ... len-1 (slot b, or kv_slots[b]).  Returns (T, Hq, D).  With cos/sin (bf16 (T, D)
    rows of each token's position) the query rows are un-rotated and the kernel applies
    RoPE as it loads them (bf16-exact, as ``rotary``).

    ``kv_lens`` (int32 (B,), device): request b's queries see only its first kv_lens[b]
    keys (a right-padded batch: query i sees keys j <= i with j < kv_lens[b], the
    key-valid and causal mask of PrefillGraph.compute, prefill_graph.py:36-37).
    ``mask`` (B or 1, 1, len or 1, capacity): an SDPA-style mask (additive bf16 / fp16 /
    fp32, or bool with True = attend) over every key of the view; the causal rule is then
    off and the mask alone decides, as with the reference's explicit masks.  A query that
    sees no key gets a zero row.

    ``new_values`` (T, Hkv, D) bf16: the step's value rows as the projection wrote them
    (``prefill_rope_write(value=None)`` left them out of the arena): the products read them
    and the same launch copies each into ``values`` at its token's position.  Not with
    ``mask``."""
    if query.ndim != 3 or keys.ndim != 4 or values.shape != keys.shape:
        raise ValueError('expected (T, Hq, D) queries and arena key/value views')
    total, q_heads, head_dim = query.shape
    kv_heads = keys.shape[1]
    if query.dtype != torch.bfloat16 or keys.dtype != torch.bfloat16 or values.dtype != torch.bfloat16:
        raise ValueError('prefill attention is bf16-only')
    if cu_seqlens.dtype != torch.int32 or cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError('cu_seqlens must be an int32 (B+1,) tensor')
    if keys.shape[3] != head_dim or q_heads % kv_heads:
        raise ValueError('head_dim mismatch or q_heads not a multiple of kv_heads')
    if query.stride(2) != 1 or keys.stride(3) != 1 or values.stride(3) != 1:
        raise ValueError('rows must be unit-stride along head_dim')
    batch = cu_seqlens.numel() - 1
    if kv_slots is None and keys.shape[0] < batch:
        raise ValueError('the arena views have fewer slots than requests')
    device = _lib.require_gpu(query, keys, values, cu_seqlens)
    if out is None:
        out = torch.empty(total, q_heads, head_dim, device=device, dtype=query.dtype)
    else:
        _check_out(out, (total, q_heads, head_dim), query.dtype, device, 'prefill attention')
    a = _lib.PrefillArgs()
    a.batch, a.total_tokens, a.max_seqlen = batch, total, int(max_seqlen)
    a.q_heads, a.kv_heads, a.head_dim = q_heads, kv_heads, head_dim
    a.scale = head_dim ** -0.5 if scale is None else float(scale)
    a.cu_seqlens = cu_seqlens.data_ptr()
    a.query = query.data_ptr()
    a.q_stride_t, a.q_stride_h = query.stride()[:2]
    a.keys, a.values = keys.data_ptr(), values.data_ptr()
    a.k_stride_b, a.k_stride_h, a.k_stride_t = keys.stride()[:3]
    a.v_stride_b, a.v_stride_h, a.v_stride_t = values.stride()[:3]
    if kv_slots is not None:
        if kv_slots.dtype != torch.int64 or kv_slots.shape != (batch,):
            raise ValueError('kv_slots must be an int64 (B,) tensor')
        _lib.require_gpu(query, kv_slots)
        a.kv_slots = kv_slots.data_ptr()
    a.out = out.data_ptr()
    a.o_stride_t, a.o_stride_h = out.stride()[:2]
    a.capacity = keys.shape[2]
    if (cos is None) != (sin is None):
        raise ValueError('cos and sin come together')
    if cos is not None:
        if (cos.shape != (total, head_dim) or sin.shape != cos.shape or cos.dtype != torch.bfloat16
                or sin.dtype != torch.bfloat16 or cos.stride(1) != 1 or sin.stride() != cos.stride()):
            raise ValueError('cos/sin must be bf16 (tokens, head_dim) rows')
        _lib.require_gpu(query, cos, sin)
        a.cos, a.sin, a.cs_stride_t = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    if kv_lens is not None:
        if kv_lens.dtype != torch.int32 or kv_lens.shape != (batch,):
            raise ValueError('kv_lens must be an int32 (B,) tensor')
        _lib.require_gpu(query, kv_lens)
        a.kv_lens = kv_lens.data_ptr()
    if new_values is not None:
        if mask is not None:
            raise ValueError('new_values needs the causal rule: not with an explicit mask')
        if (new_values.ndim != 3 or tuple(new_values.shape) != (total, kv_heads, head_dim)
                or new_values.dtype != torch.bfloat16 or new_values.stride(2) != 1):
            raise ValueError(f'new_values must be bf16 ({total}, {kv_heads}, {head_dim}) token rows')
        _lib.require_gpu(query, new_values)
        a.new_values = new_values.data_ptr()
        a.nv_stride_t, a.nv_stride_h = new_values.stride()[:2]
    if mask is not None:
        m = _prefill_mask(mask.to(device), batch, int(max_seqlen), keys.shape[2])
        a.mask = m.data_ptr()
        a.mask_dtype = _lib.DTYPE_CODES[m.dtype]
        a.mask_stride_b, a.mask_stride_q = m.stride(0), m.stride(2)
    status = _lib.library().q3t_prefill_attention(a, _lib.stream_handle(device))
    _lib.check(status, 'prefill attention')
    return out


def _prefill_mask(mask, batch, queries, keys):
    """An SDPA-style (B or 1, 1, Lq or 1, Lk) mask as the kernel reads it: additive bf16 /
    fp16 / fp32 (bool: True = 0, False = -inf, in bf16), unit-stride keys, 16-byte aligned
    query rows (broadcast dimensions keep a zero stride)."""
    if mask.ndim == 2:
        mask = mask[None, None]
    elif mask.ndim == 3:
        mask = mask[:, None]
    if (mask.ndim != 4 or mask.shape[1] != 1 or mask.shape[0] not in (1, batch)
            or mask.shape[2] not in (1, queries) or mask.shape[3] != keys):
        raise ValueError('prefill mask must be (B or 1, 1, Lq or 1, Lk)')
    if mask.dtype == torch.bool:
        zero = torch.zeros((), dtype=torch.bfloat16, device=mask.device)
        mask = torch.where(mask, zero, torch.full_like(zero, float('-inf')))
    elif mask.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError('attention mask must be bool, bf16, fp16 or fp32')
    mask = mask.expand(batch, 1, queries, keys)
    es = mask.element_size()
    if (mask.stride(3) != 1 or (mask.stride(2) * es) % 16 or (mask.stride(0) * es) % 16
            or mask.data_ptr() % 16):
        mask = mask.contiguous()
        if (mask.stride(2) * es) % 16:
            raise ValueError('prefill masks need a key count whose rows are 16-byte multiples')
    return mask
