"""Drop-in ``PackedAttention`` for the Qwen3-TTS attention modules on the package's kernels.

Same plug-in mechanism as the reference (qwen3_tts_engine/packed_attention.py:11-95,
operators.py:36-38): ``install_packed_attention`` swaps every child whose class is named
``Qwen3TTSTalkerAttention`` or ``Qwen3TTSAttention`` for a ``PackedAttention`` wrapping it
and returns ``(parent, name, original)`` tuples for ``restore_modules``.  The constructor
takes the reference's flags with the same validation.

Forward, as the reference: one fused QKV projection, the module's own q/k RMSNorm, rotary
embedding, cache update, attention, o_proj.  Rotary and attention always run on the HIP
kernels (the flags that select the reference's Ascend operators are accepted for
signature compatibility):

* a one-token bf16 step over a ``SlotCache`` is a single ``decode_step`` launch: RoPE of q
  and k, the paired K/V write at the cache positions and ragged GQA attention over keys
  0 ... position, with the layer's mask (SlotGraph.compute's ``j <= pos[b]`` as 0 /
  finfo.min, continuous.py:191-192) added to the scores as the reference's operator does;
  rows past a request's position hold stale data and are never read;
* so is an unmasked one-token step s >= 1 of the code predictor over a ``PredictorCache``:
  it writes position s + 1 and attends positions 0 ... s + 1 (predictor.py:19-24, the
  unmasked steps of UniformPredictor.run, continuous.py:55-62), which is ``decode_step`` with
  every position at s + 1;
* and the predictor's first step, two tokens under the 2x2 causal mask (continuous.py:39-40,
  zeros with finfo.min above the diagonal, or no mask, which the attention treats as causal
  for two queries): ``decode_step`` writes positions 0 and 1 and attends them causally.  The
  mask's values are read once, outside graph capture, and the result is kept per mask
  tensor;
* every other call rotates q/k with ``rotary`` (bf16-exact to torch eager), lets the cache
  update and calls ``attention`` (the npu_attention.attention drop-in).

``fused_qk_norm=True`` (an extension, off by default) also moves the module's q_norm /
k_norm (RMSNorm over head_dim, packed_attention.py:42-45) into that fused launch: the raw
projection rows go in, and the per-layer chain of norm kernels disappears.  The norm's fp32
row sums then follow the kernel's order, so normalised rows can differ from the module's in
the last bf16 bit (the reference's own norm runs with yet another order on its device).
"""
from __future__ import annotations

import torch

from .attention import attention, decode_step, plan_shape, prefill_attention
from .prefill import prefill_rope_write
from .rotary import rotary
from .slots import PredictorCache, PrefillCache, SlotCache

_ATTENTION_CLASSES = ('Qwen3TTSTalkerAttention', 'Qwen3TTSAttention')

_CAUSAL_PAIR: dict = {}
_CAUSAL_PAIR_LIMIT = 64


def _is_causal_pair(mask, batch):
    """True if ``mask`` is the code predictor's first-step mask: (1 or batch, 1, 2, 2) with 0
    on and below the diagonal and a value at or below the dtype's finfo.min above it
    (continuous.py:39-40), or None (two queries without a mask attend causally,
    npu_attention.py:17-18).  The values are read on the host once per tensor version
    outside graph capture; during capture an unseen mask counts as not causal."""
    if mask is None:
        return True
    if (not isinstance(mask, torch.Tensor) or mask.ndim != 4 or mask.shape[0] not in (1, batch)
            or mask.shape[1:] != (1, 2, 2) or not mask.dtype.is_floating_point):
        return False
    key = (mask.data_ptr(), mask._version, tuple(mask.shape), tuple(mask.stride()), mask.dtype, mask.device)
    seen = _CAUSAL_PAIR.get(key)
    if seen is None:
        if mask.is_cuda and torch.cuda.is_current_stream_capturing():
            return False
        values = mask.detach().float().cpu()
        low = torch.finfo(mask.dtype).min
        causal = bool((values[..., 0, 0] == 0).all() and (values[..., 1, 0] == 0).all()
                      and (values[..., 1, 1] == 0).all() and (values[..., 0, 1] <= low).all())
        # the entry keeps the mask alive, so its address cannot be reused by another tensor;
        # the oldest entries go once a caller has shown many distinct masks
        if len(_CAUSAL_PAIR) >= _CAUSAL_PAIR_LIMIT:
            del _CAUSAL_PAIR[next(iter(_CAUSAL_PAIR))]
        seen = _CAUSAL_PAIR[key] = (causal, mask)
    return seen[0]


def _section_axes(head_dim, sections, interleaved, device):
    """Per-dimension axis (0 temporal, 1 height, 2 width) of a sectioned multimodal RoPE:
    consecutive sections of each half, or, interleaved, frequency f reads axis a in {1, 2}
    when f % 3 == a and f < 3 * sections[a] and the temporal axis otherwise (the Qwen3-Omni
    talker's layout, which qwen_tts's apply_multimodal_rotary_pos_emb applies at
    packed_attention.py:66-69)."""
    half = head_dim // 2
    if interleaved:
        axes = [0] * half
        for a in (1, 2):
            for f in range(a, min(half, 3 * sections[a]), 3):
                axes[f] = a
    else:
        axes = [i % 3 for i, n in enumerate(sections) for _ in range(n)]
    if len(axes) != half:
        raise ValueError('mrope sections must cover half of head_dim')
    return torch.tensor(axes + axes, device=device, dtype=torch.int64)


class PackedAttention(torch.nn.Module):
    def __init__(self, reference, native_gqa=False, text_only_rope=False, reference_single=False,
                 native_rope=False, native_rope_scope="all", triton_talker_rope=False,
                 fused_qk_norm=False):
        super().__init__()
        self.reference = reference
        projections = [reference.q_proj, reference.k_proj, reference.v_proj]
        self.sizes = [projection.out_features for projection in projections]
        self.weight = torch.nn.Parameter(torch.cat([p.weight.detach() for p in projections], dim=0),
                                         requires_grad=False)
        self.bias = None
        if projections[0].bias is not None:
            self.bias = torch.nn.Parameter(torch.cat([p.bias.detach() for p in projections], dim=0),
                                           requires_grad=False)
        self.multimodal = reference.__class__.__name__ == 'Qwen3TTSTalkerAttention'
        if native_rope_scope not in ('all', 'talker', 'predictor'):
            raise ValueError('Native rotary scope must be all, talker or predictor')
        self.native_rope = native_rope and (native_rope_scope == 'all'
                                            or (native_rope_scope == 'talker') == self.multimodal)
        if native_rope and self.multimodal and not text_only_rope:
            raise ValueError("Native rotary requires identical CustomVoice position axes")
        self.triton_talker_rope = triton_talker_rope and self.multimodal
        if self.triton_talker_rope and not text_only_rope:
            raise ValueError("Triton talker rotary requires identical CustomVoice position axes")
        self.native_gqa = native_gqa
        self.reference_single = reference_single
        self.text_only_rope = text_only_rope
        self._axes = None
        self._norms = self._fusable_norms(reference) if fused_qk_norm else None

    @staticmethod
    def _fusable_norms(reference):
        """(q weight, k weight, eps) when both norms are plain RMSNorms over head_dim with bf16
        weights and one epsilon, else None (the module's own norms run)."""
        norms = []
        for norm in (reference.q_norm, reference.k_norm):
            weight = getattr(norm, 'weight', None)
            eps = getattr(norm, 'variance_epsilon', getattr(norm, 'eps', None))
            if (weight is None or eps is None or weight.dtype != torch.bfloat16
                    or tuple(weight.shape) != (reference.head_dim,)):
                return None
            norms.append((weight, float(eps)))
        if norms[0][1] != norms[1][1]:
            return None
        return norms[0][0], norms[1][0], norms[0][1]

    def _tables(self, position_embeddings, batch, length):
        """cos/sin as contiguous (batch, length, head_dim) rows."""
        cos, sin = position_embeddings
        if self.multimodal:
            if self.text_only_rope:
                cos, sin = cos[0], sin[0]
            else:
                scaling = self.reference.rope_scaling
                if self._axes is None or self._axes.device != cos.device:
                    self._axes = _section_axes(cos.shape[-1], scaling['mrope_section'],
                                               scaling.get('interleaved', False), cos.device)
                index = self._axes.view(1, 1, 1, -1).expand(1, *cos.shape[1:])
                cos, sin = cos.gather(0, index)[0], sin.gather(0, index)[0]
        cos = cos.expand(batch, length, cos.shape[-1]).contiguous()
        sin = sin.expand(batch, length, sin.shape[-1]).contiguous()
        return cos, sin

    def _fused_target(self, cache, attention_mask, batch, length, query):
        """(keys, values, positions, mask, plan) of a step the fused launch can take, else None
        (plan: the slot cache's plan of the step's requests, SlotCache.prepare).

        The mask the layer is given is applied in the launch (the reference's operator applies
        it, npu_attention.py:16-25), except the predictor's first-step 2x2 causal mask, which
        is recognised and applied as the causal rule of two queries."""
        reference = self.reference
        if (length not in (1, 2) or reference.training or query.dtype != torch.bfloat16
                or reference.head_dim != 128):
            return None
        layer = reference.layer_idx
        if length == 2:
            if (isinstance(cache, PredictorCache) and cache.step == 0
                    and _is_causal_pair(attention_mask, batch)):
                keys, values = cache.keys[layer], cache.values[layer]
                if (keys.is_contiguous() and values.is_contiguous() and keys.shape[0] == batch
                        and keys.shape[2] >= 2):
                    return keys, values, cache.positions_at(batch, 1, query.device), None, None
            return None
        if attention_mask is not None and not isinstance(attention_mask, torch.Tensor):
            return None
        if isinstance(cache, SlotCache):
            keys, values = cache.arena.keys[layer], cache.arena.values[layer]
            if keys.is_contiguous() and values.is_contiguous():
                return keys, values, cache.positions, attention_mask, cache.plan
        elif isinstance(cache, PredictorCache) and cache.step >= 1:
            keys, values = cache.keys[layer], cache.values[layer]
            if (keys.is_contiguous() and values.is_contiguous() and keys.shape[0] == batch
                    and cache.step + 1 < keys.shape[2]):
                return keys, values, cache.positions_at(batch, cache.step + 1, query.device), attention_mask, None
        return None

    def _prefill(self, query, key, value, cos, sin, cache, batch, length):
        """One layer of a padded prefill batch (PrefillGraph): the module's q/k norms, then the
        prologue kernel rotating the keys into this layer's planes of the packed cache, then
        causal attention over each row's valid keys with the queries rotated in the kernel and
        the values read from the projection (the same launch copies them into the cache).  The layer's mask is not needed: the rows are
        right-padded prompts and the cache carries their lengths."""
        reference = self.reference
        if reference.training:
            raise ValueError('Native GQA is inference-only')
        if query.dtype != torch.bfloat16:
            raise ValueError('padded prefill through PackedAttention is bf16-only')
        tokens, width = batch * length, reference.head_dim
        planes = cache.layers[reference.layer_idx]
        q = reference.q_norm(query).reshape(tokens, -1, width)
        k = reference.k_norm(key).reshape(tokens, -1, width)
        v = value.reshape(tokens, -1, width)
        c, s = cos.reshape(tokens, width), sin.reshape(tokens, width)
        prefill_rope_write(q, k, None, c, s, cache.cu_seqlens, planes.keys, planes.values, rotate_query=False)
        out = prefill_attention(q, planes.keys, planes.values, cache.cu_seqlens, length,
                                scale=reference.scaling, cos=c, sin=s, kv_lens=cache.kv_lens, new_values=v)
        return reference.o_proj(out.view(batch, length, -1))

    def forward(self, hidden_states, position_embeddings, attention_mask, past_key_values=None,
                cache_position=None, **kwargs):
        reference = self.reference
        shape = hidden_states.shape[:-1]
        batch, length = shape[0], shape[1]
        heads = (*shape, -1, reference.head_dim)
        projected = torch.nn.functional.linear(hidden_states, self.weight, self.bias)
        query, key, value = projected.split(self.sizes, dim=-1)
        query, key, value = query.reshape(heads), key.reshape(heads), value.reshape(heads)  # BSND
        cos, sin = self._tables(position_embeddings, batch, length)

        if isinstance(past_key_values, PrefillCache):
            return self._prefill(query, key, value, cos, sin, past_key_values, batch, length), None

        fused = self._fused_target(past_key_values, attention_mask, batch, length, query)
        if fused is not None:
            keys, values, positions, mask, plan = fused
            if plan is not None and tuple(plan.shape) != plan_shape(batch, query.shape[2], key.shape[2]):
                plan = None  # a plan of another batch (a graph bucket the cache was not prepared for)
            if self._norms is not None and self._norms[0].device == query.device:
                q_weight, k_weight, eps = self._norms
                output = decode_step(query, key, value, keys, values, positions, cos, sin,
                                     scale=reference.scaling, q_norm_weight=q_weight,
                                     k_norm_weight=k_weight, norm_eps=eps, mask=mask, plan=plan)
            else:
                output = decode_step(reference.q_norm(query), reference.k_norm(key), value, keys, values,
                                     positions, cos, sin, scale=reference.scaling, mask=mask, plan=plan)
            return reference.o_proj(output.reshape(*shape, -1)), None

        query = reference.q_norm(query)
        key = reference.k_norm(key)

        query = rotary(query.contiguous(), cos, sin).transpose(1, 2)
        key = rotary(key.contiguous(), cos, sin).transpose(1, 2)
        value = value.transpose(1, 2)
        if past_key_values is not None:
            key, value = past_key_values.update(key, value, reference.layer_idx,
                                                {'sin': sin, 'cos': cos, 'cache_position': cache_position})
        if isinstance(past_key_values, SlotCache):
            kwargs['kv_positions'] = past_key_values.positions
        else:
            lengths = getattr(past_key_values, 'actual_seq_lengths_kv', None)
            if lengths is not None:
                kwargs['actual_seq_lengths_kv'] = lengths
        output, weights = attention(reference, query, key, value, attention_mask,
                                    dropout=0.0 if not reference.training else reference.attention_dropout,
                                    scaling=reference.scaling, sliding_window=reference.sliding_window,
                                    **kwargs)
        return reference.o_proj(output.reshape(*shape, -1).contiguous()), weights


def install_packed_attention(model, native_gqa=False, text_only_rope=False, reference_single=False,
                             native_rope=False, native_rope_scope="all", triton_talker_rope=False,
                             fused_qk_norm=False):
    """Swap every Qwen3-TTS attention module of ``model`` for a PackedAttention."""
    replacements = []
    for parent in list(model.modules()):
        for name, child in list(parent.named_children()):
            if child.__class__.__name__ in _ATTENTION_CLASSES:
                replacements.append((parent, name, child))
                setattr(parent, name, PackedAttention(
                    child, native_gqa=native_gqa, text_only_rope=text_only_rope,
                    reference_single=reference_single, native_rope=native_rope,
                    native_rope_scope=native_rope_scope, triton_talker_rope=triton_talker_rope,
                    fused_qk_norm=fused_qk_norm))
    return replacements


def restore_modules(replacements):
    """Undo install_packed_attention (latest replacement first)."""
    for parent, name, original in reversed(replacements):
        setattr(parent, name, original)
