"""Stand-in Qwen3-TTS talker with the attribute surface the drop-ins read.

``qwen_tts`` and the weights are not available, so the decoder layers here carry only what
the attention path touches: an input RMSNorm, a ``Qwen3TTSTalkerAttention`` (q/k/v/o
projections, q/k RMSNorm over head_dim, head_dim, layer_idx, scaling, rope_scaling) and the
residual add; the MLP of a real decoder layer is not on the path and is left out.  The
rotary module returns the (3, batch, length, head_dim) cos/sin tables of the default RoPE
with theta 1e6 for the three (equal, CustomVoice) position axes.  Weights are seeded random
bf16.
"""
import torch


class RMSNorm(torch.nn.Module):
    def __init__(self, width, eps=1e-6, scale=1.0, dtype=torch.bfloat16):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.full((width,), scale, dtype=dtype))
        self.eps = eps

    def forward(self, x):
        y = x.float()
        y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * y.to(x.dtype)


class _Config:
    _attn_implementation = 'sdpa'


class Qwen3TTSTalkerAttention(torch.nn.Module):
    def __init__(self, layer_idx, hidden, q_heads, kv_heads, head_dim, gen, dtype=torch.bfloat16):
        super().__init__()
        self.head_dim, self.layer_idx, self.scaling = head_dim, layer_idx, head_dim ** -0.5
        self.sliding_window, self.attention_dropout, self.is_causal = None, 0.0, True
        self.config = _Config()
        self.rope_scaling = {'mrope_section': [24, 20, 20], 'interleaved': False}
        self.q_proj = torch.nn.Linear(hidden, q_heads * head_dim, bias=False, dtype=dtype)
        self.k_proj = torch.nn.Linear(hidden, kv_heads * head_dim, bias=False, dtype=dtype)
        self.v_proj = torch.nn.Linear(hidden, kv_heads * head_dim, bias=False, dtype=dtype)
        self.o_proj = torch.nn.Linear(q_heads * head_dim, hidden, bias=False, dtype=dtype)
        with torch.no_grad():
            for p in (self.q_proj, self.k_proj, self.v_proj, self.o_proj):
                p.weight.copy_((torch.randn(p.weight.shape, generator=gen) * p.in_features ** -0.5).to(dtype))
        self.q_norm, self.k_norm = RMSNorm(head_dim, scale=1.5, dtype=dtype), RMSNorm(head_dim, scale=1.5, dtype=dtype)

    def forward(self, *args, **kwargs):  # replaced by PackedAttention before use
        raise NotImplementedError


class DecoderLayer(torch.nn.Module):
    def __init__(self, layer_idx, hidden, q_heads, kv_heads, head_dim, gen, dtype=torch.bfloat16):
        super().__init__()
        self.input_layernorm = RMSNorm(hidden, dtype=dtype)
        self.self_attn = Qwen3TTSTalkerAttention(layer_idx, hidden, q_heads, kv_heads, head_dim, gen, dtype)

    def forward(self, hidden_states, attention_mask=None, position_ids=None, past_key_values=None,
                output_attentions=False, use_cache=True, cache_position=None, position_embeddings=None):
        attended, _ = self.self_attn(hidden_states=self.input_layernorm(hidden_states),
                                     position_embeddings=position_embeddings,
                                     attention_mask=attention_mask, past_key_values=past_key_values,
                                     cache_position=cache_position)
        return (hidden_states + attended,)


class RotaryEmbedding(torch.nn.Module):
    def __init__(self, head_dim, theta=1e6):
        super().__init__()
        self.register_buffer('inv_freq', 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)),
                             persistent=False)

    def forward(self, x, position_ids):
        freqs = position_ids[..., None].float() * self.inv_freq.to(x.device)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


class Talker(torch.nn.Module):
    def __init__(self, layers=28, hidden=2048, q_heads=16, kv_heads=8, head_dim=128, seed=0,
                 dtype=torch.bfloat16):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.config = type('TalkerConfig', (), {'hidden_size': hidden, 'num_key_value_heads': kv_heads,
                                                'head_dim': head_dim, 'num_hidden_layers': layers})()
        self.layers = torch.nn.ModuleList(DecoderLayer(i, hidden, q_heads, kv_heads, head_dim, gen, dtype)
                                          for i in range(layers))
        self.rotary_emb = RotaryEmbedding(head_dim)
        self.norm = RMSNorm(hidden, dtype=dtype)
