"""CPU oracle of the continuous-batching attention path - TEST INFRASTRUCTURE ONLY.

A restatement, in numpy (and torch-CPU for the timed baseline), of what the reference
engine (InferMatrixLab/qwen3-tts-rsi-engine) computes on this path.  Each function cites
the reference file:line it follows.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg may import this package, and only to check results or as
the timed CPU baseline; the product path (the ``qwen3-tts-rsi-engine_amd`` package) never
calls it.

How each part is pinned (checked by tests/test_oracle.py, never by retyping a formula):
  bf16       rounding vs torch's own bf16 casts (exhaustive over special values + random)
  kv         the reference's test fixtures (tests/test_packed_kv.py arange tensors,
             tests/test_slot_context.py seed-42 arenas) and the closed forms they state
  rope       bit-exact vs torch-eager bf16/fp32 apply_rotary_pos_emb; the equal-axes MRoPE
             identity of tests/test_text_rope.py; position 0 is the identity; norm
             preservation in float64; the complex-multiplication form
  attention  torch-CPU scaled_dot_product_attention (repeat-KV GQA, additive and bool
             masks); brute-force loops on tiny inputs; closed forms (one key -> V row,
             equal scores -> mean of V, a dominant score -> its V row); trimmed context
             == full arena under the mask (tests/test_slot_context.py)
  scheduler  decode_batch_size known answers and invariants of tests/test_batching.py;
             capacity-rule and compaction invariants
"""
