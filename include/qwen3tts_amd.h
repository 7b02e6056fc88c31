/*
 * qwen3tts_amd.h - C ABI of the MI355X (gfx950) continuous-batching attention path.
 *
 * Every entry point takes plain device pointers, element strides and sizes, and an
 * optional HIP stream (`void *stream`, a hipStream_t; NULL = the legacy default stream).
 * Nothing here allocates device memory, synchronises the host or touches PyTorch, so
 * every call may be captured into a HIP graph.  Arguments are validated on the host
 * before anything is launched: a rejected call returns a negative status and writes
 * nothing.  A positive status is the hipError_t reported by the launch.
 *
 * Layouts follow the reference engine (InferMatrixLab/qwen3-tts-rsi-engine):
 *   - KV arena per layer: (slots, kv_heads, capacity, head_dim), contiguous rows;
 *     the packed arena stacks 2*layers of them, keys first
 *     (qwen3_tts_engine/continuous.py:107-113).
 *   - Queries and new keys/values are BSND rows of the fused QKV projection
 *     (qwen3_tts_engine/packed_attention.py:42-45), passed with explicit strides.
 *
 * Strides are in ELEMENTS, never bytes.
 */
#ifndef QWEN3TTS_AMD_H
#define QWEN3TTS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------ */
#define Q3T_OK 0
#define Q3T_EINVAL (-1)        /* malformed argument (null pointer, bad size or stride)    */
#define Q3T_EUNSUPPORTED (-2)  /* well-formed but outside the compiled kernel variants      */
#define Q3T_EWORKSPACE (-3)    /* workspace pointer missing or too small                     */

/* ---- element types ----------------------------------------------------------------- */
#define Q3T_BF16 0
#define Q3T_F16 1
#define Q3T_F32 2
#define Q3T_BOOL 3  /* masks only: nonzero = attend, as a torch bool SDPA mask */

/* Human-readable text for a status returned by any entry point.  The reference's wrappers
   raise ValueError with such a text before launching (kv_triton_ascend.py:40-53); the
   Python bindings here do the same with this string. */
const char *q3t_status_string(int status);

/* ABI revision of this header (8); bumps on any incompatible change.  No counterpart in the
   reference (its operators are Python functions); the bindings refuse another revision. */
int q3t_abi_version(void);

/* ---- KV arena writes and copies ------------------------------------------------------ */

/*
 * Paired K/V write of `tokens` new rows per request into a slot arena:
 *   target_keys  [b, h, positions[b] + t, :] = keys  [b, h, t, :]
 *   target_values[b, h, positions[b] + t, :] = values[b, h, t, :]
 * for b < batch, h < heads, t < tokens.  Bit-exact copy of `elem_size`-byte elements.
 * Source strides (b, h, t) are free (the fused QKV row stride is (Hq+2*Hkv)*D);
 * the last dimension must be unit-stride.  Targets are (batch, heads, capacity, width)
 * with strides (b, h, s) given in target_strides.  Rows whose position falls outside
 * [0, capacity) are skipped on the device (the reference leaves them undefined).
 *
 * Replaces: SlotCache.update's scatter_ / npu_scatter_nd_update_ (continuous.py:152-166),
 * kv_triton_ascend.write (kv_triton_ascend.py:39-64), PredictorCache.update
 * (predictor.py:19-24) with tokens = 2 at step 0.
 */
int q3t_kv_write(const void *keys, const void *values, void *target_keys, void *target_values,
                 const int64_t *positions, int64_t batch, int64_t heads, int64_t tokens,
                 int64_t width, int64_t elem_size, const int64_t key_strides[3],
                 const int64_t value_strides[3], const int64_t target_strides[3],
                 int64_t capacity, void *stream);

/*
 * Strided element copy over up to 5 dimensions: dst[i...] = src[i...].
 * Used for the packed prefix copy, slot compaction and arena regrowth.
 * Replaces: copy_packed_prefix (packed_kv.py:6-31), SlotArena.load / move
 * (continuous.py:118-128), ensure_capacity's copy (continuous.py:362-363).
 */
int q3t_copy_strided(void *dst, const void *src, int64_t elem_size, int ndim,
                     const int64_t *sizes, const int64_t *dst_strides,
                     const int64_t *src_strides, void *stream);

/* Plain contiguous byte copy: the calibration kernel for the HBM byte counters (a copy of
   known size).  No counterpart in the reference; slot moves go through q3t_copy_strided. */
int q3t_copy_bytes(void *dst, const void *src, int64_t nbytes, void *stream);

/* ---- rotary position embedding ------------------------------------------------------ */

/*
 * Rotate-half RoPE on BSND rows with torch-eager rounding (Q3T_BF16 or Q3T_F32):
 *   bf16: y1 = bf16(bf16(x1*c1) + bf16(-x2*s1)),  y2 = bf16(bf16(x2*c2) + bf16(x1*s2))
 *   fp32: the same with every product and sum rounded to fp32 separately (no FMA)
 * x, y: (rows, heads, width) contiguous; cos, sin: (rows, width) contiguous, same dtype.
 * width in {64, 128}.  Replaces: rotary_triton_ascend.rotary (rotary_triton_ascend.py:29-44)
 * and apply_rotary_pos_emb on the talker's equal-axis positions (packed_attention.py:62-65).
 */
int q3t_rotary(const void *x, const void *cos, const void *sin, void *y, int64_t rows,
               int64_t heads, int64_t width, int64_t dtype, void *stream);

/*
 * Default-RoPE cos/sin tables: for n positions and width = 2*half,
 *   f = inv_freq[i] * (float)positions[r];  cos[r, i] = cos[r, i + half] = cos(f)*scaling
 * (same for sin), stored as dtype (Q3T_BF16, rounded to nearest even, or Q3T_F32).
 * inv_freq is a device fp32 array of `half` entries computed by the caller.
 * Replaces: the talker rotary_emb cos/sin (continuous.py:193, prefill_graph.py:38).
 */
int q3t_rope_tables(const int64_t *positions, int64_t n, const float *inv_freq, int64_t half,
                    float scaling, int64_t dtype, void *cos, void *sin, void *stream);

/* ---- attention ----------------------------------------------------------------------- */

/*
 * Ragged grouped-query decode attention over a slot arena.
 * Request b has query_len queries at positions p_b - query_len + 1 ... p_b, where
 * p_b = positions[b]; keys 0 ... p_b of its slot are read (the reference's additive mask
 * `j <= pos[b]`, continuous.py:191-192).  Without a mask, query i attends keys
 * 0 ... p_b - query_len + 1 + i (the predictor's 2x2 causal step, continuous.py:39-40);
 * with a mask (batch, query_len, ctx) the mask alone decides, added to the scaled scores
 * as SDPA does (bool masks: nonzero attends).  Requests with p_b outside [0, ctx) attend
 * nothing and get zero rows.  Query head hq reads KV head hq / (q_heads / kv_heads).
 *
 * Three grids compute the same result (to rounding; `grid` picks one, Q3T_GRID_*):
 *   - bundled: one workgroup per CU, streaming keys through LDS and scoring them on bf16
 *     MFMA tiles.  Each workgroup takes whole requests of one KV head, longest paired with
 *     shortest, as the step's `plan` (q3t_decode_plan) bundles them or, without one, as the
 *     workgroup ranks them itself.  A mask needs unit key stride and 4-byte alignment (bf16
 *     masks take a branch-free path).  bf16, head_dim 128, query_len 1,
 *     q_heads / kv_heads <= 4, batch <= 128.  The default when batch * kv_heads is
 *     192..511 from ctx >= 512, 512 or more from ctx >= 1024 (the talker step), and 384 or
 *     more from ctx >= 4096.
 *   - balanced (`splits` workgroups per KV head): the concatenated keys of all requests of a
 *     head cut into equal shares, one per workgroup; the default otherwise for ctx >= 2048.
 *   - chunked: each request's keys cut into chunks of 64-key blocks (at most `max_chunks`
 *     per request), one workgroup per (request, chunk, KV head); the default otherwise (the
 *     code predictor's 16-row caches, short arenas, few requests).
 * A request covered by several workgroups (balanced, chunked) merges their partial softmax
 * states through `workspace`; the last workgroup to finish writes the output.
 *
 * fused != 0 additionally performs, for query_len S in {1, 2} (the step's tokens sit at
 * positions p_b - S + 1 ... p_b):
 *   - RoPE of the query rows and of the new keys with each token's cos/sin row (bf16-exact,
 *     as q3t_rotary),
 *   - the paired K/V write of the new (rotated) keys and values at those positions,
 * and uses the new keys/values for those key positions without re-reading the arena; with
 * S == 2, query token 0 does not attend key p_b (the code predictor's first step with its
 * 2x2 causal mask, continuous.py:39-40).  Then `query`, `new_key`, `new_value` are the
 * un-rotated BSND rows of the QKV projection.
 * Replaces: PackedAttention.forward's RoPE + cache update + attention dispatch
 * (packed_attention.py:46-84), npu_attention.attention (npu_attention.py:11-26).
 */
typedef struct q3t_decode_args {
    /* sizes */
    int64_t batch, query_len, q_heads, kv_heads, head_dim;
    int64_t ctx;        /* keys addressable per slot (arena capacity or context view) */
    int64_t dtype;      /* Q3T_BF16 or Q3T_F32 (fused requires Q3T_BF16) */
    float scale;        /* softmax scale, normally head_dim ** -0.5 */
    int32_t fused;
    /* query (batch, query_len, q_heads, head_dim) */
    const void *query;
    int64_t q_stride_b, q_stride_s, q_stride_h;
    /* arena views for this layer: key (b, h, j) at base + off_b + h*stride_h + j*stride_t,
       off_b = kv_offsets ? kv_offsets[b] : b*stride_b (elements) */
    void *keys, *values;
    int64_t k_stride_b, k_stride_h, k_stride_t;
    int64_t v_stride_b, v_stride_h, v_stride_t;
    const int64_t *kv_offsets; /* optional, device, (batch,) */
    const int64_t *positions;  /* device, (batch,): last query position p_b */
    /* optional additive mask (batch, query_len, ctx); dtype = mask_dtype; NULL = none */
    const void *mask;
    int64_t mask_dtype, mask_stride_b, mask_stride_s, mask_stride_t;
    /* output (batch, query_len, q_heads, head_dim), same dtype as query */
    void *out;
    int64_t o_stride_b, o_stride_s, o_stride_h;
    /* fused only: new key/value rows (batch, S, kv_heads, head_dim) and cos/sin
       (batch, S, head_dim); the token strides are the last fields below */
    const void *new_key, *new_value;
    int64_t nk_stride_b, nk_stride_h, nv_stride_b, nv_stride_h;
    const void *cos, *sin;
    int64_t cs_stride_b;
    /* workspace (chunked and balanced grids): a fixed 256 KiB counter region
       (kv_heads * batch <= 65536), then the partial states of split requests; zero-filled
       before first use, its counters left zeroed by every launch.  Launches that overlap in
       time must not share one.  The bundled grid uses none (may be NULL). */
    void *workspace;
    int64_t workspace_bytes;
    int64_t max_chunks;      /* chunked grid: chunks per request and KV head, <= 1024; <= 0:
                                enough for about 512 workgroups over the batch */
    /* fused only, optional: RMSNorm of the query rows / the new key rows before RoPE (the
       q_norm / k_norm of the attention module, packed_attention.py:42-45):
       bf16(weight * bf16(x * rsqrt(mean(x^2) + norm_eps))) with the fp32 sum of squares of a
       row; weights are bf16 (head_dim,); NULL = that row is used as given */
    const void *q_norm_weight, *k_norm_weight;
    float norm_eps;
    /* fused, S == 2: token strides of new_key, new_value and cos/sin (elements) */
    int64_t nk_stride_s, nv_stride_s, cs_stride_s;
    /* balanced grid: workgroups per KV head (<= 32768; fewer run when the keys are few: at
       least 32 keys per workgroup); 0: 256 workgroups in all.  With grid == Q3T_GRID_AUTO,
       splits > 0 selects the balanced grid and splits < 0 the chunked grid. */
    int64_t splits;
    /* Q3T_GRID_AUTO (0), Q3T_GRID_CHUNKED, Q3T_GRID_BALANCED or Q3T_GRID_BUNDLED; a grid the
       call does not qualify for returns Q3T_EUNSUPPORTED */
    int64_t grid;
    /* bundled grid, optional: the plan q3t_decode_plan wrote for these `positions`, `batch`,
       `ctx` and `kv_heads` (device, q3t_decode_plan_bytes): the launch takes whole requests
       as the plan bundles them instead of ranking and pairing them itself.  A plan made for
       other positions gives wrong outputs, and a fused launch then writes the new K/V rows
       at the rows the plan names (the last key of each request it lists), never outside the
       arena.  One made for another batch is not used (the launch ranks by itself).
       Ignored by the other grids. */
    const int32_t *plan;
} q3t_decode_args;

enum { Q3T_GRID_AUTO = 0, Q3T_GRID_CHUNKED = 1, Q3T_GRID_BALANCED = 2, Q3T_GRID_BUNDLED = 3 };

/* Bytes of workspace q3t_decode_attention needs for this call (its sizes, `fused`, `mask`,
   `max_chunks`, `splits` and `grid`; pointers are not read), 0 on the bundled grid; -1 for
   malformed sizes.  No
   counterpart in the reference (its attention operator allocates internally); callers size
   the buffer once, outside graph capture. */
int64_t q3t_decode_workspace_bytes(const q3t_decode_args *args);

int q3t_decode_attention(const q3t_decode_args *args, void *stream);

/* The grid q3t_decode_attention would run this call on (Q3T_GRID_CHUNKED, _BALANCED or
   _BUNDLED), from its sizes, `mask`, `splits` and `grid`; Q3T_EUNSUPPORTED when a named grid
   does not take the call, Q3T_EINVAL for malformed sizes.  No counterpart in the reference
   (its operator has one implementation). */
int q3t_decode_grid(const q3t_decode_args *args);

/* q3t_decode_attention without a caller workspace, for callers that cannot allocate device
   memory (code under graph capture that may not call hipMalloc, tight serving loops,
   harnesses that forbid allocation).  No counterpart in the reference.  `workspace` and
   `workspace_bytes` are ignored: the library uses its own fixed 8 MiB device array, one
   per GPU, held until the process ends (its counters are cleared on the first call on a
   device, on that call's stream).  A call that would need more than 8 MiB
   (q3t_decode_workspace_bytes) returns Q3T_EWORKSPACE and launches nothing.  It calls no
   allocating routine.  Every call on one GPU shares that GPU's array: calls that overlap in
   time on one GPU (on two streams) race. */
int q3t_decode_attention_static(const q3t_decode_args *args, void *stream);

/* The bundled grid's plan of a step, written once per step and passed as `plan` to every
   layer's launch of that step (the talker's layers all attend the same lengths).  With
   L_b = positions[b] + 1 for a position in [0, ctx) and 0 otherwise, and M =
   max(ceil(256 / kv_heads), ceil(batch / 4)) workgroups (bundles) per KV head, one per CU:
   plan[0] = batch, plan[1] = M, then for each bundle m four (b, L_b) int32 pairs ((-1, 0):
   none), every request of the batch listed once: bundle m holds the requests of length ranks
   m, 2M-1-m, 2M+m and 4M-1-m (longest first, ties by ascending b), so the i-th longest
   request shares a workgroup with the i-th shortest.  batch <= 128, ctx <= 2^20,
   q_heads / kv_heads <= 4; `plan` holds q3t_decode_plan_bytes bytes (16-byte aligned).
   One small kernel on `stream`; it may be captured.  No counterpart in the reference (its
   attention operator takes no per-step state; positions are fixed for a step's layers in
   SlotGraph.compute, continuous.py:188-198). */
int q3t_decode_plan(const int64_t *positions, int64_t batch, int64_t ctx, int64_t q_heads, int64_t kv_heads,
                    int32_t *plan, void *stream);

/* Bytes of the plan q3t_decode_plan writes for this launch shape; -1 for a shape it does not
   plan.  No counterpart in the reference. */
int64_t q3t_decode_plan_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads);

/* Re-zero the counter region of a decode workspace on `stream` (a kernel, so it may be
   captured).  Every completed launch leaves the counters zeroed; a launch that failed
   part-way may not, and the next launch that splits a request would then miscount.  No
   counterpart in the reference (its operator keeps no state between calls). */
int q3t_decode_reset_workspace(void *workspace, int64_t workspace_bytes, void *stream);

/*
 * Varlen causal prefill attention with GQA on bf16 MFMA tiles.
 * Requests are packed along the token axis by cu_seqlens (batch + 1, int32, device):
 * query rows (tokens, q_heads, head_dim); key/value rows are read from the slot arena
 * (slot = kv_slots ? kv_slots[b] : b) at positions 0 ... len_b - 1, with strides as in
 * q3t_decode_args.  Query token i of request b attends keys 0 ... i (keys at or past
 * `capacity` do not exist), and with kv_lens only keys below kv_lens[b]: the padded
 * batch of PrefillGraph.compute, whose mask is key-valid and causal (prefill_graph.py:36-37),
 * is len_b = the padded length with kv_lens[b] = the prompt's length.  With a mask
 * (batch, 1, len_b, capacity) the causal rule is off: every key 0 ... capacity - 1 is scored
 * and the mask is added to the scaled scores, as SDPA adds an attention mask (the drop-in
 * path for any mask).  A query that sees no key gets a zero row.  max_seqlen bounds len_b;
 * query blocks past it are not computed.  bf16 only; head_dim 64 or 128;
 * q_heads / kv_heads in {1, 2, 4}.
 * Replaces: PrefillGraph.compute's padded causal attention (prefill_graph.py:31-50).
 */
typedef struct q3t_prefill_args {
    int64_t batch, total_tokens, max_seqlen, q_heads, kv_heads, head_dim;
    float scale;
    const int32_t *cu_seqlens;     /* device (batch + 1), non-decreasing */
    const void *query;             /* (tokens, q_heads, head_dim) bf16 */
    int64_t q_stride_t, q_stride_h;
    const void *keys;              /* arena views; `values` is written only with new_values */
    void *values;
    int64_t k_stride_b, k_stride_h, k_stride_t;
    int64_t v_stride_b, v_stride_h, v_stride_t;
    const int64_t *kv_slots;       /* optional device (batch,) */
    void *out;                     /* (tokens, q_heads, head_dim) bf16 */
    int64_t o_stride_t, o_stride_h;
    int64_t capacity;              /* key rows per slot in the arena views */
    /* optional bf16 cos/sin rows (tokens, head_dim) of each query token's position: the
       query rows are then un-rotated and RoPE (bf16-exact, as q3t_rotary) is applied as
       they are loaded, so no rotated copy of the queries is written; NULL = the query rows
       are already rotated */
    const void *cos, *sin;
    int64_t cs_stride_t;
    /* optional device (batch,) int32: keys of each request (right-padded batches) */
    const int32_t *kv_lens;
    /* optional additive mask, element (b, 0, i, j) at mask + b*mask_stride_b +
       i*mask_stride_q + j (elements); Q3T_BF16, Q3T_F16 or Q3T_F32 (bool masks are passed as
       0 / -inf); 16-byte aligned rows */
    const void *mask;
    int64_t mask_dtype, mask_stride_b, mask_stride_q;
    /* optional bf16 value rows (tokens, kv_heads, head_dim) of the step's tokens as the
       projection wrote them (strides in elements, 16-byte aligned): the products read key
       j's value of request b from token cu_seqlens[b] + j instead of `values`, and the
       launch copies every token's row into `values` at its position (rows < capacity), the
       value half of q3t_prefill_rope_write (which then runs with value == NULL).  Causal
       launches only (mask == NULL): Q3T_EINVAL with a mask. */
    const void *new_values;
    int64_t nv_stride_t, nv_stride_h;
} q3t_prefill_args;

int q3t_prefill_attention(const q3t_prefill_args *args, void *stream);

/*
 * Prefill prologue: RoPE of packed query/key rows at positions 0 ... len_b - 1 (cos/sin
 * rows indexed by token) and the paired write of rotated keys and raw values into the
 * arena slot of each request.  q_out receives the rotated queries; with q_out == NULL only
 * the keys and values are handled (query and its strides are then ignored) and
 * q3t_prefill_attention rotates the queries itself from its cos/sin arguments.  With
 * value == NULL only the keys are written (value, its strides and arena_values are ignored):
 * q3t_prefill_attention then copies the values (its new_values).
 * Replaces: the per-layer RoPE + DynamicCache fill of PrefillGraph.compute
 * (prefill_graph.py:38-43) and the later copy_packed_prefix into the arena
 * (continuous.py:468-469).
 */
typedef struct q3t_prefill_rope_write_args {
    int64_t batch, total_tokens, q_heads, kv_heads, head_dim, capacity;
    const int32_t *cu_seqlens;
    const void *query; int64_t q_stride_t, q_stride_h;
    const void *key;   int64_t k_stride_t, k_stride_h;
    const void *value; int64_t v_stride_t, v_stride_h;
    const void *cos, *sin; int64_t cs_stride_t;
    void *q_out; int64_t qo_stride_t, qo_stride_h;
    void *arena_keys, *arena_values;
    int64_t a_stride_b, a_stride_h, a_stride_t;
    const int64_t *kv_slots;
} q3t_prefill_rope_write_args;

int q3t_prefill_rope_write(const q3t_prefill_rope_write_args *args, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN3TTS_AMD_H */
