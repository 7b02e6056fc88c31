// The parameter block of the decode attention launches (every grid's kernels take it by value)
// and the helpers for its optional SDPA-style mask.  Shared by decode_attention.hip (the
// chunked, balanced and bundled grids) and decode_shares.hip (the shares grid).
#pragma once

#include "q3t_common.hpp"

namespace q3t {

struct DecodeParams {
    int B, Hq, Hkv, ctx, nchunks;
    int splits;             // balanced grid: workgroups per KV head (0: chunked grid)
    int bundles;            // bundled grid: workgroups per KV head (0: another grid)
    float scale_log2;
    int has_mask, mask_dtype;
    const char *q;
    int64_t q_sb, q_ss, q_sh;
    char *k, *v;
    int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
    const int64_t *offs;
    const int64_t *pos;
    const char *mask;
    int64_t m_sb, m_ss, m_st;
    char *out;
    int64_t o_sb, o_ss, o_sh;
    const char *nk, *nv;
    int64_t nk_sb, nk_sh, nv_sb, nv_sh;
    const char *cs, *sn;
    int64_t cs_sb;
    float *partials;
    int *counters;
    const char *qnw, *knw;  // fused: optional RMSNorm weights (bf16, D) of query / new key rows
    float eps;
    int stream;             // read K/V rows with the non-temporal cache policy (host choice)
    int64_t nk_ss, nv_ss, cs_ss;  // fused, two tokens: token strides of new K/V and cos/sin
    const int32_t *plan;    // bundled grid: the step's plan (decode_shares.hip), null without one
};

// The shares grid (decode_shares.hip): shares per KV head, segment columns per share, plan
// size, published-state floats and flag counters of a launch shape; the launch itself.
int64_t shares_bundle_count(int64_t batch, int64_t kv_heads);
int shares_slot_cap(int64_t group);
int64_t shares_plan_ints(int64_t batch, int64_t kv_heads);
int64_t shares_rank_offset(int64_t batch, int64_t kv_heads);  // ints before the ranking section
int64_t shares_partial_floats(int64_t batch, int64_t kv_heads, int64_t group);
int64_t shares_flag_count(int64_t batch, int64_t kv_heads);
int shares_launch(const DecodeParams &p, int group, bool fused, bool norm, bool mask, hipStream_t s);
int shares_plan_launch(const int64_t *pos, int batch, int ctx, int bundles, int cap, int32_t *plan, hipStream_t s);

Q3T_DEVICE int mask_elem_size(int dtype) { return dtype == Q3T_F32 ? 4 : dtype == Q3T_BOOL ? 1 : 2; }

Q3T_DEVICE float load_mask(const char *m, int dtype) {
    switch (dtype) {
        case Q3T_BF16: return bf16_to_float(*reinterpret_cast<const uint16_t *>(m));
        case Q3T_F16: return (float)*reinterpret_cast<const _Float16 *>(m);
        case Q3T_F32: return *reinterpret_cast<const float *>(m);
        default: return *reinterpret_cast<const uint8_t *>(m) ? 0.0f : -INFINITY;  // bool: True attends
    }
}

}  // namespace q3t
