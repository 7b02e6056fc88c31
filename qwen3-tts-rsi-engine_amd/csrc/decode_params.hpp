// The parameter block of the decode attention launches (every grid's kernels take it by value),
// the helpers for its optional SDPA-style mask, and the step plan's entry points
// (decode_plan.hip).
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
    const int32_t *plan;    // bundled grid: the step's plan (decode_plan.hip), null without one
};

// The step plan (decode_plan.hip): bundles per KV head, plan size in int32 and its launch.
int64_t plan_bundle_count(int64_t batch, int64_t kv_heads);
int64_t plan_ints(int64_t batch, int64_t kv_heads);
int plan_launch(const int64_t *pos, int batch, int ctx, int bundles, int32_t *plan, hipStream_t s);

// 4 bytes per lane from global memory into LDS at lds_base + 4 * lane (the mask words of a
// stage's rows); offsets past the resource's range write zeros.
Q3T_DEVICE void load_to_lds4(i32x4_t rsrc, uint32_t voffset, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\t" Q3T_VMEM_SGPR_WAIT "buffer_load_dword %1, %2, 0 offen lds"
                 :: "s"(lds_base), "v"(voffset), "s"(rsrc) : "memory", "m0");
}

// A mask term (log2 units) from the 4-byte word holding it; `sub` = its byte offset in the word.
Q3T_DEVICE float mask_term(uint32_t word, uint32_t sub, int dtype) {
    const uint32_t x = word >> (8 * sub);
    switch (dtype) {
        case Q3T_BF16: return bf16_to_float(x & 0xffffu) * 1.4426950408889634f;
        case Q3T_F16: return (float)__builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu)) * 1.4426950408889634f;
        case Q3T_F32: return __uint_as_float(word) * 1.4426950408889634f;
        default: return (x & 0xffu) ? 0.0f : -INFINITY;  // bool: True attends
    }
}

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
