// Varlen causal prefill: RoPE + arena write prologue and the attention kernel.
//
// Reference behaviour: PrefillGraph.compute (prefill_graph.py:31-50) runs padded causal
// self-attention with positions cumsum(mask)-1 and mask key_valid & causal; the per-layer
// prefill KV is later copied into the request's arena slot (continuous.py:468-471,
// packed_kv.py:6-31).  Here requests are packed along the token axis by cu_seqlens, so
// only valid rows exist, and rotated keys/values go straight into the arena slot.
#include "q3t_common.hpp"

namespace q3t {

struct PrefillRopeWriteParams {
    int B, Hq, Hkv, D;
    int64_t T, capacity;
    const int32_t *cu;
    const char *q, *k, *v;
    int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh;
    const char *cs, *sn;
    int64_t cs_st;
    char *qo;
    int64_t qo_st, qo_sh;
    char *ak, *av;
    int64_t a_sb, a_sh, a_st;
    const int64_t *slots;
};

Q3T_DEVICE int request_of(const int32_t *cu, int B, int64_t t) {
    int lo = 0, hi = B - 1;  // last b with cu[b] <= t
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// One work item: 8 dims of each half of one (token, head) row.  Heads [0, Hq) are query
// heads (rotated into q_out); heads [Hq, Hq+Hkv) rotate the key and copy the value into
// the arena at the token's position within its request.
__global__ void __launch_bounds__(256) prefill_rope_write_kernel(PrefillRopeWriteParams p) {
    const int vecs = p.D / 16;
    const int heads = p.Hq + p.Hkv;
    const int64_t total = p.T * heads * vecs;
    const int half = p.D / 2;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % vecs);
        const int64_t th = i / vecs;
        const int hd = (int)(th % heads);
        const int64_t t = th / heads;
        const char *crow = p.cs + t * p.cs_st * 2, *srow = p.sn + t * p.cs_st * 2;
        U4 c1 = load16(crow + c * 16), c2 = load16(crow + (half + c * 8) * 2);
        U4 s1 = load16(srow + c * 16), s2 = load16(srow + (half + c * 8) * 2);
        if (hd < p.Hq) {
            const char *row = p.q + (t * p.q_st + hd * p.q_sh) * 2;
            U4 x1 = load16(row + c * 16), x2 = load16(row + (half + c * 8) * 2), y1, y2;
            rope8(&x1.x, &x2.x, &c1.x, &c2.x, &s1.x, &s2.x, &y1.x, &y2.x);
            char *orow = p.qo + (t * p.qo_st + hd * p.qo_sh) * 2;
            store16(orow + c * 16, y1);
            store16(orow + (half + c * 8) * 2, y2);
        } else {
            const int h = hd - p.Hq;
            const int b = request_of(p.cu, p.B, t);
            const int64_t pos = t - p.cu[b];
            if (pos < 0 || pos >= p.capacity) continue;
            const int64_t slot = p.slots ? p.slots[b] : b;
            const char *krow = p.k + (t * p.k_st + h * p.k_sh) * 2;
            const char *vrow = p.v + (t * p.v_st + h * p.v_sh) * 2;
            U4 x1 = load16(krow + c * 16), x2 = load16(krow + (half + c * 8) * 2), y1, y2;
            rope8(&x1.x, &x2.x, &c1.x, &c2.x, &s1.x, &s2.x, &y1.x, &y2.x);
            const int64_t a = (slot * p.a_sb + h * p.a_sh + pos * p.a_st) * 2;
            store16(p.ak + a + c * 16, y1);
            store16(p.ak + a + (half + c * 8) * 2, y2);
            store16(p.av + a + c * 16, load16(vrow + c * 16));
            store16(p.av + a + (half + c * 8) * 2, load16(vrow + (half + c * 8) * 2));
        }
    }
}

}  // namespace q3t

using namespace q3t;

extern "C" int q3t_prefill_rope_write(const q3t_prefill_rope_write_args *a, void *stream) {
    if (!a) return Q3T_EINVAL;
    if (a->batch < 1 || a->total_tokens < 0 || a->q_heads < 1 || a->kv_heads < 1 ||
        a->capacity < 1 || a->batch > (1 << 20))
        return Q3T_EINVAL;
    if (a->head_dim != 64 && a->head_dim != 128) return Q3T_EUNSUPPORTED;
    if (a->total_tokens == 0) return Q3T_OK;
    if (!a->cu_seqlens || !a->query || !a->key || !a->value || !a->cos || !a->sin || !a->q_out ||
        !a->arena_keys || !a->arena_values)
        return Q3T_EINVAL;
    const int64_t st[] = {a->q_stride_t, a->q_stride_h, a->k_stride_t, a->k_stride_h,
                          a->v_stride_t, a->v_stride_h, a->cs_stride_t, a->qo_stride_t,
                          a->qo_stride_h, a->a_stride_b, a->a_stride_h, a->a_stride_t};
    for (int64_t s : st)
        if ((s * 2) % 16) return Q3T_EINVAL;
    const void *ptrs[] = {a->query, a->key, a->value, a->cos, a->sin, a->q_out, a->arena_keys, a->arena_values};
    for (const void *q : ptrs)
        if (!aligned(q, 16)) return Q3T_EINVAL;
    PrefillRopeWriteParams p;
    p.B = (int)a->batch; p.Hq = (int)a->q_heads; p.Hkv = (int)a->kv_heads; p.D = (int)a->head_dim;
    p.T = a->total_tokens; p.capacity = a->capacity; p.cu = a->cu_seqlens;
    p.q = (const char *)a->query; p.k = (const char *)a->key; p.v = (const char *)a->value;
    p.q_st = a->q_stride_t; p.q_sh = a->q_stride_h; p.k_st = a->k_stride_t; p.k_sh = a->k_stride_h;
    p.v_st = a->v_stride_t; p.v_sh = a->v_stride_h;
    p.cs = (const char *)a->cos; p.sn = (const char *)a->sin; p.cs_st = a->cs_stride_t;
    p.qo = (char *)a->q_out; p.qo_st = a->qo_stride_t; p.qo_sh = a->qo_stride_h;
    p.ak = (char *)a->arena_keys; p.av = (char *)a->arena_values;
    p.a_sb = a->a_stride_b; p.a_sh = a->a_stride_h; p.a_st = a->a_stride_t;
    p.slots = a->kv_slots;
    const int64_t total = p.T * (p.Hq + p.Hkv) * (p.D / 16);
    int64_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(prefill_rope_write_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, p);
    return launch_status();
}

extern "C" int q3t_prefill_attention(const q3t_prefill_args *a, void *stream) {
    (void)a;
    (void)stream;
    return Q3T_EUNSUPPORTED;
}
