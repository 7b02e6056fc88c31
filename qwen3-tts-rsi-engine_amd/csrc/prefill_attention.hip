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


// ---- varlen causal attention on bf16 MFMA tiles ------------------------------------------
//
// One workgroup of 4 waves per (request, 64-query block, G query heads of one KV head);
// wave w owns queries q0 + 16w ... q0 + 16w + 15.  The launch uses G = 1 (one query head
// per workgroup: fewer accumulators, three workgroups per CU).  Keys stream in tiles of 32
// through LDS: K row-major, V transposed (rows padded to 4-byte multiples so that the
// transposed writes spread over 8 banks), so that both products read 16-byte (K) or 4-byte
// (V) runs.  With v_mfma_f32_16x16x32_bf16 (lane l = 16g + c holds
// A[c][8g..8g+7], B[8g..8g+7][c] and D[4g..4g+3][c]):
//   S^T (keys x queries) = K . Q^T   A = K rows from LDS, B = the wave's Q rows (registers);
//                                    lane (g, c) gets keys 4g..4g+3 of query c per 16 keys;
//   O^T (dims x queries) += V^T . P^T   B = P^T straight from the S^T registers, its K index
//                                    ordering keys {4g..4g+3, 16+4g..16+4g+3}; A = V^T rows
//                                    read from LDS in that same key order.
// Each lane therefore keeps the online-softmax state of one query per head, with no data
// movement between the two products.
constexpr int kQBlock = 64;
constexpr int kKTile = 32;   // keys staged per barrier pair
constexpr int kKSub = 32;    // keys per product step
constexpr float kLog2eP = 1.4426950408889634f;
constexpr float kEmptyP = -1.0e30f;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct PrefillParams {
    int B, Hq, Hkv, nqb, group;
    int64_t T;
    float scale_log2;
    const int32_t *cu;
    const char *q;
    int64_t q_st, q_sh;
    const char *k, *v;
    int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
    int64_t cap;
    const int64_t *slots;
    char *out;
    int64_t o_st, o_sh;
};

Q3T_DEVICE bf16x8_t as_bf16x8(const U4 &v) { return __builtin_bit_cast(bf16x8_t, v); }

template <int D, int G>
__global__ void __launch_bounds__(256) prefill_attention_kernel(PrefillParams p) {
    // G: query heads per workgroup (a divisor of the GQA group p.group)
    constexpr int KK = D / 32;   // MFMA steps over the head dimension
    constexpr int DB = D / 16;   // 16-row blocks of O^T
    constexpr int KROW = D + 8;  // padded LDS row of K (bf16)
    constexpr int VROW = kKTile + 2;  // 4-byte rows: the transposed writes of 16 lanes spread over 8 banks
    constexpr int CPR = D / 8;   // 16-byte chunks per row
    __shared__ uint16_t sK[kKTile][KROW];
    __shared__ uint16_t sVt[D][VROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int hgroups = p.Hq / G;
    const int hq0 = (blockIdx.x % hgroups) * G;  // first query head of this workgroup
    const int h = hq0 / p.group;                  // its KV head
    const int rest = blockIdx.x / hgroups;
    const int b = rest % p.B;
    const int qb = p.nqb - 1 - rest / p.B;  // the longest blocks are dispatched first
    const int t0 = p.cu[b];
    if (t0 < 0 || t0 >= p.T) return;
    const int n = (int)min((int64_t)(p.cu[b + 1] - t0), p.T - t0);  // rows past the packed tokens do not exist
    const int q0 = qb * kQBlock;
    if (q0 >= n) return;
    // keys 0 ... kv_end-1 are visible to this block; the arena holds at most `cap` of them
    const int kv_end = (int)min((int64_t)min(n, q0 + kQBlock), p.cap);
    const int ntiles = (kv_end + kKTile - 1) / kKTile;
    const int64_t slot = p.slots ? p.slots[b] : b;

    // the wave's query rows as B operands: Q[query c][8g + 32kk ...], zeros past the request
    const int qpos = q0 + 16 * wave + c;
    const bool qvalid = qpos < n;
    bf16x8_t qB[G][KK];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const char *row = p.q + ((int64_t)(t0 + (qvalid ? qpos : 0)) * p.q_st + (hq0 + j) * p.q_sh) * 2;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            U4 v = load16(row + (32 * kk + 8 * g) * 2);
            if (!qvalid) v = U4{0u, 0u, 0u, 0u};
            qB[j][kk] = as_bf16x8(v);
        }
    }

    // K/V tile loader: 256 threads x 16 bytes per pass; rows past kv_end read zeros
    const char *kbase = p.k + (slot * p.k_sb + h * p.k_sh) * 2;
    const char *vbase = p.v + (slot * p.v_sb + h * p.v_sh) * 2;
    const auto krs = buffer_rsrc(uniform_ptr(kbase), (uint32_t)((kv_end - 1) * p.k_st * 2 + D * 2));
    const auto vrs = buffer_rsrc(uniform_ptr(vbase), (uint32_t)((kv_end - 1) * p.v_st * 2 + D * 2));
    constexpr int PASSES = kKTile * CPR / 256;
    U4 kreg[PASSES], vreg[PASSES];
    auto fetch = [&](int kt) {
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int idx = ps * 256 + tid, row = idx / CPR, ch = idx % CPR;
            const int key = kt * kKTile + row;
            const bool ok = key < kv_end;
            kreg[ps] = buffer_load16(krs, ok ? (uint32_t)(key * p.k_st * 2 + ch * 16) : 0xfffffff0u);
            vreg[ps] = buffer_load16(vrs, ok ? (uint32_t)(key * p.v_st * 2 + ch * 16) : 0xfffffff0u);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int idx = ps * 256 + tid, row = idx / CPR, ch = idx % CPR;
            *reinterpret_cast<U4 *>(&sK[row][ch * 8]) = kreg[ps];
            const uint32_t w[4] = {vreg[ps].x, vreg[ps].y, vreg[ps].z, vreg[ps].w};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                sVt[ch * 8 + 2 * m][row] = (uint16_t)(w[m] & 0xffffu);
                sVt[ch * 8 + 2 * m + 1][row] = (uint16_t)(w[m] >> 16);
            }
        }
    };

    f32x4_t acc[G][DB];
    float m[G], l[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        m[j] = kEmptyP;
        l[j] = 0.f;
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[j][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    fetch(0);
    for (int kt = 0; kt < ntiles; ++kt) {
        __syncthreads();  // every wave is done reading the previous tile
        stage();
        __syncthreads();
        if (kt + 1 < ntiles) fetch(kt + 1);  // in flight during this tile's products
#pragma unroll
        for (int sub = 0; sub < kKTile / kKSub; ++sub) {
        const int kbase_idx = kt * kKTile + sub * kKSub;
        if (kbase_idx > q0 + 16 * wave + 15) break;  // the rest of the tile is above this wave's diagonal

        // S^T for the 16-key blocks of the tile and every head
        constexpr int NKB = kKSub / 16;
        f32x4_t st[NKB][G];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
            for (int j = 0; j < G; ++j) st[kb][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                const bf16x8_t a = as_bf16x8(*reinterpret_cast<const U4 *>(&sK[sub * kKSub + 16 * kb + c][32 * kk + 8 * g]));
#pragma unroll
                for (int j = 0; j < G; ++j)
                    st[kb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qB[j][kk], st[kb][j], 0, 0, 0);
            }
        }
        // scale, causal mask, online softmax per (head, query c); P^T packed to bf16, one
        // B operand per 32 keys (blocks 2s and 2s+1)
        bf16x8_t pB[NKB / 2][G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            float x[NKB * 4];
            float mx = kEmptyP;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kbase_idx + 16 * kb + 4 * g + i;
                    const float s = st[kb][j][i] * p.scale_log2;
                    x[kb * 4 + i] = (key <= qpos && key < kv_end) ? s : -INFINITY;
                    mx = fmaxf(mx, x[kb * 4 + i]);
                }
            mx = fmaxf(mx, xor16(mx));
            mx = fmaxf(mx, xor32(mx));
            const float mn = fmaxf(m[j], mx);
            const float alpha = fexp2(m[j] - mn);
            m[j] = mn;
            float ps = 0.f;
            float pv[NKB * 4];
#pragma unroll
            for (int e = 0; e < NKB * 4; ++e) {
                pv[e] = fexp2(x[e] - mn);
                ps += pv[e];
            }
            l[j] = l[j] * alpha + ps;  // this lane's keys only; summed over g at the end
#pragma unroll
            for (int db = 0; db < DB; ++db) acc[j][db] *= alpha;
#pragma unroll
            for (int sp = 0; sp < NKB / 2; ++sp) {
                const float *q8 = pv + 8 * sp;
                const U4 packed = {cvt_pk_bf16(q8[0], q8[1]), cvt_pk_bf16(q8[2], q8[3]),
                                   cvt_pk_bf16(q8[4], q8[5]), cvt_pk_bf16(q8[6], q8[7])};
                pB[sp][j] = as_bf16x8(packed);
            }
        }
        // O^T += V^T . P^T, 32 keys per product
#pragma unroll
        for (int sp = 0; sp < NKB / 2; ++sp) {
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const uint32_t *row = reinterpret_cast<const uint32_t *>(&sVt[16 * db + c][0]);
                const int k0 = (sub * kKSub + 32 * sp + 4 * g) / 2, k1 = (sub * kKSub + 32 * sp + 16 + 4 * g) / 2;
                const bf16x8_t a = as_bf16x8(U4{row[k0], row[k0 + 1], row[k1], row[k1 + 1]});
#pragma unroll
                for (int j = 0; j < G; ++j)
                    acc[j][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pB[sp][j], acc[j][db], 0, 0, 0);
            }
        }
        }
    }

    if (!qvalid) return;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float lt = l[j] + xor16(l[j]);
        lt += xor32(lt);
        const float inv = __builtin_amdgcn_rcpf(lt);
        char *orow = p.out + ((int64_t)(t0 + qpos) * p.o_st + (hq0 + j) * p.o_sh) * 2;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const uint2 v = {cvt_pk_bf16_canon(acc[j][db][0] * inv, acc[j][db][1] * inv),
                             cvt_pk_bf16_canon(acc[j][db][2] * inv, acc[j][db][3] * inv)};
            *reinterpret_cast<uint2 *>(orow + (16 * db + 4 * g) * 2) = v;
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


template <int D, int G>
static void launch_prefill(const PrefillParams &p, hipStream_t s) {
    hipLaunchKernelGGL((prefill_attention_kernel<D, G>), dim3((uint32_t)p.B * p.nqb * (p.Hq / G)), dim3(256), 0, s, p);
}

extern "C" int q3t_prefill_attention(const q3t_prefill_args *a, void *stream) {
    if (!a) return Q3T_EINVAL;
    if (a->batch < 1 || a->batch > (1 << 20) || a->total_tokens < 0 || a->total_tokens > INT32_MAX ||
        a->max_seqlen < 0 || a->capacity < 1 || a->q_heads < 1 || a->kv_heads < 1 ||
        a->q_heads % a->kv_heads)
        return Q3T_EINVAL;
    if (a->head_dim != 64 && a->head_dim != 128) return Q3T_EUNSUPPORTED;
    const int64_t G = a->q_heads / a->kv_heads;
    if (G != 1 && G != 2 && G != 4) return Q3T_EUNSUPPORTED;
    if (a->total_tokens == 0 || a->max_seqlen == 0) return Q3T_OK;
    if (!a->cu_seqlens || !a->query || !a->keys || !a->values || !a->out) return Q3T_EINVAL;
    const int64_t st[] = {a->q_stride_t, a->q_stride_h, a->k_stride_b, a->k_stride_h, a->k_stride_t,
                          a->v_stride_b, a->v_stride_h, a->v_stride_t, a->o_stride_t, a->o_stride_h};
    for (int64_t v : st)
        if (v < 0 || (v * 2) % 16) return Q3T_EINVAL;
    if (!aligned(a->query, 16) || !aligned(a->keys, 16) || !aligned(a->values, 16) || !aligned(a->out, 8))
        return Q3T_EINVAL;
    // key rows of one (slot, head) are addressed by 32-bit byte offsets
    const int64_t max_st = a->k_stride_t > a->v_stride_t ? a->k_stride_t : a->v_stride_t;
    if (a->capacity * max_st * 2 + a->head_dim * 2 > INT32_MAX) return Q3T_EUNSUPPORTED;
    PrefillParams p;
    p.B = (int)a->batch; p.Hq = (int)a->q_heads; p.Hkv = (int)a->kv_heads;
    p.group = (int)G;
    p.nqb = (int)((a->max_seqlen + kQBlock - 1) / kQBlock);
    if ((int64_t)p.B * p.nqb * p.Hq > INT32_MAX) return Q3T_EUNSUPPORTED;
    p.scale_log2 = a->scale * kLog2eP;
    p.cu = a->cu_seqlens;
    p.q = (const char *)a->query; p.q_st = a->q_stride_t; p.q_sh = a->q_stride_h;
    p.k = (const char *)a->keys; p.v = (const char *)a->values;
    p.k_sb = a->k_stride_b; p.k_sh = a->k_stride_h; p.k_st = a->k_stride_t;
    p.v_sb = a->v_stride_b; p.v_sh = a->v_stride_h; p.v_st = a->v_stride_t;
    p.slots = a->kv_slots;
    p.cap = a->capacity;
    p.T = a->total_tokens;
    p.out = (char *)a->out; p.o_st = a->o_stride_t; p.o_sh = a->o_stride_h;
    hipStream_t s = (hipStream_t)stream;
    // one query head per workgroup: the accumulators of a single head keep the kernel at a
    // register count that leaves two workgroups per CU's SIMDs busy
    if (a->head_dim == 128) launch_prefill<128, 1>(p, s);
    else launch_prefill<64, 1>(p, s);
    return launch_status();
}
