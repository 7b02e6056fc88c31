// Ragged grouped-query decode attention over the slot arena, with split-K.
//
// Reference behaviour (InferMatrixLab/qwen3-tts-rsi-engine):
//   out[b, hq] = softmax(q[b, hq] . K[b, hq/G, :L_b]^T * scale + mask) . V[b, hq/G, :L_b]
//   with L_b = pos[b] + 1 (SlotGraph.compute's mask `j <= pos[b]`, continuous.py:191-192,
//   dispatched from PackedAttention.forward, packed_attention.py:75-84, to SDPA or
//   npu_attention.attention, npu_attention.py:11-26).
// Fused variant: RoPE of q and of the new key (packed_attention.py:46-51,
// rotary_triton_ascend.py:19-24) and the paired K/V write at pos[b]
// (continuous.py:152-166, kv_triton_ascend.py:24-36) happen inside the same launch.
//
// Work decomposition (stream-K over keys, per KV head):
//   * grid = kv_heads x P workgroups of 256 threads; workgroup x serves KV head x % kv_heads,
//     so with 8 KV heads every head maps onto one XCD under the round-robin dispatch and
//     all partial states of a head stay in that XCD's L2.
//   * The keys of one head are flattened over requests (T = sum L_b) and cut into P equal
//     ranges; every workgroup therefore streams the same number of K/V bytes whatever the
//     length mix.  A range covers pieces of one or more requests.
//   * Inside a workgroup each wave takes blocks of 8*U keys; within a wave 8 lanes share one
//     key (each lane holds 16 bytes of two 128-byte half rows, so one load instruction reads
//     8 whole 128-byte lines) and every 8-lane group keeps its own online-softmax state.
//   * End of a piece: the 32 group states are merged with lane shuffles and then through
//     LDS (the "LDS-staged online-softmax merge").  A request split over several workgroups
//     publishes its partial (m, l, acc) to the workspace; the last workgroup to arrive
//     (atomic counter) merges the partials in piece order and writes the output, then
//     re-zeroes the counter, so results are deterministic and the launch is graph-replayable.
#include "q3t_common.hpp"

namespace q3t {

constexpr int kMaxBatch = 1024;
constexpr int kWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kEmpty = -1.0e30f;  // finite "no key yet" running max

struct DecodeParams {
    int B, Hq, Hkv, ctx, P;
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
};

template <typename T> struct ElemInfo;
template <> struct ElemInfo<uint16_t> { static constexpr int CW = 8; };  // bf16 per 16 bytes
template <> struct ElemInfo<float> { static constexpr int CW = 4; };

Q3T_DEVICE float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

Q3T_DEVICE float load_mask(const char *m, int dtype) {
    switch (dtype) {
        case Q3T_BF16: return bf16_to_float(*reinterpret_cast<const uint16_t *>(m));
        case Q3T_F16: return (float)*reinterpret_cast<const _Float16 *>(m);
        case Q3T_F32: return *reinterpret_cast<const float *>(m);
        default: return *reinterpret_cast<const uint8_t *>(m) ? 0.0f : -INFINITY;  // bool: True attends
    }
}

// Score partial for one lane: its 16-byte chunks of q row and key row.
template <typename T, int NCH>
Q3T_DEVICE float lane_dot(const U4 (&q)[NCH], const U4 (&k)[NCH]) {
    float s = 0.f;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            s = dot2_bf16(q[c].x, k[c].x, s);
            s = dot2_bf16(q[c].y, k[c].y, s);
            s = dot2_bf16(q[c].z, k[c].z, s);
            s = dot2_bf16(q[c].w, k[c].w, s);
        }
    } else {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            s += __uint_as_float(q[c].x) * __uint_as_float(k[c].x);
            s += __uint_as_float(q[c].y) * __uint_as_float(k[c].y);
            s += __uint_as_float(q[c].z) * __uint_as_float(k[c].z);
            s += __uint_as_float(q[c].w) * __uint_as_float(k[c].w);
        }
    }
    return s;
}

template <typename T, int NCH, int EPL>
Q3T_DEVICE void unpack_v(const U4 (&v)[NCH], float (&out)[EPL]) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const uint32_t w[4] = {v[c].x, v[c].y, v[c].z, v[c].w};
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                out[c * 8 + 2 * i] = bf16_lo(w[i]);
                out[c * 8 + 2 * i + 1] = bf16_hi(w[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) out[c * 4 + i] = __uint_as_float(w[i]);
        }
    }
}

// One online-softmax step of an 8-lane group over UU keys held in registers.
// key_idx[u] is the key's index within its request (for query-row causal limits and the
// mask); valid[u] excludes keys outside the piece.
template <typename T, int R, int G, int SQ, int NCH, int EPL, int UU>
Q3T_DEVICE void softmax_step(const DecodeParams &p, const U4 (&qr)[R][NCH], const U4 (&kr)[UU][NCH],
                             const U4 (&vr)[UU][NCH], const bool (&valid)[UU],
                             const int (&key_idx)[UU], int last_pos, const char *mask_row,
                             float (&m)[R], float (&l)[R], float (&acc)[R][EPL]) {
    float s[UU][R];
#pragma unroll
    for (int u = 0; u < UU; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r) s[u][r] = sum8(lane_dot<T, NCH>(qr[r], kr[u]));
#pragma unroll
    for (int u = 0; u < UU; ++u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int qi = r / G;
            bool ok = valid[u];
            // with no explicit mask, several queries of a request are causal among the last keys
            if constexpr (SQ > 1) ok = ok && (p.has_mask || key_idx[u] <= last_pos - (SQ - 1) + qi);
            float x = s[u][r] * p.scale_log2;
            if (p.has_mask && ok) {
                const char *mp = mask_row + (qi * p.m_ss + (int64_t)key_idx[u] * p.m_st) *
                                                (p.mask_dtype == Q3T_F32 ? 4 : p.mask_dtype == Q3T_BOOL ? 1 : 2);
                x += load_mask(mp, p.mask_dtype) * kLog2e;
            }
            s[u][r] = ok ? x : -INFINITY;
        }
    }
    float vf[UU][EPL];
#pragma unroll
    for (int u = 0; u < UU; ++u) unpack_v<T, NCH, EPL>(vr[u], vf[u]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float mx = m[r];
#pragma unroll
        for (int u = 0; u < UU; ++u) mx = fmaxf(mx, s[u][r]);
        const float alpha = fexp2(m[r] - mx);
        float pu[UU], psum = 0.f;
#pragma unroll
        for (int u = 0; u < UU; ++u) {
            pu[u] = fexp2(s[u][r] - mx);
            psum += pu[u];
        }
        l[r] = l[r] * alpha + psum;
        m[r] = mx;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float a = acc[r][e] * alpha;
#pragma unroll
            for (int u = 0; u < UU; ++u) a += pu[u] * vf[u][e];
            acc[r][e] = a;
        }
    }
}

// Workgroup owning key x of a head's flattened key range when it is cut into P ranges
// [floor(T*i/P), floor(T*(i+1)/P)).
Q3T_DEVICE int owner_of(int64_t x, int64_t T, int P) { return (int)(((x + 1) * P - 1) / T); }
Q3T_DEVICE int64_t range_start(int i, int64_t T, int P) { return T * i / P; }

template <typename T>
Q3T_DEVICE void store_out(char *base, float v) {
    if constexpr (sizeof(T) == 2)
        *reinterpret_cast<uint16_t *>(base) = (uint16_t)float_to_bf16(v);
    else
        *reinterpret_cast<float *>(base) = v;
}

template <typename T, int D, int G, int SQ, bool FUSED>
__global__ void __launch_bounds__(256) decode_attention_kernel(DecodeParams p) {
    constexpr int R = G * SQ;
    constexpr int CW = ElemInfo<T>::CW;
    constexpr int NCH = D / (8 * CW);
    constexpr int EPL = NCH * CW;
    constexpr int U = R <= 2 ? 4 : (R <= 4 ? 2 : 1);
    constexpr int KPW = 8 * U;
    constexpr int ES = sizeof(T);
    static_assert(!FUSED || (ES == 2 && D == 128 && SQ == 1), "fused path: bf16, D=128, one query");

    __shared__ int sm_len[kMaxBatch];
    __shared__ int sm_start[kMaxBatch];
    __shared__ int sm_wsum[kWaves];
    __shared__ float sm_acc[kWaves][R][D];
    __shared__ float sm_m[kWaves][R], sm_l[kWaves][R];
    __shared__ int sm_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 3, cl = lane & 7;
    const int h = blockIdx.x % p.Hkv;
    const int wg = blockIdx.x / p.Hkv;
    const int B = p.B;

    // ---- 1. per-request key counts and their exclusive prefix sum (block scan) ----
    int vals[4], tsum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid * 4 + i;
        int L = 0;
        if (idx < B) {
            const int64_t pp = p.pos[idx];
            L = (pp >= 0 && pp < p.ctx) ? (int)pp + 1 : 0;
        }
        vals[i] = L;
        tsum += L;
    }
    int incl = tsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) sm_wsum[wave] = incl;
    __syncthreads();
    int excl = incl - tsum, total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        if (w < wave) excl += sm_wsum[w];
        total += sm_wsum[w];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = tid * 4 + i;
        if (idx < B) {
            sm_len[idx] = vals[i];
            sm_start[idx] = excl;
        }
        excl += vals[i];
    }
    __syncthreads();

    // Requests without a valid position attend nothing; their rows are written as zeros.
    if (wg == 0) {
        for (int b = 0; b < B; ++b) {
            if (sm_len[b]) continue;
            for (int t = tid; t < R * D; t += blockDim.x) {
                const int r = t / D, d = t % D;
                const int qi = r / G, hq = h * G + r % G;
                store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, 0.f);
            }
        }
    }

    const int64_t Ttot = total;
    const int P = (int)(Ttot < p.P ? Ttot : p.P);  // every range non-empty
    if (wg >= P) return;
    const int64_t start = range_start(wg, Ttot, P), end = range_start(wg + 1, Ttot, P);

    // first request whose keys contain `start`
    int lo = 0, hi = B - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (sm_start[mid] <= start) lo = mid; else hi = mid - 1;
    }
    const int b_first = lo;

    for (int b = b_first; b < B && sm_start[b] < end; ++b) {
        const int Lb = sm_len[b];
        if (Lb == 0) continue;
        const int64_t sb = sm_start[b];
        const int ka = (int)((start > sb ? start : sb) - sb);
        const int ke = (int)((end < sb + Lb ? end : sb + Lb) - sb);
        const int last_pos = Lb - 1;
        const bool own_last = (ke == Lb);

        // ---- query rows of this KV head: R = G heads x SQ queries ----
        U4 qr[R][NCH];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int qi = r / G, hq = h * G + r % G;
            const char *row = p.q + (b * p.q_sb + qi * p.q_ss + hq * p.q_sh) * ES;
#pragma unroll
            for (int c = 0; c < NCH; ++c) qr[r][c] = load16(row + ((c * 8 + cl) * CW) * ES);
        }
        U4 cs1, cs2, sn1, sn2;
        if constexpr (FUSED) {
            const char *crow = p.cs + b * p.cs_sb * 2, *srow = p.sn + b * p.cs_sb * 2;
            cs1 = load16(crow + cl * 16); cs2 = load16(crow + 128 + cl * 16);
            sn1 = load16(srow + cl * 16); sn2 = load16(srow + 128 + cl * 16);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                U4 y1, y2;
                rope8(&qr[r][0].x, &qr[r][1].x, &cs1.x, &cs2.x, &sn1.x, &sn2.x, &y1.x, &y2.x);
                qr[r][0] = y1;
                qr[r][1] = y2;
            }
        }

        const int64_t koff = p.offs ? p.offs[b] : (int64_t)b * p.k_sb;
        const int64_t voff = p.offs ? p.offs[b] : (int64_t)b * p.v_sb;
        char *kb = p.k + (koff + h * p.k_sh) * ES;
        char *vb = p.v + (voff + h * p.v_sh) * ES;
        const char *mask_row = p.has_mask ? p.mask + b * p.m_sb * (p.mask_dtype == Q3T_F32 ? 4 : p.mask_dtype == Q3T_BOOL ? 1 : 2) : nullptr;

        float m[R], l[R], acc[R][EPL];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            m[r] = kEmpty;
            l[r] = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[r][e] = 0.f;
        }

        // ---- stream the arena keys of the piece ----
        const int kend = (FUSED && own_last) ? last_pos : ke;
        for (int base = ka + wave * KPW; base < kend; base += kWaves * KPW) {
            U4 kr[U][NCH], vr[U][NCH];
            bool valid[U];
            int kidx[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = base + grp + 8 * u;
                valid[u] = j < kend;
                kidx[u] = j;
                const int js = valid[u] ? j : base;
                const char *krow = kb + (int64_t)js * p.k_st * ES;
                const char *vrow = vb + (int64_t)js * p.v_st * ES;
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    kr[u][c] = load16(krow + ((c * 8 + cl) * CW) * ES);
                    vr[u][c] = load16(vrow + ((c * 8 + cl) * CW) * ES);
                }
            }
            softmax_step<T, R, G, SQ, NCH, EPL, U>(p, qr, kr, vr, valid, kidx, last_pos, mask_row,
                                                  m, l, acc);
        }

        // ---- fused: rotate, store and attend the new key at position pos[b] ----
        if constexpr (FUSED) {
            if (own_last && wave == 0) {
                U4 kr[1][NCH], vr[1][NCH];
                bool valid[1] = {grp == 0};
                int kidx[1] = {last_pos};
                kr[0][0] = kr[0][1] = vr[0][0] = vr[0][1] = U4{0u, 0u, 0u, 0u};
                if (grp == 0) {
                    const char *nkrow = p.nk + (b * p.nk_sb + h * p.nk_sh) * ES;
                    const char *nvrow = p.nv + (b * p.nv_sb + h * p.nv_sh) * ES;
                    U4 k1 = load16(nkrow + cl * 16), k2 = load16(nkrow + 128 + cl * 16);
                    vr[0][0] = load16(nvrow + cl * 16);
                    vr[0][1] = load16(nvrow + 128 + cl * 16);
                    rope8(&k1.x, &k2.x, &cs1.x, &cs2.x, &sn1.x, &sn2.x, &kr[0][0].x, &kr[0][1].x);
                    char *dk = kb + (int64_t)last_pos * p.k_st * ES;
                    char *dv = vb + (int64_t)last_pos * p.v_st * ES;
                    store16(dk + cl * 16, kr[0][0]);
                    store16(dk + 128 + cl * 16, kr[0][1]);
                    store16(dv + cl * 16, vr[0][0]);
                    store16(dv + 128 + cl * 16, vr[0][1]);
                }
                softmax_step<T, R, G, SQ, NCH, EPL, 1>(p, qr, kr, vr, valid, kidx, last_pos,
                                                      mask_row, m, l, acc);
            }
        }

        // ---- merge the 8 group states of each wave (lanes differing in bits 3..5) ----
#pragma unroll
        for (int x = 8; x < 64; x <<= 1) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float mo = __shfl_xor(m[r], x), lo2 = __shfl_xor(l[r], x);
                const float mn = fmaxf(m[r], mo);
                const float a = fexp2(m[r] - mn), bb = fexp2(mo - mn);
                l[r] = l[r] * a + lo2 * bb;
                m[r] = mn;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[r][e] = acc[r][e] * a + __shfl_xor(acc[r][e], x) * bb;
            }
        }
        if (grp == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
#pragma unroll
                for (int c = 0; c < NCH; ++c)
#pragma unroll
                    for (int e = 0; e < CW; ++e) sm_acc[wave][r][(c * 8 + cl) * CW + e] = acc[r][c * CW + e];
                if (cl == 0) {
                    sm_m[wave][r] = m[r];
                    sm_l[wave][r] = l[r];
                }
            }
        }
        __syncthreads();

        // ---- merge the waves: thread t owns (row, dim) pairs ----
        const int first_wg = owner_of(sb, Ttot, P), last_wg = owner_of(sb + Lb - 1, Ttot, P);
        const int pieces = last_wg - first_wg + 1;
        float *part = nullptr;
        if (pieces > 1) {
            const int which = (b == b_first) ? 0 : 1;
            part = p.partials + ((int64_t)(wg * p.Hkv + h) * 2 + which) * (R * (D + 2));
        }
        for (int t = tid; t < R * D; t += blockDim.x) {
            const int r = t / D, d = t % D;
            float M = sm_m[0][r];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm_m[w][r]);
            float Ls = 0.f, A = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float wt = fexp2(sm_m[w][r] - M);
                Ls += sm_l[w][r] * wt;
                A += sm_acc[w][r][d] * wt;
            }
            if (pieces == 1) {
                const int qi = r / G, hq = h * G + r % G;
                store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, A / Ls);
            } else {
                part[r * (D + 2) + d] = A;
                if (d == 0) {
                    part[r * (D + 2) + D] = M;
                    part[r * (D + 2) + D + 1] = Ls;
                }
            }
        }

        if (pieces > 1) {
            // publish the partial; the last of the request's workgroups merges them all
            __threadfence();
            __syncthreads();
            if (tid == 0) {
                const int old = atomicAdd(&p.counters[h * B + b], 1);
                sm_last = (old == pieces - 1);
            }
            __syncthreads();
            if (sm_last) {
                __threadfence();
                for (int t = tid; t < R * D; t += blockDim.x) {
                    const int r = t / D, d = t % D;
                    float M = kEmpty;
                    for (int i = first_wg; i <= last_wg; ++i) {
                        const int which = (i == first_wg && sb > range_start(i, Ttot, P)) ? 1 : 0;
                        const float *pp = p.partials + ((int64_t)(i * p.Hkv + h) * 2 + which) * (R * (D + 2));
                        M = fmaxf(M, __builtin_nontemporal_load(pp + r * (D + 2) + D));
                    }
                    float Ls = 0.f, A = 0.f;
                    for (int i = first_wg; i <= last_wg; ++i) {
                        const int which = (i == first_wg && sb > range_start(i, Ttot, P)) ? 1 : 0;
                        const float *pp = p.partials + ((int64_t)(i * p.Hkv + h) * 2 + which) * (R * (D + 2));
                        const float wt = fexp2(__builtin_nontemporal_load(pp + r * (D + 2) + D) - M);
                        Ls += __builtin_nontemporal_load(pp + r * (D + 2) + D + 1) * wt;
                        A += __builtin_nontemporal_load(pp + r * (D + 2) + d) * wt;
                    }
                    const int qi = r / G, hq = h * G + r % G;
                    store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, A / Ls);
                }
                if (tid == 0) atomicExch(&p.counters[h * B + b], 0);
            }
        }
        __syncthreads();  // LDS state is reused by the next piece
    }
}

// ---------------------------------------------------------------------------------------

static int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

static int64_t default_splits(int64_t kv_heads) {
    int64_t s = (2 * (int64_t)device_cus()) / (kv_heads > 0 ? kv_heads : 1);
    return s < 1 ? 1 : s;
}

// The counter region has one fixed size, so that the counters of every launch sit on bytes
// that only ever hold counters (all zero between launches), whatever batch and head count
// earlier launches on the same workspace used.
constexpr int64_t kMaxCounters = 65536;  // kv_heads * batch
static int64_t counters_bytes() { return kMaxCounters * 4; }

}  // namespace q3t

using namespace q3t;

extern "C" int64_t q3t_decode_workspace_bytes(int64_t batch, int64_t query_len, int64_t q_heads,
                                              int64_t kv_heads, int64_t head_dim,
                                              int64_t splits_per_head) {
    if (batch < 0 || query_len < 1 || kv_heads < 1 || q_heads < kv_heads || head_dim < 1) return -1;
    const int64_t P = splits_per_head > 0 ? splits_per_head : default_splits(kv_heads);
    const int64_t R = (q_heads / kv_heads) * query_len;
    return counters_bytes() + kv_heads * P * 2 * R * (head_dim + 2) * 4;
}

template <typename T, int D, int G, int SQ, bool F>
static void launch_decode(const DecodeParams &p, hipStream_t s) {
    hipLaunchKernelGGL((decode_attention_kernel<T, D, G, SQ, F>), dim3(p.Hkv * p.P), dim3(256), 0, s, p);
}

template <typename T, int D, int G>
static int dispatch_sq(const DecodeParams &p, int sq, bool fused, hipStream_t s) {
    if (fused) {
        if constexpr (sizeof(T) == 2 && D == 128) {
            if (sq != 1) return Q3T_EUNSUPPORTED;
            launch_decode<T, D, G, 1, true>(p, s);
            return Q3T_OK;
        } else {
            return Q3T_EUNSUPPORTED;
        }
    }
    if (sq == 1) launch_decode<T, D, G, 1, false>(p, s);
    else if (sq == 2) launch_decode<T, D, G, 2, false>(p, s);
    else return Q3T_EUNSUPPORTED;
    return Q3T_OK;
}

template <typename T, int D>
static int dispatch_g(const DecodeParams &p, int g, int sq, bool fused, hipStream_t s) {
    switch (g) {
        case 1: return dispatch_sq<T, D, 1>(p, sq, fused, s);
        case 2: return dispatch_sq<T, D, 2>(p, sq, fused, s);
        case 4: return dispatch_sq<T, D, 4>(p, sq, fused, s);
        default: return Q3T_EUNSUPPORTED;
    }
}

extern "C" int q3t_decode_attention(const q3t_decode_args *a, void *stream) {
    if (!a) return Q3T_EINVAL;
    if (a->batch < 0 || a->batch > kMaxBatch || a->query_len < 1 || a->q_heads < 1 ||
        a->kv_heads < 1 || a->head_dim < 1 || a->ctx < 1 || a->ctx > (1 << 20))
        return Q3T_EINVAL;
    if (a->q_heads % a->kv_heads) return Q3T_EINVAL;
    if (a->kv_heads * a->batch > kMaxCounters) return Q3T_EUNSUPPORTED;
    if (a->batch == 0) return Q3T_OK;
    if (!a->query || !a->keys || !a->values || !a->positions || !a->out) return Q3T_EINVAL;
    if (a->dtype != Q3T_BF16 && a->dtype != Q3T_F32) return Q3T_EUNSUPPORTED;
    if (a->head_dim != 64 && a->head_dim != 128) return Q3T_EUNSUPPORTED;
    const int64_t es = a->dtype == Q3T_BF16 ? 2 : 4;
    const bool fused = a->fused != 0;
    if (fused && (!a->new_key || !a->new_value || !a->cos || !a->sin)) return Q3T_EINVAL;
    if (a->mask && (a->mask_dtype < 0 || a->mask_dtype > 3)) return Q3T_EINVAL;
    // 16-byte vector access to query rows, arena rows and (fused) new rows and cos/sin rows
    const int64_t vec_strides[] = {a->q_stride_b, a->q_stride_s, a->q_stride_h, a->k_stride_b,
                                   a->k_stride_h, a->k_stride_t, a->v_stride_b, a->v_stride_h,
                                   a->v_stride_t};
    for (int64_t st : vec_strides)
        if ((st * es) % 16) return Q3T_EINVAL;
    if (!aligned(a->query, 16) || !aligned(a->keys, 16) || !aligned(a->values, 16)) return Q3T_EINVAL;
    if (fused) {
        const int64_t fs[] = {a->nk_stride_b, a->nk_stride_h, a->nv_stride_b, a->nv_stride_h, a->cs_stride_b};
        for (int64_t st : fs)
            if ((st * es) % 16) return Q3T_EINVAL;
        if (!aligned(a->new_key, 16) || !aligned(a->new_value, 16) || !aligned(a->cos, 16) ||
            !aligned(a->sin, 16))
            return Q3T_EINVAL;
    }
    const int64_t P = a->splits_per_head > 0 ? a->splits_per_head : default_splits(a->kv_heads);
    if (P > 65535 || a->kv_heads * P > (int64_t)1 << 30) return Q3T_EINVAL;
    const int64_t need = q3t_decode_workspace_bytes(a->batch, a->query_len, a->q_heads, a->kv_heads,
                                                    a->head_dim, P);
    if (!a->workspace || a->workspace_bytes < need || !aligned(a->workspace, 16)) return Q3T_EWORKSPACE;

    DecodeParams p;
    p.B = (int)a->batch;
    p.Hq = (int)a->q_heads;
    p.Hkv = (int)a->kv_heads;
    p.ctx = (int)a->ctx;
    p.P = (int)P;
    p.scale_log2 = a->scale * kLog2e;
    p.has_mask = a->mask != nullptr;
    p.mask_dtype = (int)a->mask_dtype;
    p.q = (const char *)a->query;
    p.q_sb = a->q_stride_b; p.q_ss = a->q_stride_s; p.q_sh = a->q_stride_h;
    p.k = (char *)a->keys; p.v = (char *)a->values;
    p.k_sb = a->k_stride_b; p.k_sh = a->k_stride_h; p.k_st = a->k_stride_t;
    p.v_sb = a->v_stride_b; p.v_sh = a->v_stride_h; p.v_st = a->v_stride_t;
    p.offs = a->kv_offsets;
    p.pos = a->positions;
    p.mask = (const char *)a->mask;
    p.m_sb = a->mask_stride_b; p.m_ss = a->mask_stride_s; p.m_st = a->mask_stride_t;
    p.out = (char *)a->out;
    p.o_sb = a->o_stride_b; p.o_ss = a->o_stride_s; p.o_sh = a->o_stride_h;
    p.nk = (const char *)a->new_key; p.nv = (const char *)a->new_value;
    p.nk_sb = a->nk_stride_b; p.nk_sh = a->nk_stride_h; p.nv_sb = a->nv_stride_b; p.nv_sh = a->nv_stride_h;
    p.cs = (const char *)a->cos; p.sn = (const char *)a->sin; p.cs_sb = a->cs_stride_b;
    p.counters = (int *)a->workspace;
    p.partials = (float *)((char *)a->workspace + counters_bytes());

    const int g = (int)(a->q_heads / a->kv_heads);
    const int sq = (int)a->query_len;
    hipStream_t s = (hipStream_t)stream;
    int st;
    if (a->dtype == Q3T_BF16)
        st = a->head_dim == 128 ? dispatch_g<uint16_t, 128>(p, g, sq, fused, s)
                                : dispatch_g<uint16_t, 64>(p, g, sq, fused, s);
    else
        st = a->head_dim == 128 ? dispatch_g<float, 128>(p, g, sq, fused, s)
                                : dispatch_g<float, 64>(p, g, sq, fused, s);
    if (st != Q3T_OK) return st;
    return launch_status();
}
