// Ragged grouped-query decode attention over the slot arena, split along the keys.
//
// Reference behaviour (InferMatrixLab/qwen3-tts-rsi-engine):
//   out[b, hq] = softmax(q[b, hq] . K[b, hq/G, :L_b]^T * scale + mask) . V[b, hq/G, :L_b]
//   with L_b = pos[b] + 1 (SlotGraph.compute's mask `j <= pos[b]`, continuous.py:191-192,
//   dispatched from PackedAttention.forward, packed_attention.py:75-84, to SDPA or
//   npu_attention.attention, npu_attention.py:11-26).
// Fused variant: RoPE of q and of the new key (packed_attention.py:46-51,
// rotary_triton_ascend.py:19-24) and the paired K/V write at pos[b]
// (continuous.py:152-166, kv_triton_ascend.py:24-36) happen inside the same launch; with
// two tokens per request (the code predictor's first step, continuous.py:37-40) both are
// rotated, written at pos[b] - 1 and pos[b], and attended causally.
//
// Design (one launch per layer, no per-step preparation):
//   * keys are cut into chunks of kChunkRows consecutive keys (several consecutive blocks
//     per chunk when a request has more blocks than `nchunks`); one 256-thread workgroup per
//     (request, chunk, KV head).  The grid covers nchunks chunks of every request; chunks
//     past L_b leave at once.  Small independent workgroups let the hardware dispatcher keep
//     every CU saturated with loads across the ragged lengths, which measured faster than
//     any persistent per-CU assignment of the same keys.
//   * blockIdx.x % kv_heads is the KV head, so with 8 KV heads each head maps to one XCD
//     under the round-robin dispatch, together with its partial states and counters.
//   * lanes: 16 bytes of one key row per lane (LPK lanes per key); a pass of the workgroup
//     reads 4 KiB of K and 4 KiB of V, all passes of a block are issued before any math;
//     large arenas are read with the non-temporal cache policy (each row is read once).
//     Scores are reduced across the LPK lanes with DPP, the softmax max across a wave's lane
//     groups with permlane swaps, and the waves' (max, sum, acc) states merge in LDS.
//   * a request with one chunk writes its output directly.  Otherwise every chunk publishes
//     its state with device-scope stores and bumps a per-(request, head) counter; the last
//     arriver merges all chunk states in chunk order (deterministic), writes the output
//     and re-zeroes the counter, so launches can be replayed from a graph.
#include "q3t_common.hpp"

namespace q3t {

constexpr int kMaxBatch = 1024;
constexpr int kChunkRows = 64;
constexpr int kMaxChunks = 1024;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kEmpty = -1.0e30f;  // finite "no key yet" running max

struct DecodeParams {
    int B, Hq, Hkv, ctx, nchunks;
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
};

Q3T_DEVICE int mask_elem_size(int dtype) { return dtype == Q3T_F32 ? 4 : dtype == Q3T_BOOL ? 1 : 2; }

Q3T_DEVICE float load_mask(const char *m, int dtype) {
    switch (dtype) {
        case Q3T_BF16: return bf16_to_float(*reinterpret_cast<const uint16_t *>(m));
        case Q3T_F16: return (float)*reinterpret_cast<const _Float16 *>(m);
        case Q3T_F32: return *reinterpret_cast<const float *>(m);
        default: return *reinterpret_cast<const uint8_t *>(m) ? 0.0f : -INFINITY;  // bool: True attends
    }
}

// Partial score of one lane: its 16 bytes of the query row and of the key row.
template <typename T>
Q3T_DEVICE float lane_dot(const U4 &q, const U4 &k) {
    if constexpr (sizeof(T) == 2) {
        float s = dot2_bf16(q.x, k.x, 0.f);
        s = dot2_bf16(q.y, k.y, s);
        s = dot2_bf16(q.z, k.z, s);
        return dot2_bf16(q.w, k.w, s);
    } else {
        float s = __uint_as_float(q.x) * __uint_as_float(k.x);
        s += __uint_as_float(q.y) * __uint_as_float(k.y);
        s += __uint_as_float(q.z) * __uint_as_float(k.z);
        return s + __uint_as_float(q.w) * __uint_as_float(k.w);
    }
}

// Sum over each aligned group of LPK (8, 16 or 32) lanes; every lane of the group gets it.
template <int LPK>
Q3T_DEVICE float group_sum(float x) {
    x = sum8(x);
    if constexpr (LPK >= 16) x += xor8(x);
    if constexpr (LPK >= 32) x += xor16(x);
    return x;
}

// Sum / max across the lane groups of a wave (lanes that differ in the bits above the group).
template <int LPK>
Q3T_DEVICE float cross_sum(float x) {
    if constexpr (LPK <= 8) x += xor8(x);
    if constexpr (LPK <= 16) x += xor16(x);
    return x + xor32(x);
}
template <int LPK>
Q3T_DEVICE float cross_max(float x) {
    if constexpr (LPK <= 8) x = fmaxf(x, xor8(x));
    if constexpr (LPK <= 16) x = fmaxf(x, xor16(x));
    return fmaxf(x, xor32(x));
}

// RMSNorm of one bf16 row spread over LPK lanes (8 elements per lane), as the attention
// module's q_norm / k_norm compute it: fp32 sum of squares over the row, x * rsqrt(mean + eps)
// rounded to bf16, times the bf16 weight, rounded to bf16.  The sum's order is this kernel's
// (lanes, then the DPP tree); rows agree with other orders to the last bf16 bit except near
// rounding ties.
template <int LPK>
Q3T_DEVICE U4 rms_norm8(const U4 &x, const U4 &w, float eps, int width) {
    const uint32_t v[4] = {x.x, x.y, x.z, x.w}, g[4] = {w.x, w.y, w.z, w.w};
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = bf16_lo(v[i]), b = bf16_hi(v[i]);
        ss = __builtin_fmaf(a, a, ss);
        ss = __builtin_fmaf(b, b, ss);
    }
    ss = group_sum<LPK>(ss);
    const float r = __builtin_amdgcn_rsqf(ss * (1.0f / (float)width) + eps);
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t n = cvt_pk_bf16(bf16_lo(v[i]) * r, bf16_hi(v[i]) * r);
        y[i] = cvt_pk_bf16_canon(bf16_lo(n) * bf16_lo(g[i]), bf16_hi(n) * bf16_hi(g[i]));
    }
    return U4{y[0], y[1], y[2], y[3]};
}

// Cross-workgroup chunk states are written and read with device-scope (sc1) accesses, which
// are coherent across the XCDs' L2 caches without an L2 write-back.  A writer waits for its
// stores to complete (vmcnt 0) before the workgroup barrier that precedes the counter
// increment; the last workgroup reads the states only after its increment returned.
Q3T_DEVICE void publish(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
Q3T_DEVICE float collect(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
Q3T_DEVICE void wait_stores() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // all counters zero: every issued store has completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <typename T>
Q3T_DEVICE void store_out(char *base, float v) {
    if constexpr (sizeof(T) == 2)
        *reinterpret_cast<uint16_t *>(base) = (uint16_t)float_to_bf16(v);
    else
        *reinterpret_cast<float *>(base) = v;
}

// Sums of N values across the lane halves (permlane32_swap) and then across 16-lane rows
// (permlane16_swap), two values per swap: swap(a, b) leaves lanes 0-31 with the half-sums of
// a and lanes 32-63 with those of b, so every step halves the register count instead of
// reducing each value on its own.  Afterwards half[k] in half h holds element 2k + h summed
// over both halves, and quarter[m] in row g holds element 4m + kRowElem[g] summed over all
// four rows.
constexpr int kRowElem[4] = {0, 2, 1, 3};
template <int N>
Q3T_DEVICE void sum_halves(const float (&v)[N], float (&half)[N / 2]) {
#pragma unroll
    for (int k = 0; k < N / 2; ++k) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[2 * k]), __float_as_uint(v[2 * k + 1]),
                                                        false, false);
        half[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}
template <int N>
Q3T_DEVICE void sum_rows(const float (&half)[N / 2], float (&quarter)[N / 4]) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(half[2 * k]), __float_as_uint(half[2 * k + 1]),
                                                        false, false);
        quarter[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

// Reduce the lane groups' accumulators of a wave and store the wave's acc rows (R x D) to LDS.
// acc[r][e] of lane (group, cl) belongs to element e of the 16-byte chunk cl of query row r.
template <int LPK, int CW, int R, int D>
Q3T_DEVICE void store_wave_acc(float (&acc)[R][CW], float (&dst)[R][D], int lane) {
    constexpr int N = R * CW;
    float v[N];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < CW; ++e) v[r * CW + e] = acc[r][e];
    if constexpr (LPK == 32) {  // two groups: the lane halves
        float h2[N / 2];
        sum_halves<N>(v, h2);
        const int cl = lane & 31, hf = lane >> 5;
#pragma unroll
        for (int k = 0; k < N / 2; ++k) {
            const int i = 2 * k + hf;
            dst[i / CW][cl * CW + i % CW] = h2[k];
        }
    } else {
        if constexpr (LPK == 8) {  // two groups per 16-lane row first
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] += xor8(v[i]);
        }
        float h2[N / 2], q4[N / 4];
        sum_halves<N>(v, h2);
        sum_rows<N>(h2, q4);
        const int row = (lane >> 4) & 3, cl = lane & (LPK - 1);
        const int sel = kRowElem[row];
        if (LPK == 16 || (lane & 8) == 0) {
#pragma unroll
            for (int k = 0; k < N / 4; ++k) {
                const int i = 4 * k + sel;
                dst[i / CW][cl * CW + i % CW] = q4[k];
            }
        }
    }
}

// Lane geometry of a variant: one 16-byte vector of a key row per lane.
template <typename T, int D>
struct DecodeShape {
    static constexpr int ES = sizeof(T);
    static constexpr int LPK = D * ES / 16;       // lanes per key row: 8, 16 or 32
    static constexpr int CW = 16 / ES;            // elements per lane
    static constexpr int RPW = 64 / LPK;          // rows per wave per pass
    static constexpr int RPP = RPW * kWaves;      // rows per workgroup pass
    static constexpr int P = kChunkRows / RPP;    // passes per block
    static_assert(P >= 1 && kChunkRows % RPP == 0, "block must be whole passes");
};

// Waves per SIMD the register allocation aims for: the kernel is latency-bound, so the
// bf16 variants with at most two query rows per KV head are held to 80 VGPRs (6 waves),
// which they meet without spilling; wider variants keep the compiler's choice.
// bf16 launches of one or two query rows per KV head fit 80 VGPRs (6 waves per SIMD); the
// mask's per-key terms need a few more, which 5 waves per SIMD leave room for without spills
constexpr int decode_waves_per_eu(int es, int rows, bool mask) {
    return es == 2 && rows <= 2 ? (mask ? 5 : 6) : 1;
}

template <typename T, int D, int G, int SQ, bool FUSED, bool MASK, bool STREAM>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(decode_waves_per_eu(sizeof(T), G * SQ, MASK))))
decode_attention_kernel(DecodeParams p) {
    constexpr int R = G * SQ;
    using S = DecodeShape<T, D>;
    constexpr int LPK = S::LPK, CW = S::CW, RPW = S::RPW, RPP = S::RPP, P = S::P, ES = S::ES;
    static_assert(!FUSED || (ES == 2 && D == 128 && SQ <= 2), "fused path: bf16, D=128, one or two tokens");

    __shared__ float sm_acc[kWaves][R][D];
    __shared__ float sm_ml[kWaves][R][2];
    __shared__ U4 sm_new[FUSED ? 2 : 1][FUSED ? SQ : 1][16];  // rotated new keys, new values

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane / LPK, cl = lane % LPK;
    const int h = blockIdx.x % p.Hkv;
    const int rest = blockIdx.x / p.Hkv;
    const int c = rest % p.nchunks, b = rest / p.nchunks;

    // what depends only on (request, head) is requested together with the position: the query
    // rows and, fused, the cos/sin rows of the step's tokens and the new key/value rows (16
    // bytes per lane each; lane group t holds token t's new rows)
    const int64_t pb = p.pos[b];
    U4 qr[R];
    U4 nk, nv, cv[SQ], sv[SQ];
    if constexpr (FUSED) {
#pragma unroll
        for (int t = 0; t < SQ; ++t) {
            cv[t] = load16(p.cs + (b * p.cs_sb + t * p.cs_ss) * 2 + cl * 16);
            sv[t] = load16(p.sn + (b * p.cs_sb + t * p.cs_ss) * 2 + cl * 16);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int qi = r / G, hq = h * G + r % G;
            qr[r] = load16(p.q + (b * p.q_sb + qi * p.q_ss + hq * p.q_sh) * ES + cl * 16);
        }
        const int tk = grp < SQ ? grp : SQ - 1;
        nk = load16(p.nk + (b * p.nk_sb + tk * p.nk_ss + h * p.nk_sh) * ES + cl * 16);
        nv = load16(p.nv + (b * p.nv_sb + tk * p.nv_ss + h * p.nv_sh) * ES + cl * 16);
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int qi = r / G, hq = h * G + r % G;
            qr[r] = load16(p.q + (b * p.q_sb + qi * p.q_ss + hq * p.q_sh) * ES + cl * 16);
        }
    }

    const int L = (pb >= 0 && pb < p.ctx) ? (int)pb + 1 : 0;
    if (L == 0) {  // no valid position: attends nothing, zero rows (written by chunk 0)
        if (c == 0)
            for (int t = tid; t < R * D; t += kThreads) {
                const int r = t / D, d = t % D, qi = r / G, hq = h * G + r % G;
                store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, 0.f);
            }
        return;
    }
    const int nblocks = (L + kChunkRows - 1) / kChunkRows;
    const int per = (nblocks + p.nchunks - 1) / p.nchunks;  // blocks per chunk
    const int n = (nblocks + per - 1) / per;                // live chunks of this request
    if (c >= n) return;
    const int j0 = c * per * kChunkRows;
    const int j1 = min(L, j0 + per * kChunkRows);
    // fused: keys L-SQ ... L-1 are the step's new keys; the last chunk writes them and attends
    // them from LDS, no chunk reads them from the arena
    const bool with_new = FUSED && c == n - 1;
    const int jend = FUSED ? min(j1, L - SQ) : j1;  // arena keys of this chunk: [j0, jend)

    const char *kb = p.k + ((p.offs ? p.offs[b] : (int64_t)b * p.k_sb) + h * p.k_sh) * ES;
    const char *vb = p.v + ((p.offs ? p.offs[b] : (int64_t)b * p.v_sb) + h * p.v_sh) * ES;
    const int kst = (int)(p.k_st * ES), vst = (int)(p.v_st * ES);
    const bool same_stride = kst == vst;
    // K/V rows 0 .. ctx-1 of (b, h) through buffer resources (32-bit row offsets)
    const auto krs = buffer_rsrc(uniform_ptr(kb), (uint32_t)((p.ctx - 1) * kst + D * ES));
    const auto vrs = buffer_rsrc(uniform_ptr(vb), (uint32_t)((p.ctx - 1) * vst + D * ES));

    if constexpr (FUSED) {
        if (p.qnw) {
            const U4 w = load16(p.qnw + cl * 16);
#pragma unroll
            for (int r = 0; r < R; ++r) qr[r] = rms_norm8<LPK>(qr[r], w, p.eps, D);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) qr[r] = rope_half8(qr[r], xor8_u4(qr[r]), cv[r / G], sv[r / G], cl < 8);
        if (with_new && wave == 0 && grp < SQ && L - SQ + grp >= 0) {
            // lane group t of wave 0 holds token t's whole rows, so the half exchange (and the
            // norm's row sum) sees every element
            const U4 ct = SQ == 1 || grp == 0 ? cv[0] : cv[SQ - 1];
            const U4 st = SQ == 1 || grp == 0 ? sv[0] : sv[SQ - 1];
            U4 kx = nk;
            if (p.knw) kx = rms_norm8<LPK>(nk, load16(p.knw + cl * 16), p.eps, D);
            const U4 kn = rope_half8(kx, xor8_u4(kx), ct, st, cl < 8);
            const int row = L - SQ + grp;
            buffer_store16(krs, (uint32_t)(row * kst) + cl * 16, kn);
            buffer_store16(vrs, (uint32_t)(row * vst) + cl * 16, nv);
            sm_new[0][grp][cl] = kn;
            sm_new[1][grp][cl] = nv;
        }
    }

    const char *mask_row = MASK ? p.mask + b * p.m_sb * mask_elem_size(p.mask_dtype) : nullptr;

    float m[R], l[R], acc[R][CW];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = kEmpty;
        l[r] = 0.f;
#pragma unroll
        for (int e = 0; e < CW; ++e) acc[r][e] = 0.f;
    }

    // one online-softmax step over P key vectors per lane (invalid ones carry -inf scores)
    auto step = [&](const U4 (&kr)[P], const U4 (&vr)[P], const int (&kidx)[P], const bool (&valid)[P],
                    const float (&mk)[P][SQ], bool rescale) {
        float s[P][R];
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int qi = r / G;
                bool ok = valid[pp];
                // several queries of a request without a mask: causal among the last keys
                if constexpr (SQ > 1 && !MASK) ok = ok && kidx[pp] <= L - SQ + qi;
                float x = group_sum<LPK>(lane_dot<T>(qr[r], kr[pp])) * p.scale_log2;
                if constexpr (MASK) x += mk[pp][qi];
                s[pp][r] = ok ? x : -INFINITY;
            }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float mb = s[0][r];
#pragma unroll
            for (int pp = 1; pp < P; ++pp) mb = fmaxf(mb, s[pp][r]);
            const float mn = fmaxf(m[r], cross_max<LPK>(mb));
            if (rescale) {  // nothing to rescale before the first block
                const float alpha = fexp2(m[r] - mn);
                l[r] *= alpha;
#pragma unroll
                for (int e = 0; e < CW; ++e) acc[r][e] *= alpha;
            }
            m[r] = mn;
#pragma unroll
            for (int pp = 0; pp < P; ++pp) {
                const float w = fexp2(s[pp][r] - mn);
                l[r] += w;
                const uint32_t x[4] = {vr[pp].x, vr[pp].y, vr[pp].z, vr[pp].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (ES == 2) {
                        acc[r][2 * i] += w * bf16_lo(x[i]);
                        acc[r][2 * i + 1] += w * bf16_hi(x[i]);
                    } else {
                        acc[r][i] += w * __uint_as_float(x[i]);
                    }
                }
            }
        }
    };

    // keys of the block at jb: rows at or past jend get an offset outside the resource, which
    // reads zeros without a memory access
    auto load_block = [&](int jb, U4 (&kr)[P], U4 (&vr)[P]) {
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
            const int j = jb + pp * RPP + wave * RPW + grp;
            const bool ok = j < jend;
            const uint32_t ko = ok ? (uint32_t)(j * kst) + cl * 16 : 0xfffffff0u;
            const uint32_t vo = ok ? (same_stride ? ko : (uint32_t)(j * vst) + cl * 16) : 0xfffffff0u;
            if constexpr (STREAM) {
                kr[pp] = buffer_load16_stream(krs, ko);
                vr[pp] = buffer_load16_stream(vrs, vo);
            } else {
                kr[pp] = buffer_load16(krs, ko);
                vr[pp] = buffer_load16(vrs, vo);
            }
        }
    };
    auto block_keys = [&](int jb, int (&kidx)[P], bool (&valid)[P]) {
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
            kidx[pp] = jb + pp * RPP + wave * RPW + grp;
            valid[pp] = kidx[pp] < jend;
        }
    };
    // mask terms of the block's keys (log2 units), requested right after the block's key and
    // value rows so that the scores wait for one round trip, not two
    auto block_mask = [&](const int (&kidx)[P], const bool (&valid)[P], float (&mk)[P][SQ]) {
#pragma unroll
        for (int pp = 0; pp < P; ++pp)
#pragma unroll
            for (int qi = 0; qi < SQ; ++qi) {
                mk[pp][qi] = 0.f;
                if constexpr (MASK) {
                    if (valid[pp])
                        mk[pp][qi] = load_mask(mask_row + (qi * p.m_ss + (int64_t)kidx[pp] * p.m_st) *
                                                              mask_elem_size(p.mask_dtype),
                                               p.mask_dtype) * kLog2e;
                }
            }
    };
    for (int jb = j0; jb < jend; jb += kChunkRows) {
        U4 kr[P], vr[P];
        int kidx[P];
        bool valid[P];
        float mk[P][SQ];
        load_block(jb, kr, vr);
        block_keys(jb, kidx, valid);
        block_mask(kidx, valid, mk);
        step(kr, vr, kidx, valid, mk, jb != j0);
    }
    if constexpr (FUSED) {
        if (with_new && wave == 0) {  // the new keys: token t's in lane group t of wave 0
            U4 kr[P], vr[P];
            int kidx[P];
            bool valid[P];
            float mk[P][SQ] = {};
            const U4 zero = {0u, 0u, 0u, 0u};
            const bool mine = grp < SQ && L - SQ + grp >= 0;
#pragma unroll
            for (int pp = 0; pp < P; ++pp) {
                kr[pp] = (pp == 0 && mine) ? sm_new[0][grp < SQ ? grp : 0][cl] : zero;
                vr[pp] = (pp == 0 && mine) ? sm_new[1][grp < SQ ? grp : 0][cl] : zero;
                kidx[pp] = L - SQ + grp;
                valid[pp] = pp == 0 && mine;
            }
            step(kr, vr, kidx, valid, mk, j0 < jend);
        }
    }

    // the wave's state: sums across its lane groups, then into LDS
#pragma unroll
    for (int r = 0; r < R; ++r) l[r] = cross_sum<LPK>(l[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            sm_ml[wave][r][0] = m[r];
            sm_ml[wave][r][1] = l[r];
        }
    }
    store_wave_acc<LPK, CW, R, D>(acc, sm_acc[wave], lane);
    __syncthreads();
    // from here on one wave finishes the work item; the others leave and free their slots
    if (wave != 0) return;

    constexpr int OPL = R * D / 64;  // outputs per lane
    float *part = p.partials + ((int64_t)(b * p.Hkv + h) * p.nchunks) * (R * (D + 2));
    float A[OPL], Ls[OPL], M[OPL];
#pragma unroll
    for (int i = 0; i < OPL; ++i) {
        const int t = lane + 64 * i, r = t / D, d = t % D;
        float mx = sm_ml[0][r][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, sm_ml[w][r][0]);
        float sl = 0.f, sa = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = fexp2(sm_ml[w][r][0] - mx);
            sl += sm_ml[w][r][1] * wt;
            sa += sm_acc[w][r][d] * wt;
        }
        A[i] = sa;
        Ls[i] = sl;
        M[i] = mx;
    }
    auto out_at = [&](int t) {
        const int r = t / D, d = t % D, qi = r / G, hq = h * G + r % G;
        return p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES;
    };
    if (n == 1) {
#pragma unroll
        for (int i = 0; i < OPL; ++i) store_out<T>(out_at(lane + 64 * i), A[i] * __builtin_amdgcn_rcpf(Ls[i]));
        return;
    }
    float *mine = part + (int64_t)c * (R * (D + 2));
#pragma unroll
    for (int i = 0; i < OPL; ++i) {
        const int t = lane + 64 * i, r = t / D, d = t % D;
        publish(mine + r * (D + 2) + d, A[i]);
        if (d == 0) {
            publish(mine + r * (D + 2) + D, M[i]);
            publish(mine + r * (D + 2) + D + 1, Ls[i]);
        }
    }

    // count arrivals; the last chunk of (request, head) merges every chunk state in order
    wait_stores();
    int *counter = p.counters + b * p.Hkv + h;
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
    if (!__builtin_amdgcn_readfirstlane(last)) return;
#pragma unroll
    for (int i = 0; i < OPL; ++i) {
        M[i] = kEmpty;
        Ls[i] = 0.f;
        A[i] = 0.f;
    }
    // online merge in chunk order (deterministic whichever chunk arrives last)
#pragma unroll 2
    for (int k = 0; k < n; ++k) {
        const float *st = part + (int64_t)k * (R * (D + 2));
#pragma unroll
        for (int i = 0; i < OPL; ++i) {
            const int t = lane + 64 * i, r = t / D, d = t % D;
            const float mk = collect(st + r * (D + 2) + D), lk = collect(st + r * (D + 2) + D + 1);
            const float ak = collect(st + r * (D + 2) + d);
            const float mn = fmaxf(M[i], mk);
            const float wo = fexp2(M[i] - mn), wk = fexp2(mk - mn);
            Ls[i] = Ls[i] * wo + lk * wk;
            A[i] = A[i] * wo + ak * wk;
            M[i] = mn;
        }
    }
#pragma unroll
    for (int i = 0; i < OPL; ++i) store_out<T>(out_at(lane + 64 * i), A[i] * __builtin_amdgcn_rcpf(Ls[i]));
    if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------

// The counter region has one fixed size, so that the counters of every launch sit on bytes
// that only ever hold counters (all zero between launches), whatever batch and head count
// earlier launches on the same workspace used.
constexpr int64_t kMaxCounters = 65536;  // batch * kv_heads
static int64_t counters_bytes() { return kMaxCounters * 4; }

// Chunks per (request, KV head): ceil(ctx / 64) at most; by default as many as give about
// kTargetGroups workgroups for the whole batch, two per CU of the MI355X.  Measured over
// 8 ... 128 requests (contexts U[64, 1024]), this count was the fastest at every batch size:
// fewer chunks leave small batches without parallelism, more add chunk states to merge
// and merge chains at the end of the launch (a 64-request batch runs with one chunk, no
// merge at all).
constexpr int64_t kTargetGroups = 512;

// K/V rows are read with the non-temporal policy when the launch may read more than
// kStreamBytes of them: a talker arena layer (64 requests x 1024 rows: 268 MB) is read once
// per step, so caching it only evicts other data (10% faster streamed at 8-128 requests);
// a code-predictor cache (64 requests x 16 rows: 4 MB per layer) is re-read by the next
// step and stays cached (7% slower streamed).
constexpr int64_t kStreamBytes = 16 << 20;
static int stream_kv(int64_t batch, int64_t kv_heads, int64_t ctx, int64_t row_bytes) {
    return batch * kv_heads * ctx * row_bytes * 2 >= kStreamBytes ? 1 : 0;
}
static int64_t chunk_count(int64_t batch, int64_t kv_heads, int64_t ctx, int64_t max_chunks) {
    const int64_t blocks = (ctx + kChunkRows - 1) / kChunkRows;
    if (max_chunks <= 0) {
        const int64_t units = batch * kv_heads > 0 ? batch * kv_heads : 1;
        max_chunks = (kTargetGroups + units - 1) / units;
        if (max_chunks > kMaxChunks) max_chunks = kMaxChunks;
    }
    return blocks < max_chunks ? blocks : max_chunks;
}

}  // namespace q3t

using namespace q3t;

extern "C" int64_t q3t_decode_workspace_bytes(int64_t batch, int64_t query_len, int64_t q_heads,
                                              int64_t kv_heads, int64_t head_dim, int64_t ctx,
                                              int64_t max_chunks) {
    if (batch < 0 || batch > kMaxBatch || query_len < 1 || kv_heads < 1 || q_heads < kv_heads ||
        head_dim < 1 || ctx < 1 || ctx > (1 << 20) || max_chunks > kMaxChunks)
        return -1;
    const int64_t R = (q_heads / kv_heads) * query_len;
    return counters_bytes() + batch * kv_heads * chunk_count(batch, kv_heads, ctx, max_chunks) * R * (head_dim + 2) * 4;
}

template <typename T, int D, int G, int SQ, bool F, bool M>
static void launch_decode(const DecodeParams &p, hipStream_t s) {
    const dim3 grid((uint32_t)p.B * p.Hkv * p.nchunks);
    // streamed instances only for the talker-shaped single-query launches
    if constexpr (sizeof(T) == 2 && D == 128 && SQ == 1) {
        if (p.stream) {
            hipLaunchKernelGGL((decode_attention_kernel<T, D, G, SQ, F, M, true>), grid, dim3(kThreads), 0, s, p);
            return;
        }
    }
    hipLaunchKernelGGL((decode_attention_kernel<T, D, G, SQ, F, M, false>), grid, dim3(kThreads), 0, s, p);
}

template <typename T, int D, int G>
static int dispatch_sq(const DecodeParams &p, int sq, bool fused, hipStream_t s) {
    if (fused) {
        if constexpr (sizeof(T) == 2 && D == 128) {
            if (p.has_mask) return Q3T_EUNSUPPORTED;
            if (sq == 1) launch_decode<T, D, G, 1, true, false>(p, s);
            else if (sq == 2) launch_decode<T, D, G, 2, true, false>(p, s);
            else return Q3T_EUNSUPPORTED;
            return Q3T_OK;
        } else {
            return Q3T_EUNSUPPORTED;
        }
    }
    if (sq == 1) {
        if (p.has_mask) launch_decode<T, D, G, 1, false, true>(p, s);
        else launch_decode<T, D, G, 1, false, false>(p, s);
    } else if (sq == 2) {
        if (p.has_mask) launch_decode<T, D, G, 2, false, true>(p, s);
        else launch_decode<T, D, G, 2, false, false>(p, s);
    } else {
        return Q3T_EUNSUPPORTED;
    }
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
        a->kv_heads < 1 || a->head_dim < 1 || a->ctx < 1 || a->ctx > (1 << 20) ||
        a->max_chunks > kMaxChunks)
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
        const int64_t fs[] = {a->nk_stride_b, a->nk_stride_h, a->nv_stride_b, a->nv_stride_h, a->cs_stride_b,
                              a->nk_stride_s, a->nv_stride_s, a->cs_stride_s};
        for (int64_t st : fs)
            if ((st * es) % 16) return Q3T_EINVAL;
        if (!aligned(a->new_key, 16) || !aligned(a->new_value, 16) || !aligned(a->cos, 16) ||
            !aligned(a->sin, 16))
            return Q3T_EINVAL;
    }
    // key rows are addressed by 32-bit byte offsets from a request's base
    const int64_t max_st = a->k_stride_t > a->v_stride_t ? a->k_stride_t : a->v_stride_t;
    if (max_st < 0 || a->ctx * max_st * es + a->head_dim * es > INT32_MAX) return Q3T_EUNSUPPORTED;
    const int64_t nchunks = chunk_count(a->batch, a->kv_heads, a->ctx, a->max_chunks);
    if (a->batch * a->kv_heads * nchunks > INT32_MAX) return Q3T_EUNSUPPORTED;
    const int64_t need = q3t_decode_workspace_bytes(a->batch, a->query_len, a->q_heads, a->kv_heads,
                                                    a->head_dim, a->ctx, a->max_chunks);
    if (!a->workspace || a->workspace_bytes < need || !aligned(a->workspace, 16)) return Q3T_EWORKSPACE;

    hipStream_t s = (hipStream_t)stream;
    char *ws = (char *)a->workspace;
    DecodeParams p;
    p.B = (int)a->batch;
    p.Hq = (int)a->q_heads;
    p.Hkv = (int)a->kv_heads;
    p.ctx = (int)a->ctx;
    p.nchunks = (int)nchunks;
    p.stream = stream_kv(a->batch, a->kv_heads, a->ctx, a->head_dim * es);
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
    p.nk_ss = a->nk_stride_s; p.nv_ss = a->nv_stride_s; p.cs_ss = a->cs_stride_s;
    p.counters = (int *)ws;
    p.partials = (float *)(ws + counters_bytes());
    p.qnw = nullptr;
    p.knw = nullptr;
    p.eps = a->norm_eps;
    if (a->q_norm_weight || a->k_norm_weight) {
        if (!fused || !(a->norm_eps >= 0.f)) return Q3T_EINVAL;
        if ((a->q_norm_weight && !aligned(a->q_norm_weight, 16)) ||
            (a->k_norm_weight && !aligned(a->k_norm_weight, 16)))
            return Q3T_EINVAL;
        p.qnw = (const char *)a->q_norm_weight;
        p.knw = (const char *)a->k_norm_weight;
    }

    const int g = (int)(a->q_heads / a->kv_heads);
    const int sq = (int)a->query_len;
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
