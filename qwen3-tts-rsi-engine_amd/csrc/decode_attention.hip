// Ragged grouped-query decode attention over the slot arena.
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
// Design (one launch per layer): three grids.  The bundled grid (the talker step: whole
// requests per workgroup, longest paired with shortest, bf16 MFMA tiles fed from an LDS ring;
// its own section below) reads an optional per-step plan (decode_plan.hip).  The other two
// share a per-range core (PairWork):
//   * balanced (long arenas): each KV head's keys of all requests are cut into equal shares,
//     one per workgroup, so ragged lengths do not leave the longest requests to a few
//     workgroups at the end of the launch; the shares are derived on the device from the
//     positions;
//   * chunked (small caches, the code predictor, short arenas): one workgroup per (request,
//     chunk of 64-key blocks, KV head), whose rows are requested together with its position.
// For these two:
//   * lanes: 16 bytes of one key row per lane (LPK lanes per key); a pass of the workgroup
//     reads 4 KiB of K and 4 KiB of V, all passes of a block are issued before any math;
//     large arenas are read with the non-temporal cache policy (each row is read once).
//     Scores are reduced across the LPK lanes with DPP, the softmax max across a wave's lane
//     groups with permlane swaps, and the waves' (max, sum, acc) states merge in LDS.
//   * a (request, head) covered by several workgroups combines their states through the
//     workspace (finish_split): the last one to arrive merges in part order, writes the
//     output and re-zeroes the pair's counter, so launches can be replayed from a graph.
#include "decode_params.hpp"

#include <mutex>

namespace q3t {

constexpr int kMaxBatch = 1024;
constexpr int kChunkRows = 64;
constexpr int kMaxChunks = 1024;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kEmpty = -1.0e30f;  // finite "no key yet" running max
constexpr int kMinShare = 32;       // balanced grid: fewest keys per workgroup

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

// The work of one workgroup on one (request, KV head) pair over a key range [j0, j1): the
// online softmax of the pair's G * SQ query rows, shared by both grids below.
//   load_rows  requests the rows that depend only on (request, head): the query rows and,
//              fused, the step's cos/sin rows and new key/value rows (16 bytes per lane
//              each; lane group t holds token t's new rows).  Callers issue it before the
//              request's key count is known.
//   attend     streams the arena keys of the range in 64-key blocks (every pass of a block
//              issued before any math; with PIPE the next block is requested before the
//              current one is folded in, which costs a second block of registers), folds in the step's new keys when `finisher`
//              (fused: rotated, written to the arena at L-SQ ... L-1 and attended from LDS;
//              no workgroup reads those arena rows in the same launch), and leaves the
//              range's merged state in wave 0: for output t = lane + 64 i (query row
//              t / D, dim t % D) the unnormalised accumulator A[i], the weight sum Ls[i]
//              and the running maximum Mx[i] in scaled log2 units.
template <typename T, int D, int G, int SQ, int FUSE, bool MASK, bool STREAM, bool PIPE>
struct PairWork {
    // FUSE: 0 attention only, 1 the fused step, 2 the fused step with its q/k norms (a separate
    // instance: the norm code, even unexecuted, slowed the fused bundled kernel by 1.8 us)
    static constexpr bool FUSED = FUSE > 0, NORM = FUSE > 1;
    static constexpr int R = G * SQ;
    using S = DecodeShape<T, D>;
    static constexpr int LPK = S::LPK, CW = S::CW, RPW = S::RPW, RPP = S::RPP, P = S::P, ES = S::ES;
    static constexpr int OPL = R * D / 64;  // outputs per lane of wave 0
    static constexpr int HD = D;
    static_assert(!FUSED || (ES == 2 && D == 128 && SQ <= 2), "fused path: bf16, D=128, one or two tokens");

    struct Lds {
        float acc[kWaves][R][D];
        float ml[kWaves][R][2];
    };
    using NewRows = U4[2][FUSED ? SQ : 1][16];  // rotated new keys, new values (fused)

    U4 qr[R];
    U4 nk, nv, cv[SQ], sv[SQ];

    Q3T_DEVICE void load_rows(const DecodeParams &p, int b, int h) {
        const int lane = threadIdx.x & 63, grp = lane / LPK, cl = lane % LPK;
        if constexpr (FUSED) {
#pragma unroll
            for (int t = 0; t < SQ; ++t) {
                cv[t] = load16(p.cs + (b * p.cs_sb + t * p.cs_ss) * 2 + cl * 16);
                sv[t] = load16(p.sn + (b * p.cs_sb + t * p.cs_ss) * 2 + cl * 16);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int qi = r / G, hq = h * G + r % G;
            qr[r] = load16(p.q + (b * p.q_sb + qi * p.q_ss + hq * p.q_sh) * ES + cl * 16);
        }
        if constexpr (FUSED) {
            const int tk = grp < SQ ? grp : SQ - 1;
            nk = load16(p.nk + (b * p.nk_sb + tk * p.nk_ss + h * p.nk_sh) * ES + cl * 16);
            nv = load16(p.nv + (b * p.nv_sb + tk * p.nv_ss + h * p.nv_sh) * ES + cl * 16);
        }
    }

    // Zero output rows of a request without a valid position (it attends nothing).
    static Q3T_DEVICE void write_zeros(const DecodeParams &p, int b, int h) {
        for (int t = threadIdx.x; t < R * D; t += kThreads) {
            const int r = t / D, d = t % D, qi = r / G, hq = h * G + r % G;
            store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, 0.f);
        }
    }

    // Wave 0: final output rows A / Ls of request b.
    static Q3T_DEVICE void write_out(const DecodeParams &p, int b, int h, const float (&A)[OPL],
                                     const float (&Ls)[OPL]) {
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int i = 0; i < OPL; ++i) {
            const int t = lane + 64 * i, r = t / D, d = t % D, qi = r / G, hq = h * G + r % G;
            store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES,
                         A[i] * __builtin_amdgcn_rcpf(Ls[i]));
        }
    }

    Q3T_DEVICE void attend(const DecodeParams &p, int b, int h, int L, int j0, int j1, bool finisher,
                           Lds &lds, NewRows &snew, float (&A)[OPL], float (&Ls)[OPL], float (&Mx)[OPL]) {
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int grp = lane / LPK, cl = lane % LPK;
        const bool with_new = FUSED && finisher;
        const int jend = FUSED ? min(j1, L - SQ) : j1;  // arena keys of the range: [j0, jend)

        const char *kb = p.k + ((p.offs ? p.offs[b] : (int64_t)b * p.k_sb) + h * p.k_sh) * ES;
        const char *vb = p.v + ((p.offs ? p.offs[b] : (int64_t)b * p.v_sb) + h * p.v_sh) * ES;
        const int kst = (int)(p.k_st * ES), vst = (int)(p.v_st * ES);
        const bool same_stride = kst == vst;
        // K/V rows 0 .. ctx-1 of (b, h) through buffer resources (32-bit row offsets)
        const auto krs = buffer_rsrc(uniform_ptr(kb), (uint32_t)((p.ctx - 1) * kst + D * ES));
        const auto vrs = buffer_rsrc(uniform_ptr(vb), (uint32_t)((p.ctx - 1) * vst + D * ES));
        const char *mask_row = MASK ? p.mask + b * p.m_sb * mask_elem_size(p.mask_dtype) : nullptr;

        // keys of the block at jb: rows at or past jend get an offset outside the resource,
        // which reads zeros without a memory access
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

        // with PIPE the first block is requested before the query prologue and every later
        // block while the one before it is being folded in; without, each block after the
        // previous one (fewer registers: the chunked grid's rows arrive with the position)
        U4 kr[PIPE ? P : 1], vr[PIPE ? P : 1];
        if constexpr (PIPE) load_block(j0, kr, vr);

        U4 q[R];
#pragma unroll
        for (int r = 0; r < R; ++r) q[r] = qr[r];
        if constexpr (FUSED) {
            if (NORM && p.qnw) {
                const U4 w = load16(p.qnw + cl * 16);
#pragma unroll
                for (int r = 0; r < R; ++r) q[r] = rms_norm8<LPK>(q[r], w, p.eps, D);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) q[r] = rope_half8(q[r], xor8_u4(q[r]), cv[r / G], sv[r / G], cl < 8);
            if (with_new && wave == 0 && grp < SQ && L - SQ + grp >= 0) {
                // lane group t of wave 0 holds token t's whole rows, so the half exchange (and
                // the norm's row sum) sees every element
                const U4 ct = SQ == 1 || grp == 0 ? cv[0] : cv[SQ - 1];
                const U4 st = SQ == 1 || grp == 0 ? sv[0] : sv[SQ - 1];
                U4 kx = nk;
                if (NORM && p.knw) kx = rms_norm8<LPK>(nk, load16(p.knw + cl * 16), p.eps, D);
                const U4 kn = rope_half8(kx, xor8_u4(kx), ct, st, cl < 8);
                const int row = L - SQ + grp;
                buffer_store16(krs, (uint32_t)(row * kst) + cl * 16, kn);
                buffer_store16(vrs, (uint32_t)(row * vst) + cl * 16, nv);
                snew[0][grp][cl] = kn;
                snew[1][grp][cl] = nv;
            }
        }


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
                    float x = group_sum<LPK>(lane_dot<T>(q[r], kr[pp])) * p.scale_log2;
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

        // mask terms of keys (log2 units), requested right after the block's key and value
        // rows so that the scores wait for one round trip, not two
        auto key_mask = [&](const int (&kidx)[P], const bool (&valid)[P], float (&mk)[P][SQ]) {
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
        auto block_keys = [&](int jb, int (&kidx)[P], bool (&valid)[P]) {
#pragma unroll
            for (int pp = 0; pp < P; ++pp) {
                kidx[pp] = jb + pp * RPP + wave * RPW + grp;
                valid[pp] = kidx[pp] < jend;
            }
        };
        if constexpr (PIPE) {
            // two register buffers in turn (the loop handles two blocks per trip, so neither
            // buffer is ever copied): while one block is folded in, the next one is in flight.
            // The next block is requested unconditionally (rows past the range read zeros from
            // outside the buffer resource, without a memory access), so the number of loads in
            // flight is the same on every path and each block waits only for its own loads.
            U4 kb2[P], vb2[P];
            for (int jb = j0; jb < jend; jb += 2 * kChunkRows) {
                int kidx[P];
                bool valid[P];
                float mk[P][SQ];
                const int j2 = jb + kChunkRows;
                load_block(j2, kb2, vb2);
                block_keys(jb, kidx, valid);
                key_mask(kidx, valid, mk);
                step(kr, vr, kidx, valid, mk, jb != j0);
                if (j2 >= jend) break;
                load_block(j2 + kChunkRows, kr, vr);
                block_keys(j2, kidx, valid);
                key_mask(kidx, valid, mk);
                step(kb2, vb2, kidx, valid, mk, true);
            }
        } else {
            for (int jb = j0; jb < jend; jb += kChunkRows) {
                U4 kb_[P], vb_[P];
                int kidx[P];
                bool valid[P];
                float mk[P][SQ];
                load_block(jb, kb_, vb_);
                block_keys(jb, kidx, valid);
                key_mask(kidx, valid, mk);
                step(kb_, vb_, kidx, valid, mk, jb != j0);
            }
        }
        if constexpr (FUSED) {
            if (with_new && wave == 0) {  // the new keys: token t's in lane group t of wave 0
                U4 kr[P], vr[P];
                int kidx[P];
                bool valid[P];
                float mk[P][SQ];
                const U4 zero = {0u, 0u, 0u, 0u};
                const bool mine = grp < SQ && L - SQ + grp >= 0;
#pragma unroll
                for (int pp = 0; pp < P; ++pp) {
                    kr[pp] = (pp == 0 && mine) ? snew[0][grp < SQ ? grp : 0][cl] : zero;
                    vr[pp] = (pp == 0 && mine) ? snew[1][grp < SQ ? grp : 0][cl] : zero;
                    kidx[pp] = L - SQ + grp;
                    valid[pp] = pp == 0 && mine;
                }
                key_mask(kidx, valid, mk);
                step(kr, vr, kidx, valid, mk, j0 < jend);
            }
        }

        // the wave's state: sums across its lane groups, then into LDS
#pragma unroll
        for (int r = 0; r < R; ++r) l[r] = cross_sum<LPK>(l[r]);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                lds.ml[wave][r][0] = m[r];
                lds.ml[wave][r][1] = l[r];
            }
        }
        store_wave_acc<LPK, CW, R, D>(acc, lds.acc[wave], lane);
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int i = 0; i < OPL; ++i) {
            const int t = lane + 64 * i, r = t / D, d = t % D;
            float mx = lds.ml[0][r][0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, lds.ml[w][r][0]);
            float sl = 0.f, sa = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float wt = fexp2(lds.ml[w][r][0] - mx);
                sl += lds.ml[w][r][1] * wt;
                sa += lds.acc[w][r][d] * wt;
            }
            A[i] = sa;
            Ls[i] = sl;
            Mx[i] = mx;
        }
    }
};

// A (request, head) pair split over n workgroups: this one holds part k in registers (wave 0).
// One counter word per pair counts arrivals (low 16 bits) and published states (high 16
// bits).  A workgroup that is not the last to arrive publishes its state with device-scope
// stores, waits for them to complete and then counts itself published; the last arriver does
// not publish: it waits until every other part is published (those workgroups have arrived,
// so they are running and finish publishing without waiting on anything), merges the parts in
// part order with its own from registers (the same order whichever part arrives last), writes
// the output and zeroes the counter for the next launch (no memset node in a graph).  A
// published wait longer than kSpinLimit polls (never expected) gives NaN rows rather than a
// hang.
constexpr int kSpinLimit = 1 << 22;

template <typename Work, typename PartAt>
Q3T_DEVICE void finish_split(const DecodeParams &p, int b, int h, int n, int k, float *mine,
                             PartAt part_at, float (&A)[Work::OPL], float (&Ls)[Work::OPL],
                             float (&Mx)[Work::OPL]) {
    constexpr int OPL = Work::OPL, DD = Work::HD;
    const int lane = threadIdx.x & 63;
    int *counter = p.counters + b * p.Hkv + h;
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if ((old & 0xffff) != n - 1) {
#pragma unroll
        for (int i = 0; i < OPL; ++i) {
            const int t = lane + 64 * i, r = t / DD, d = t % DD;
            publish(mine + r * (DD + 2) + d, A[i]);
            if (d == 0) {
                publish(mine + r * (DD + 2) + DD, Mx[i]);
                publish(mine + r * (DD + 2) + DD + 1, Ls[i]);
            }
        }
        wait_stores();
        if (lane == 0) __hip_atomic_fetch_add(counter, 1 << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    int ready = old >> 16;
    bool failed = false;
    for (int tries = 0; ready < n - 1; ++tries) {
        if (tries >= kSpinLimit) {
            failed = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        int v = 0;
        if (lane == 0) v = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ready = __builtin_amdgcn_readfirstlane(v) >> 16;
    }
    float a[OPL], s[OPL], mm[OPL];
#pragma unroll
    for (int i = 0; i < OPL; ++i) {
        a[i] = 0.f;
        s[i] = 0.f;
        mm[i] = kEmpty;
    }
    for (int kk = 0; kk < n; ++kk) {
        const float *st = kk == k ? nullptr : part_at(kk);
#pragma unroll
        for (int i = 0; i < OPL; ++i) {
            const int t = lane + 64 * i, r = t / DD, d = t % DD;
            float ak = A[i], lk = Ls[i], mk = Mx[i];
            if (st) {
                mk = collect(st + r * (DD + 2) + DD);
                lk = collect(st + r * (DD + 2) + DD + 1);
                ak = collect(st + r * (DD + 2) + d);
            }
            const float mn = fmaxf(mm[i], mk);
            const float wo = fexp2(mm[i] - mn), wk = fexp2(mk - mn);
            s[i] = s[i] * wo + lk * wk;
            a[i] = a[i] * wo + ak * wk;
            mm[i] = mn;
        }
    }
    if (failed) {
#pragma unroll
        for (int i = 0; i < OPL; ++i) a[i] = __builtin_nanf("");
    }
    Work::write_out(p, b, h, a, s);
    if (lane == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- chunked grid: one workgroup per (request, chunk, KV head) ------------------------
// For short contexts (the code predictor's 16-row caches): every pair's rows are requested
// together with its position, so a workgroup's whole life is two memory round trips.
template <typename T, int D, int G, int SQ, int FUSE, bool MASK, bool STREAM>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(decode_waves_per_eu(sizeof(T), G * SQ, MASK))))
decode_chunks_kernel(DecodeParams p) {
    using Work = PairWork<T, D, G, SQ, FUSE, MASK, STREAM, false>;
    constexpr bool FUSED = Work::FUSED;
    constexpr int OPL = Work::OPL, R = Work::R;
    __shared__ typename Work::Lds lds;
    __shared__ typename Work::NewRows snew;

    const int h = blockIdx.x % p.Hkv;
    const int rest = blockIdx.x / p.Hkv;
    const int c = rest % p.nchunks, b = rest / p.nchunks;

    const int64_t pb = p.pos[b];
    Work work;
    work.load_rows(p, b, h);
    const int L = (pb >= 0 && pb < p.ctx) ? (int)pb + 1 : 0;
    if (L == 0) {  // no valid position: attends nothing, zero rows (written by chunk 0)
        if (c == 0) Work::write_zeros(p, b, h);
        return;
    }
    const int nblocks = (L + kChunkRows - 1) / kChunkRows;
    const int per = (nblocks + p.nchunks - 1) / p.nchunks;  // blocks per chunk
    const int n = (nblocks + per - 1) / per;                // live chunks of this request
    if (c >= n) return;
    const int j0 = c * per * kChunkRows;
    const int j1 = min(L, j0 + per * kChunkRows);
    float A[OPL], Ls[OPL], Mx[OPL];
    work.attend(p, b, h, L, j0, j1, c == n - 1, lds, snew, A, Ls, Mx);
    if ((threadIdx.x >> 6) != 0) return;
    if (n == 1) {
        Work::write_out(p, b, h, A, Ls);
        return;
    }
    float *part = p.partials + ((int64_t)(b * p.Hkv + h) * p.nchunks) * (R * (D + 2));
    finish_split<Work>(p, b, h, n, c, part + (int64_t)c * (R * (D + 2)),
                       [&](int kk) { return part + (int64_t)kk * (R * (D + 2)); }, A, Ls, Mx);
}

// ---- balanced grid: equal shares of each KV head's ragged key space ---------------------
// The pairs (b, h) of one KV head laid end to end form a key space of W = sum_b w_b keys,
// w_b = max(L_b, 1) (a request without a valid position keeps one key slot, whose owner
// writes its zero rows).  Workgroup i of the head's M covers keys [i W / M, (i + 1) W / M):
// every workgroup streams the same number of keys, whatever the spread of the lengths, so
// they all finish together instead of leaving the longest requests to a few workgroups at
// the end of the launch.  A range crosses request boundaries: it is processed as segments,
// one per request it touches, in key order.  A segment that is a whole request writes its
// output; the parts of a split request are combined by finish_split.  Parts of a request
// always sit in consecutive workgroups, and a request's last part is the first segment of
// its workgroup, so the states that the last arriver waits for were mostly published long
// before.  The lengths and their prefix sums are computed by every workgroup from the
// positions (one load round trip, as a single pair's position costs), so the split needs no
// preparation launch and follows positions rewritten between graph replays.
// The balanced kernel keeps two blocks of K/V rows in registers per lane (PIPE) and may use
// the registers of 2 waves per SIMD: the default grid (256 workgroups, one per CU) needs one,
// and every variant then compiles without spilling.  Measured on contexts up to 4096 rows,
// 32 workgroups per KV head (one per CU) beat 64-256: the share of each is longer, so the
// per-segment costs (query rows, the state merge) weigh less.
constexpr bool kBalancedPipe = true;
constexpr int balanced_waves_per_eu(int rows) { return rows <= 2 ? 2 : 1; }

template <typename T, int D, int G, int SQ, int FUSE, bool MASK, bool STREAM>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(balanced_waves_per_eu(G * SQ))))
decode_balanced_kernel(DecodeParams p) {
    using Work = PairWork<T, D, G, SQ, FUSE, MASK, STREAM, kBalancedPipe>;
    constexpr bool FUSED = Work::FUSED;
    constexpr int OPL = Work::OPL, R = Work::R;
    constexpr int PER = kMaxBatch / kThreads;  // requests per thread at most
    __shared__ typename Work::Lds lds[2];      // alternate segments: wave 0 may still read one
    __shared__ typename Work::NewRows snew;
    __shared__ int sm_pre[kMaxBatch + 1];      // exclusive prefix sums of w_b
    __shared__ int sm_len[kMaxBatch];          // L_b, 0 without a valid position
    __shared__ int sm_wave[kWaves];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x % p.Hkv;
    const int wi = blockIdx.x / p.Hkv;
    {
        const int per = (p.B + kThreads - 1) / kThreads;
        int w[PER];
        int total = 0;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int b = tid * per + e;
            w[e] = 0;
            if (e < per && b < p.B) {
                const int64_t pb = p.pos[b];
                const int L = (pb >= 0 && pb < p.ctx) ? (int)pb + 1 : 0;
                sm_len[b] = L;
                w[e] = L > 0 ? L : 1;
            }
            total += w[e];
        }
        int x = total;  // inclusive scan over the wave
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        if (lane == 63) sm_wave[wave] = x;
        __syncthreads();
        int run = x - total;
        for (int v = 0; v < wave; ++v) run += sm_wave[v];
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int b = tid * per + e;
            if (e < per && b < p.B) {
                sm_pre[b] = run;
                run += w[e];
            }
        }
        if (tid == 0) sm_pre[p.B] = sm_wave[0] + sm_wave[1] + sm_wave[2] + sm_wave[3];
        __syncthreads();
    }
    const int W = __builtin_amdgcn_readfirstlane(sm_pre[p.B]);
    // at most one workgroup per kMinShare keys (and never more than keys): every range is
    // non-empty, so every part of a split request arrives
    int M = W / kMinShare;
    M = M < 1 ? 1 : (M > p.splits ? p.splits : M);
    if (wi >= M) return;
    const int s = (int)((int64_t)wi * W / M), e = (int)((int64_t)(wi + 1) * W / M);
    int b;  // the request holding key s: the last b with sm_pre[b] <= s
    {
        int lo = 0, hi = p.B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (__builtin_amdgcn_readfirstlane(sm_pre[mid]) <= s) lo = mid;
            else hi = mid - 1;
        }
        b = lo;
    }
    for (int seg = 0;; ++seg, ++b) {
        const int pb0 = __builtin_amdgcn_readfirstlane(sm_pre[b]);
        const int pb1 = __builtin_amdgcn_readfirstlane(sm_pre[b + 1]);
        const int L = __builtin_amdgcn_readfirstlane(sm_len[b]);
        const int j0 = max(s, pb0) - pb0, j1 = min(e, pb1) - pb0;
        const bool whole = j0 == 0 && pb0 + j1 == pb1;
        const bool last_segment = pb1 >= e;
        if (L == 0) {  // one key slot, always whole: zero rows
            Work::write_zeros(p, b, h);
        } else {
            Work work;
            work.load_rows(p, b, h);
            float A[OPL], Ls[OPL], Mx[OPL];
            work.attend(p, b, h, L, j0, j1, j1 == L, lds[seg & 1], snew, A, Ls, Mx);
            if (wave == 0) {
                if (whole) {
                    Work::write_out(p, b, h, A, Ls);
                } else {
                    // the request's parts: workgroups ia ... iz (the ones holding its first and
                    // last key); a part's state sits in slot 0 of its workgroup when the request
                    // is the workgroup's first segment, else in slot 1
                    const int ia = (int)(((int64_t)(pb0 + 1) * M - 1) / W);
                    const int iz = (int)(((int64_t)pb1 * M - 1) / W);
                    auto part_at = [&](int kk) {
                        const int j = ia + kk;
                        const int slot = (j > ia || (int)((int64_t)j * W / M) == pb0) ? 0 : 1;
                        return p.partials + ((int64_t)(h * p.splits + j) * 2 + slot) * (R * (D + 2));
                    };
                    float *mine = p.partials + ((int64_t)(h * p.splits + wi) * 2 + (seg == 0 ? 0 : 1)) * (R * (D + 2));
                    finish_split<Work>(p, b, h, iz - ia + 1, wi - ia, mine, part_at, A, Ls, Mx);
                }
            }
        }
        if (last_segment) break;
    }
}

// ---- bundled grid: whole requests in length-balanced bundles, bf16 MFMA tiles -------------
// For arena-sized single-token launches over many requests (the talker step).  The grid is one
// workgroup per CU: Hkv x M workgroups, workgroup (m, h) owning bundle m of KV head h, which
// holds the requests of length ranks m, 2M-1-m, 2M+m, 4M-1-m (snake order): the longest
// requests are paired with the shortest, so bundles carry about the same number of keys, and
// each request is attended by one workgroup (no cross-workgroup merge, no workspace).  The
// bundle's four (request, length) entries come from the step's plan (decode_plan.hip) in the
// same scalar round trip as the kernel arguments, or, without a plan for this batch, from a
// ranking of the positions that every wave does in its own LDS copy of the keys.
//   * K/V rows stream through two LDS stages of 64 keys, 16 per wave, loaded by global-to-LDS
//     buffer loads one stage ahead of the one being scored; the waits are explicit, and the
//     stream runs across request boundaries.  Masked launches bring each key's 4-byte mask
//     word with its rows and add the term to its score.  The ring and the request rows keep
//     one workgroup per CU.
//   * each wave scores its 16 keys against the request's G query rows with
//     v_mfma_f32_16x16x32_bf16 (S^T = K . Q^T: A = 16 key rows from LDS, B = the query rows as
//     16 columns, G of them live), keeps an online softmax per column in log2 units, and
//     accumulates O^T += V^T . P^T with v_mfma_f32_16x16x16_bf16 (A = V^T by the transposing
//     LDS read, B = the bf16 weights straight from the S^T registers).  Rows sit in LDS with
//     their 16-byte chunks XOR-swizzled (K chunk ch of row r at ch ^ r, V at ch ^ 2r mod 16),
//     which keeps both reads on distinct banks.
//   * request k's rows (query rows and, fused, the cos/sin rows and new K/V rows) are loaded by
//     wave k % 4 into one shared area ahead of the stream and rotated there while the first
//     stages are in flight; fused launches place the new key and value in the ring at row
//     L-1, so the step's key is attended like any other, and store them into the arena right
//     after the first stage's wait (a store shares the load counter that the ring waits on).
//   * at the end of a request the waves' (max, sum, accumulator) states merge in LDS (two
//     buffers by request parity); the outputs are stored after the stream.
constexpr int kBundleGroups = 256;    // workgroups of a launch: one per CU
constexpr int kBundleMaxBatch = 128;  // requests ranked per launch: two per lane
constexpr int kBundleMaxSeg = 4;      // requests per bundle
// K/V stages: the one being scored and the next one in flight.  Measured on the talker step:
// two stages in flight (three LDS stages) 27.6 us against 26.5 us with one; two only over a
// workgroup's last 4 or 8 stages, no gain either.
constexpr int kRingStages = 2;
constexpr int kStageKeys = 64;
constexpr int kWaveKeys = kStageKeys / kWaves;  // 16
constexpr int kRowBytes = 256;                  // bf16 rows of D = 128
constexpr int kWaveStage = 2 * kWaveKeys * kRowBytes;  // K rows then V rows: 8 KiB
constexpr int kStageBytes = kWaves * kWaveStage;       // 32 KiB
constexpr int kStageLoads = 2 * kWaveKeys * kRowBytes / 1024;  // 1 KiB loads per wave and stage: 8
constexpr float kRescaleLog2 = 8.0f;  // the running maximum moves when exceeded by more than this

template <int G>
struct BundleLds {
    char ring[kRingStages][kStageBytes];
    // per request (shared by the waves): rows 0..G-1 query, 4 cos, 5 sin, 6 new K, 7 new V
    char head[kBundleMaxSeg][8][kRowBytes];
    float acc[2][kWaves][G][128];
    float ml[2][kWaves][G][2];
    alignas(16) uint16_t outq[kBundleMaxSeg][G][128];  // bf16 outputs, stored after the stream
    alignas(16) int keys[kWaves][kBundleMaxBatch];  // each wave's copy of the ranking keys
    uint32_t maskw[kRingStages][kWaves][64];        // masked: the mask words of a stage's rows
};

// The bundle's requests as wave-uniform values (scalar registers): request index, length and
// row-0 element offsets of its K and V rows, selected by a uniform index without memory (four
// named slots rather than arrays, which the compiler would place in scratch memory when
// indexed by a run-time value).
template <typename X>
struct Slots4 {
    X s0, s1, s2, s3;
    Q3T_DEVICE X get(int k) const { return k == 0 ? s0 : k == 1 ? s1 : k == 2 ? s2 : s3; }
    Q3T_DEVICE void set(int k, X v) {
        if (k == 0) s0 = v;
        else if (k == 1) s1 = v;
        else if (k == 2) s2 = v;
        else s3 = v;
    }
};

// NORM: the fused q/k RMSNorm is compiled in (a separate instance: its code, even unexecuted,
// cost the talker step 1.8 us per launch in the instance without norms).  MASK: an additive or
// bool (batch, 1, ctx) mask with unit key stride is added to the scores of keys 0 ... pos[b]
// (SlotGraph.compute hands every layer one, continuous.py:188-197): each wave loads the mask
// words of its 16 rows of a stage with the stage, one 4-byte load per row into LDS.  MK: 0 no
// mask, 1 a bf16 mask (SlotGraph.compute's, in the model's dtype: a branch-free term), 2 any
// other dtype.  With one wave per SIMD the scoring instructions sit on each stage's critical
// path, so the terms' byte offsets are fixed once per request (keys 4g ... 4g+3 of a lane start
// at a multiple of 4): a per-element 64-bit index and dtype switch cost the talker step 3.9 us.
template <int G, bool FUSED, bool STREAM, bool NORM, int MK>
__global__ void __launch_bounds__(kThreads) decode_bundled_kernel(const int32_t *plan, int nb, int hkv, int bundles, DecodeParams p) {
    constexpr bool MASK = MK != 0;
    static_assert(G >= 1 && G <= 4, "query rows are the first G of 16 MFMA columns, four LDS rows");
    __shared__ __attribute__((aligned(16))) BundleLds<G> s;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases stay scalar
    const int h = blockIdx.x % hkv, m = blockIdx.x / hkv, M = bundles;
    // The plan entries of this bundle, the plan's batch and every line of the argument block in
    // one scalar round trip: the plan pointer and the sizes its addresses need are the leading
    // kernel arguments, which the hardware preloads into scalar registers.  The plan's bundle
    // section is (B, 0) and then four (b, L) pairs per bundle.
    auto bundle_rank = [&](int i) { return (i >> 1) * 2 * M + ((i & 1) ? 2 * M - 1 - m : m); };
    uint64_t e[kBundleMaxSeg] = {0, 0, 0, 0};
    uint32_t plan_batch = 0;
    if (plan) {
        const uint64_t base = reinterpret_cast<uint64_t>(plan);
        uint64_t a[kBundleMaxSeg];
#pragma unroll
        for (int i = 0; i < kBundleMaxSeg; ++i)
            a[i] = base + 8 + 8 * (uint64_t)(m * kBundleMaxSeg + i);
        constexpr int BYTES = 32 + (int)sizeof(DecodeParams);
        static_assert(BYTES <= 8 * 64, "eight 64-byte lines at most");
        const uint64_t ka = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
        uint32_t d0, d1, d2, d3, d4, d5, d6, d7;
        asm volatile("s_load_dwordx2 %[e0], %[a0], 0x0\n\ts_load_dwordx2 %[e1], %[a1], 0x0\n\t"
                     "s_load_dwordx2 %[e2], %[a2], 0x0\n\ts_load_dwordx2 %[e3], %[a3], 0x0\n\t"
                     "s_load_dword %[nb], %[base], 0x0\n\t"
                     "s_load_dword %[d0], %[ka], 0x0\n\ts_load_dword %[d1], %[ka], 0x40\n\t"
                     "s_load_dword %[d2], %[ka], 0x80\n\ts_load_dword %[d3], %[ka], 0xc0\n\t"
                     "s_load_dword %[d4], %[ka], %[o4]\n\ts_load_dword %[d5], %[ka], %[o5]\n\t"
                     "s_load_dword %[d6], %[ka], %[o6]\n\ts_load_dword %[d7], %[ka], %[o7]\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : [e0] "=&s"(e[0]), [e1] "=&s"(e[1]), [e2] "=&s"(e[2]), [e3] "=&s"(e[3]),
                       [nb] "=&s"(plan_batch), [d0] "=&s"(d0), [d1] "=&s"(d1), [d2] "=&s"(d2), [d3] "=&s"(d3),
                       [d4] "=&s"(d4), [d5] "=&s"(d5), [d6] "=&s"(d6), [d7] "=&s"(d7)
                     : [a0] "s"(a[0]), [a1] "s"(a[1]), [a2] "s"(a[2]), [a3] "s"(a[3]), [base] "s"(base),
                       [ka] "s"(ka), [o4] "n"(BYTES > 0x100 ? 0x100 : 0), [o5] "n"(BYTES > 0x140 ? 0x140 : 0),
                       [o6] "n"(BYTES > 0x180 ? 0x180 : 0), [o7] "n"(BYTES > 0x1c0 ? 0x1c0 : 0)
                     : "memory");
    } else {
        prefetch_kernargs<32 + sizeof(DecodeParams)>();
    }

    // weights of the fused norms (chunk c of the row), loaded with the positions and waited for
    // before any ring load is issued: a wait the compiler placed at their first use would also
    // wait for the ring's loads, which it does not count
    U4 qw = {0u, 0u, 0u, 0u}, kw = {0u, 0u, 0u, 0u};
    if constexpr (FUSED && NORM) {
        if (p.qnw) qw = load16(p.qnw + c * 16);
        if (p.knw) kw = load16(p.knw + c * 16);
    }
    // The bundle's requests are those of ranks m, 2M-1-m, 2M+m, 4M-1-m below B (rank 0 the
    // longest, ties by index).  Request slot k of the bundle: b (-1: none), length L (0: attends
    // nothing) and the row-0 element offsets of its K and V rows.
    Slots4<int> tb_b = {-1, -1, -1, -1}, tb_l = {0, 0, 0, 0};
    Slots4<int64_t> tb_k = {0, 0, 0, 0}, tb_v = {0, 0, 0, 0};
    int nseg = 0;
    auto set_slot = [&](int i, int b, int L) {
        const int64_t o = p.offs && b >= 0 ? p.offs[b] : 0;
        tb_b.set(i, b);
        tb_l.set(i, L);
        tb_k.set(i, (p.offs ? o : (int64_t)b * p.k_sb) + h * p.k_sh);
        tb_v.set(i, (p.offs ? o : (int64_t)b * p.v_sb) + h * p.v_sh);
        nseg = i + 1;
    };
    if (plan && (int)plan_batch == nb) {
        // the bundle's requests as the step's plan lists them (q3t_decode_plan), loaded above;
        // no ranking here.  Entries that do not name a request of this batch attend nothing and
        // write nothing.  A plan made for another batch is not used: the launch ranks by itself.
#pragma unroll
        for (int i = 0; i < kBundleMaxSeg; ++i) {
            const int b = (int)(uint32_t)e[i], L = (int)(uint32_t)(e[i] >> 32);
            const bool ok = b >= 0 && b < p.B;
            set_slot(i, ok ? b : -1, ok ? min(max(L, 0), p.ctx) : 0);
        }
        asm volatile("" :: "v"(qw.x), "v"(kw.x) : "memory");
    } else {
        // ranks: key = L * 1024 + (1023 - b) (longest first, ties by index; L = 0 without a
        // valid position).  Lane holds requests lane and lane + 64; each wave ranks in its own
        // LDS copy of the keys (no barrier), reading eight 16-byte groups of keys per wait.
        int key[2], len[2];
        int64_t pb[2] = {-1, -1};
#pragma unroll
        for (int e = 0; e < 2; ++e)
            if (lane + 64 * e < p.B) pb[e] = p.pos[lane + 64 * e];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int b = lane + 64 * e;
            const int L = (pb[e] >= 0 && pb[e] < p.ctx) ? (int)pb[e] + 1 : 0;
            len[e] = L;
            key[e] = b < p.B ? (L << 10) | (1023 - b) : -1;
            s.keys[wave][b] = key[e];
        }
        asm volatile("" :: "v"(qw.x), "v"(kw.x) : "memory");
        int rank[2] = {0, 0};
        for (int u0 = 0; u0 < p.B; u0 += 32) {  // keys past B are -1
            i32x4_t k4[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) k4[j] = *(const i32x4_t *)&s.keys[wave][u0 + 4 * j];
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    rank[e] += (k4[j].x > key[e]) + (k4[j].y > key[e]) + (k4[j].z > key[e]) + (k4[j].w > key[e]);
        }
#pragma unroll
        for (int i = 0; i < kBundleMaxSeg; ++i) {
            const int r = bundle_rank(i);
            if (r >= p.B) continue;
            const uint64_t m0 = __builtin_amdgcn_ballot_w64(rank[0] == r && lane < p.B);
            const uint64_t m1 = __builtin_amdgcn_ballot_w64(rank[1] == r && lane + 64 < p.B);
            const int b = m0 ? (int)__builtin_ctzll(m0) : 64 + (int)__builtin_ctzll(m1);
            set_slot(i, b, m0 ? __builtin_amdgcn_readlane(len[0], b) : __builtin_amdgcn_readlane(len[1], b - 64));
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // offsets loaded before any ring load

    auto seg_b = [&](int k) { return tb_b.get(k); };
    auto seg_l = [&](int k) { return tb_l.get(k); };
    auto seg_row0 = [&](const char *plane, const Slots4<int64_t> &offsets, int k) {
        return plane + offsets.get(k) * 2;
    };
    auto next_live = [&](int k) {
        while (k < nseg && seg_l(k) == 0) ++k;
        return k;
    };
    const int first_live = next_live(0);
    if (first_live >= nseg) {  // nothing to attend (uniform: no load has been issued): zero rows
        if (wave == 0) {
            for (int k = 0; k < nseg; ++k) {
                const int b = seg_b(k);
                if (b < 0) continue;
                for (int t = lane; t < G * 128; t += 64)
                    store_out<uint16_t>(p.out + (b * p.o_sb + (h * G + t / 128) * p.o_sh + t % 128) * 2, 0.f);
            }
        }
        return;
    }

    const int kst = (int)(p.k_st * 2), vst = (int)(p.v_st * 2);
    const uint32_t kbytes = (uint32_t)((p.ctx - 1) * kst + kRowBytes), vbytes = (uint32_t)((p.ctx - 1) * vst + kRowBytes);
    const uint32_t lds_ring = (uint32_t)(uintptr_t)&s.ring[0][0];
    auto head_of = [&](int k) { return (uint32_t)(uintptr_t)&s.head[k][0][0]; };

    // producer: the next stage to load (request slot ps, first key pj); rows at or past the
    // request's keys get offsets outside the resource (zeros, no memory access).  The request's
    // resources and key counts stay in scalar registers from one stage to the next.
    int ps = first_live, pj = 0, pL = 0, pjend = 0, pb = 0;
    i32x4_t krs, vrs;
    constexpr int KL = kStageLoads + (MASK ? 1 : 0);  // loads per wave and stage
    const int mes = MASK ? mask_elem_size(p.mask_dtype) : 0;
    i32x4_t mrs = {0, 0, 0, 0};
    if constexpr (MASK) {
        const uint32_t mbytes = (uint32_t)((((int64_t)(nb - 1) * p.m_sb + p.ctx) * mes + 3) & ~(int64_t)3);
        mrs = scalar_rsrc(p.mask, mbytes);
    }
    const uint32_t lds_mask = (uint32_t)(uintptr_t)&s.maskw[0][0][0];
    auto producer_request = [&]() {
        pL = seg_l(ps);
        pb = seg_b(ps);
        pjend = FUSED ? pL - 1 : pL;  // fused: row L-1 is the step's own key
        krs = scalar_rsrc(seg_row0(p.k, tb_k, ps), kbytes);
        vrs = scalar_rsrc(seg_row0(p.v, tb_v, ps), vbytes);
    };
    producer_request();
    // No wait for this wave's earlier reads of the slot: every one of them fed a product (or,
    // for the step's key, preceded such reads of the same wave), so all have returned.
    auto issue = [&](int slot) {
        const uint32_t base = lds_ring + slot * kStageBytes + wave * kWaveStage;
#pragma unroll
        for (int i = 0; i < kWaveKeys / 4; ++i) {
            const int r = 4 * i + g, j = pj + wave * kWaveKeys + r;
            const bool ok = j < pjend;
            const uint32_t ko = ok ? (uint32_t)(j * kst + ((c ^ r) & 15) * 16) : 0xfffffff0u;
            const uint32_t vo = ok ? (uint32_t)(j * vst + ((c ^ (2 * r)) & 15) * 16) : 0xfffffff0u;
            const uint32_t kl = (uint32_t)__builtin_amdgcn_readfirstlane((int)(base + i * 1024));
            const uint32_t vl = (uint32_t)__builtin_amdgcn_readfirstlane((int)(base + kWaveKeys * kRowBytes + i * 1024));
            if constexpr (STREAM) {
                load_to_lds16_stream(krs, ko, kl);
                load_to_lds16_stream(vrs, vo, vl);
            } else {
                load_to_lds16(krs, ko, kl);
                load_to_lds16(vrs, vo, vl);
            }
        }
        if constexpr (MASK) {
            // the mask word of each of the wave's 16 rows (lane r: row r); rows past the
            // request's keys read zeros
            const int q = pj + wave * kWaveKeys + (lane & 15);
            const int64_t elem = (int64_t)pb * p.m_sb + q;
            const uint32_t off = (lane < 16 && q < pL) ? (uint32_t)((elem * mes) & ~(int64_t)3) : 0xfffffff0u;
            load_to_lds4(mrs, off, (uint32_t)__builtin_amdgcn_readfirstlane((int)(lds_mask + (slot * kWaves + wave) * 256)));
        }
        pj += kStageKeys;
        if (pj >= pL) {
            pj = 0;
            ps = next_live(ps + 1);
            if (ps < nseg) producer_request();
        }
    };
    int total = 0;  // stages of the bundle
#pragma unroll
    for (int k = 0; k < kBundleMaxSeg; ++k)
        if (k < nseg) total += (tb_l.get(k) + kStageKeys - 1) / kStageKeys;
    int issued = 0;
    auto issue_next = [&]() {
        issue(issued % kRingStages);
        ++issued;
    };
    // The rows of every request of the bundle (query rows; fused: cos/sin and the step's key
    // and value) go out first, request k's from wave k % 4, then the ring's first two stages:
    // the rows land first, so each request's rotations happen once, in its own wave, while the
    // stages are in flight.  The slots are unrolled so that the bundle table is read without
    // branches.
#pragma unroll
    for (int k = 0; k < kBundleMaxSeg; ++k) {
        if (k >= nseg || tb_l.get(k) == 0 || wave != k % kWaves) continue;
        const int b = tb_b.get(k);
        const uint32_t hd = (uint32_t)__builtin_amdgcn_readfirstlane((int)head_of(k));
        const i32x4_t qrs = scalar_rsrc(p.q + (b * p.q_sb + (int64_t)h * G * p.q_sh) * 2,
                                        (uint32_t)((G - 1) * p.q_sh * 2 + kRowBytes));
        if (lane < 16 * G) load_to_lds16(qrs, (uint32_t)((lane >> 4) * p.q_sh * 2 + (lane & 15) * 16), hd);
        if constexpr (FUSED) {
            const i32x4_t crs = scalar_rsrc(p.cs + b * p.cs_sb * 2, kRowBytes);
            const i32x4_t srs = scalar_rsrc(p.sn + b * p.cs_sb * 2, kRowBytes);
            const i32x4_t nkr = scalar_rsrc(p.nk + (b * p.nk_sb + h * p.nk_sh) * 2, kRowBytes);
            const i32x4_t nvr = scalar_rsrc(p.nv + (b * p.nv_sb + h * p.nv_sh) * 2, kRowBytes);
            if (lane < 16) {
                load_to_lds16(crs, lane * 16, hd + 4 * kRowBytes);
                load_to_lds16(srs, lane * 16, hd + 5 * kRowBytes);
                load_to_lds16(nkr, lane * 16, hd + 6 * kRowBytes);
                load_to_lds16(nvr, lane * 16, hd + 7 * kRowBytes);
            }
        }
    }
    issue_next();
    if (issued < total) issue_next();

    {
        // the rows landed before the stages (which stay in flight)
        if (issued == 1) wait_loads<KL>();
        else wait_loads<2 * KL>();
        if constexpr (FUSED) {
            // each request's rows in the wave that loaded them, while the first stages are in
            // flight: lane group r < G holds query row r and lane group G the step's key (a
            // second pass for G = 4), lane c chunk c; normalised, rotated and written back
#pragma unroll
            for (int k = 0; k < kBundleMaxSeg; ++k) {
                if (k >= nseg || tb_l.get(k) == 0 || wave != k % kWaves) continue;
                const int Lk = tb_l.get(k);
                const uint32_t hk = head_of(k);
                const U4 cv = lds_read16(hk + 4 * kRowBytes + c * 16), sv = lds_read16(hk + 5 * kRowBytes + c * 16);
                auto rotate = [&](int row, bool is_key) {
                    U4 x = lds_read16(hk + row * kRowBytes + c * 16);
                    if constexpr (NORM) {
                        if (is_key ? p.knw != nullptr : p.qnw != nullptr) x = rms_norm8<16>(x, is_key ? kw : qw, p.eps, 128);
                    }
                    return rope_half8(x, xor8_u4(x), cv, sv, c < 8);
                };
                if constexpr (G < 4) {
                    if (g <= G) lds_write16(hk + (g < G ? g : 6) * kRowBytes + c * 16, rotate(g < G ? g : 6, g == G));
                } else {
                    lds_write16(hk + g * kRowBytes + c * 16, rotate(g, false));
                    if (g == 0) lds_write16(hk + 6 * kRowBytes + c * 16, rotate(6, true));
                }
            }
        }
        lds_barrier();  // every request's rows, rotated, visible to every wave
    }

    // per-lane LDS offsets within a wave's stage: K rows as the A operand of S^T (row c, dims
    // 32 kk + 8 g ...), V rows for the transposing read (row 4g + c/4, 4 dims)
    uint32_t ka[4], va[8];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) ka[kk] = c * kRowBytes + (((4 * kk + g) ^ c) & 15) * 16;
    {
        const int r = 4 * g + (c >> 2);
#pragma unroll
        for (int db = 0; db < 8; ++db)
            va[db] = kWaveKeys * kRowBytes + r * kRowBytes + (((2 * db + ((c >> 1) & 1)) ^ (2 * r)) & 15) * 16 + 8 * (c & 1);
    }
    const float scale = p.scale_log2;

    bf16x8_t qB[4];
    float mx = kEmpty, l = 0.f;
    f32x4_t acc[8];
    int cs = first_live, cj = 0, par = 0;
    uint32_t msub = 0;  // masked: the byte offsets of the current request's mask terms
    int L = seg_l(cs);  // the consumer's request: its keys and rows, kept between stages
    uint32_t hd = head_of(cs);
    for (int t = 0; t < total; ++t) {
        // the next stage, into the slot scored last (the first two went out before the loop)
        if (issued < total && issued <= t + 1) issue_next();
        const int ahead = issued - 1 - t;  // stages issued after this one: 0 or 1
        if (cj == 0) {
            if constexpr (MASK) {
                // byte offsets within their words of the lane's keys 4g + i of any stage (one byte each)
                const int64_t e0 = (int64_t)seg_b(cs) * p.m_sb;
                msub = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) msub |= (uint32_t)(((e0 + i) * mes) & 3) << (8 * i);
            }
            // a new request: its rows as B operands, columns c >= G zero
            const U4 zero = {0u, 0u, 0u, 0u};
            const int cq = c < G ? c : 0;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const U4 x = lds_read16(hd + cq * kRowBytes + (4 * kk + g) * 16);
                qB[kk] = as_bf16x8(c < G ? x : zero);
            }
            mx = kEmpty;
            l = 0.f;
#pragma unroll
            for (int db = 0; db < 8; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        }
        // this stage has landed (the next one stays in flight)
        if (ahead == 0) wait_loads<0>();
        else wait_loads<KL>();
        if constexpr (FUSED) {
            if (t == 0) {
                // the step's keys and values into the arena, by each request's wave, only now: a
                // store shares the load counter, so one issued before this wait would have held it
                // up until part of the next stage had landed as well
#pragma unroll
                for (int k = 0; k < kBundleMaxSeg; ++k) {
                    if (k >= nseg || tb_l.get(k) == 0 || wave != k % kWaves) continue;
                    if (g == 0) {
                        const int Lk = tb_l.get(k);
                        const uint32_t hk = head_of(k);
                        const auto krs = buffer_rsrc(uniform_ptr(seg_row0(p.k, tb_k, k)), kbytes);
                        const auto vrs = buffer_rsrc(uniform_ptr(seg_row0(p.v, tb_v, k)), vbytes);
                        buffer_store16(krs, (uint32_t)((Lk - 1) * kst + c * 16), lds_read16(hk + 6 * kRowBytes + c * 16));
                        buffer_store16(vrs, (uint32_t)((Lk - 1) * vst + c * 16), lds_read16(hk + 7 * kRowBytes + c * 16));
                    }
                }
            }
        }
        const uint32_t sb = lds_ring + (t % kRingStages) * kStageBytes + wave * kWaveStage;
        if constexpr (FUSED) {
            // the step's key and value enter the ring at row L-1 of the request's last stage
            // (the loads left that row zero)
            const int r = L - 1 - cj - wave * kWaveKeys;
            if (r >= 0 && r < kWaveKeys && g == 0) {
                lds_write16(sb + r * kRowBytes + ((c ^ r) & 15) * 16, lds_read16(hd + 6 * kRowBytes + c * 16));
                lds_write16(sb + kWaveKeys * kRowBytes + r * kRowBytes + ((c ^ (2 * r)) & 15) * 16,
                            lds_read16(hd + 7 * kRowBytes + c * 16));
            }
        }

        // scores of the wave's 16 keys (rows of S^T) for the 16 columns
        f32x4_t st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(lds_read16(sb + ka[kk])), qB[kk], st, 0, 0, 0);
        const int j0 = cj + wave * kWaveKeys + 4 * g;
        float x[4];
        if constexpr (MASK) {
            const U4 w4 = lds_read16(lds_mask + ((t % kRingStages) * kWaves + wave) * 256 + 16 * g);
            const uint32_t wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float term;
                if constexpr (MK == 1) {
                    // bf16: the element is the word's high half at byte offset 2, else its low half
                    term = __uint_as_float((msub >> (8 * i)) & 2u ? (wv[i] & 0xffff0000u) : (wv[i] << 16)) * kLog2e;
                } else {
                    term = mask_term(wv[i], (msub >> (8 * i)) & 3u, p.mask_dtype);
                }
                x[i] = j0 + i < L ? st[i] * scale + term : -INFINITY;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = j0 + i < L ? st[i] * scale : -INFINITY;
        }
        // a column's maximum over the stage is the largest of its four lanes' maxima, so a
        // column passes the threshold exactly when one of its lanes does: the exchanges
        // across the lanes run only when some lane passes (the first stage of a request and
        // the rare rescale), off the chain of the other stages; the outputs are unchanged
        float mb = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        if (__builtin_amdgcn_ballot_w64(mb > mx + kRescaleLog2)) {
            mb = fmaxf(mb, xor16(mb));
            mb = fmaxf(mb, xor32(mb));
            const bool up = mb > mx + kRescaleLog2;
            const float mn = up ? mb : mx;
            const float alpha = fexp2(mx - mn);
            l *= alpha;
#pragma unroll
            for (int db = 0; db < 8; ++db) acc[db] *= alpha;
            mx = mn;
        }
        float pw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pw[i] = fexp2(x[i] - mx);
        l += (pw[0] + pw[1]) + (pw[2] + pw[3]);
        const uint2 pp = {cvt_pk_bf16(pw[0], pw[1]), cvt_pk_bf16(pw[2], pw[3])};
        const s16x4_t pb = __builtin_bit_cast(s16x4_t, pp);
#pragma unroll
        for (int db = 0; db < 8; ++db)
            acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, lds_read_tr16(sb + va[db])),
                                                               pb, acc[db], 0, 0, 0);

        cj += kStageKeys;
        if (cj >= L) {
            // the request's state: the wave's sums over its lane groups, then the merge of the
            // four waves in LDS and one output element per thread (kept in LDS)
            float lt = l + xor16(l);
            lt += xor32(lt);
            if (c < G) {
                if (g == 0) {
                    s.ml[par][wave][c][0] = mx;
                    s.ml[par][wave][c][1] = lt;
                }
#pragma unroll
                for (int db = 0; db < 8; ++db)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s.acc[par][wave][c][16 * db + 4 * g + i] = acc[db][i];
            }
            lds_barrier();
            for (int t2 = tid; t2 < G * 128; t2 += kThreads) {
                const int cc = t2 / 128, d = t2 % 128;
                float mm = s.ml[par][0][cc][0];
#pragma unroll
                for (int w = 1; w < kWaves; ++w) mm = fmaxf(mm, s.ml[par][w][cc][0]);
                float sl = 0.f, sa = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float wt = fexp2(s.ml[par][w][cc][0] - mm);
                    sl += s.ml[par][w][cc][1] * wt;
                    sa += s.acc[par][w][cc][d] * wt;
                }
                s.outq[cs][cc][d] = (uint16_t)float_to_bf16(sa * __builtin_amdgcn_rcpf(sl));
            }
            par ^= 1;
            cs = next_live(cs + 1);
            cj = 0;
            if (cs < nseg) {
                L = seg_l(cs);
                hd = head_of(cs);
            }
        }
    }
    // Output rows (zeros for requests without a valid position) once every request is merged.
    // No load is outstanding here (every stage was awaited), so the workgroup ends without
    // waiting for its stores.
    // 16-byte stores (one lane per 8 elements) when the output rows allow them, else 2-byte ones.
    lds_barrier();
    const bool vec_out = ((reinterpret_cast<uintptr_t>(p.out) | (uintptr_t)(p.o_sb * 2) | (uintptr_t)(p.o_sh * 2)) & 15) == 0;
#pragma unroll
    for (int k = 0; k < kBundleMaxSeg; ++k) {
        if (k >= nseg) continue;
        const int b = tb_b.get(k);
        const int L = tb_l.get(k);
        if (b < 0) continue;
        if (vec_out) {
            if (tid < G * 16) {
                const int cc = tid / 16, ch = tid % 16;
                const U4 v = L > 0 ? *reinterpret_cast<const U4 *>(&s.outq[k][cc][ch * 8]) : U4{0u, 0u, 0u, 0u};
                store16(p.out + (b * p.o_sb + (h * G + cc) * p.o_sh + ch * 8) * 2, v);
            }
        } else {
            for (int t = tid; t < G * 128; t += kThreads) {
                const int cc = t / 128, d = t % 128;
                *reinterpret_cast<uint16_t *>(p.out + (b * p.o_sb + (h * G + cc) * p.o_sh + d) * 2) =
                    L > 0 ? s.outq[k][cc][d] : (uint16_t)0;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------

// The counter region has one fixed size, so that the counters of every launch sit on bytes
// that only ever hold counters (all zero between launches), whatever batch and head count
// earlier launches on the same workspace used.
constexpr int64_t kMaxCounters = 65536;  // batch * kv_heads
static int64_t counters_bytes() { return kMaxCounters * 4; }

// Chunked grid: chunks per (request, KV head): ceil(ctx / 64) at most; by default as many as
// give about kTargetGroups workgroups for the whole batch, two per CU of the MI355X.
constexpr int64_t kTargetGroups = 512;

// Balanced grid: workgroups per KV head by default (kBalancedGroups over all heads), and the
// context length from which it is the automatic choice.  Measured (bf16, 16/8 heads, contexts
// drawn uniformly): 128 requests over 4096 rows 170 us balanced against 193 us chunked, over
// 2048 rows 98 against 108; 8 requests over 8192 rows 31 against 35; but 64 requests over
// 1024 rows (the talker step) 32-34 against 30 us: on short contexts the balanced grid's
// per-segment costs outweigh the imbalance it removes.
constexpr int64_t kBalancedGroups = 256;
constexpr int64_t kBalancedMinCtx = 2048;
constexpr int64_t kMaxSplits = 32768;  // a pair's arrivals fit the counter's low 16 bits

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

// The grid a call runs on (Q3T_GRID_CHUNKED, _BALANCED or _BUNDLED; -1: a requested grid the
// call does not qualify for).  The bundled grid needs bf16 rows of 128, one query token, at
// most kBundleMaxBatch requests, q_heads / kv_heads <= 4, and a mask with unit key stride.
// Automatic choice, measured (bf16, 16/8 heads, 28-layer graphs of fused steps, us per layer).
// The bundled grid pairs long requests with short ones, so it wins on ragged contexts; with
// equal contexts two whole requests per workgroup lose to the chunked grid's one per
// workgroup, two workgroups per CU (64 requests of 512 keys in a 1024-row arena: 27.2 against
// 26.5; of 64 keys in a 512-row arena: 10.9 against 8.1).  The host sees the capacity, not
// the lengths, so:
//  - 24..63 requests (192..511 (request, KV head) items) from 512 rows: bundled, which beat
//    the chunked grid on every distribution measured (32 requests of 64 keys: 7.9 against
//    11.0; 32 over 512 rows, uniform lengths: 13.5 against 16.7; 24 over 1024 rows: 19.4
//    against 21.7 balanced);
//  - 64..128 requests from 1024 rows (the talker step's ragged contexts: 26.1 against 30.3
//    chunked; 96 requests over 2048 rows: 71.7 against 78.2 balanced);
//  - from 4096 rows only with 384 items or more, where one or two whole requests per
//    workgroup leave the longest unbalanced (32 requests: 60.9 against 52.9 balanced);
//  - chunked below 512 rows (64 requests over 256 rows: 12.6 against 12.9 bundled) and for 64
//    or more requests over 512..1023 rows (the reference's valid-length probes, equal
//    contexts); balanced otherwise from 2048 rows.
constexpr int64_t kBundleMinCtx = 512;
constexpr int64_t kBundleMinItems = 192;
constexpr int64_t kBundleManyItems = 512;      // 64 requests of 8 KV heads
constexpr int64_t kBundleManyMinCtx = 1024;
constexpr int64_t kBundleLongCtx = 4096;
constexpr int64_t kBundleMinItemsLong = 384;
// A mask on the bundled grid: unit key stride, 4-byte aligned, its words addressed by 32-bit
// byte offsets.
static bool bundle_mask_ok(const q3t_decode_args *a) {
    if (!a->mask) return true;
    const int64_t es = a->mask_dtype == Q3T_F32 ? 4 : a->mask_dtype == Q3T_BOOL ? 1 : 2;
    if (a->mask_stride_t != 1 || a->mask_stride_b < 0 || !aligned(a->mask, 4)) return false;
    return ((a->batch - 1) * a->mask_stride_b + a->ctx) * es + 3 <= (int64_t)INT32_MAX;
}
static bool bundle_ok(const q3t_decode_args *a) {
    return a->dtype == Q3T_BF16 && a->head_dim == 128 && a->query_len == 1 && bundle_mask_ok(a) &&
           a->batch <= kBundleMaxBatch && a->q_heads / a->kv_heads <= 4;
}
static int decode_grid(const q3t_decode_args *a) {
    switch (a->grid) {
        case Q3T_GRID_CHUNKED: return Q3T_GRID_CHUNKED;
        case Q3T_GRID_BALANCED: return Q3T_GRID_BALANCED;
        case Q3T_GRID_BUNDLED: return bundle_ok(a) ? Q3T_GRID_BUNDLED : -1;
        default: break;
    }
    if (a->splits < 0) return Q3T_GRID_CHUNKED;
    if (a->splits > 0) return Q3T_GRID_BALANCED;
    const int64_t items = a->batch * a->kv_heads;
    const bool bundled = a->ctx >= kBundleLongCtx ? items >= kBundleMinItemsLong
                         : items >= kBundleManyItems ? a->ctx >= kBundleManyMinCtx
                                                     : items >= kBundleMinItems && a->ctx >= kBundleMinCtx;
    if (bundled && bundle_ok(a)) return Q3T_GRID_BUNDLED;
    return a->ctx >= kBalancedMinCtx ? Q3T_GRID_BALANCED : Q3T_GRID_CHUNKED;
}

// Balanced grid: workgroups per KV head.
static int64_t balanced_splits(const q3t_decode_args *a) {
    if (a->splits > 0) return a->splits;
    return (kBalancedGroups + a->kv_heads - 1) / a->kv_heads;
}

// Bundled grid: bundles (workgroups) per KV head, one workgroup per CU in all, and at most
// kBundleMaxSeg requests per bundle.
static int64_t bundle_count(const q3t_decode_args *a) {
    const int64_t m = (kBundleGroups + a->kv_heads - 1) / a->kv_heads;
    const int64_t least = (a->batch + kBundleMaxSeg - 1) / kBundleMaxSeg;
    return m < least ? least : m;
}

static int64_t partial_floats(const q3t_decode_args *a) {
    const int64_t R = (a->q_heads / a->kv_heads) * a->query_len;
    int64_t units = 0;
    switch (decode_grid(a)) {
        case Q3T_GRID_BALANCED: units = a->kv_heads * balanced_splits(a) * 2; break;
        case Q3T_GRID_CHUNKED:
            units = a->batch * a->kv_heads * chunk_count(a->batch, a->kv_heads, a->ctx, a->max_chunks);
            break;
        default: break;  // bundled: whole requests, no partial states
    }
    return units * R * (a->head_dim + 2);
}

}  // namespace q3t

using namespace q3t;

static bool decode_sizes_ok(const q3t_decode_args *a) {
    return a->batch >= 0 && a->batch <= kMaxBatch && a->query_len >= 1 && a->q_heads >= 1 &&
           a->kv_heads >= 1 && a->q_heads % a->kv_heads == 0 && a->head_dim >= 1 && a->ctx >= 1 &&
           a->ctx <= (1 << 20) && a->max_chunks <= kMaxChunks && a->splits <= kMaxSplits &&
           a->grid >= Q3T_GRID_AUTO && a->grid <= Q3T_GRID_BUNDLED;
}

extern "C" int q3t_decode_grid(const q3t_decode_args *a) {
    if (!a || !decode_sizes_ok(a)) return Q3T_EINVAL;
    const int grid = decode_grid(a);
    return grid < 0 ? Q3T_EUNSUPPORTED : grid;
}

extern "C" int64_t q3t_decode_workspace_bytes(const q3t_decode_args *a) {
    if (!a || !decode_sizes_ok(a)) return -1;
    // the bundled grid attends whole requests: no counters, no partial states
    if (decode_grid(a) == Q3T_GRID_BUNDLED) return 0;
    return counters_bytes() + partial_floats(a) * 4;
}

// The chunked and balanced grids (FUSE as in PairWork).
template <typename T, int D, int G, int SQ, int FUSE, bool M>
static void launch_split(const DecodeParams &p, hipStream_t s) {
    // streamed instances only for the talker-shaped single-query launches
    constexpr bool can_stream = sizeof(T) == 2 && D == 128 && SQ == 1;
    if (p.splits > 0) {
        const dim3 grid((uint32_t)p.splits * p.Hkv);
        if (can_stream && p.stream)
            hipLaunchKernelGGL((decode_balanced_kernel<T, D, G, SQ, FUSE, M, can_stream>), grid, dim3(kThreads), 0, s, p);
        else
            hipLaunchKernelGGL((decode_balanced_kernel<T, D, G, SQ, FUSE, M, false>), grid, dim3(kThreads), 0, s, p);
        return;
    }
    const dim3 grid((uint32_t)p.B * p.Hkv * p.nchunks);
    if (can_stream && p.stream)
        hipLaunchKernelGGL((decode_chunks_kernel<T, D, G, SQ, FUSE, M, can_stream>), grid, dim3(kThreads), 0, s, p);
    else
        hipLaunchKernelGGL((decode_chunks_kernel<T, D, G, SQ, FUSE, M, false>), grid, dim3(kThreads), 0, s, p);
}

template <int G, bool F, int M>
static void launch_bundled(const DecodeParams &p, hipStream_t s) {
    // whole requests per workgroup, bundled by the step's plan when the call brings one
    const int32_t *rank = p.plan;
    const dim3 grid((uint32_t)p.bundles * p.Hkv);
    if (F && (p.qnw || p.knw)) {
        if constexpr (F) {
            if (p.stream) hipLaunchKernelGGL((decode_bundled_kernel<G, F, true, true, M>), grid, dim3(kThreads), 0, s, rank, p.B, p.Hkv, p.bundles, p);
            else hipLaunchKernelGGL((decode_bundled_kernel<G, F, false, true, M>), grid, dim3(kThreads), 0, s, rank, p.B, p.Hkv, p.bundles, p);
        }
    } else if (p.stream) {
        hipLaunchKernelGGL((decode_bundled_kernel<G, F, true, false, M>), grid, dim3(kThreads), 0, s, rank, p.B, p.Hkv, p.bundles, p);
    } else {
        hipLaunchKernelGGL((decode_bundled_kernel<G, F, false, false, M>), grid, dim3(kThreads), 0, s, rank, p.B, p.Hkv, p.bundles, p);
    }
}

template <typename T, int D, int G, int SQ, bool F, bool M>
static void launch_decode(const DecodeParams &p, hipStream_t s) {
    if constexpr (sizeof(T) == 2 && D == 128 && SQ == 1 && G <= 4) {
        if (p.bundles > 0) {
            if constexpr (M) {
                if (p.mask_dtype == Q3T_BF16) launch_bundled<G, F, 1>(p, s);
                else launch_bundled<G, F, 2>(p, s);
            } else {
                launch_bundled<G, F, 0>(p, s);
            }
            return;
        }
    }
    if constexpr (F) {
        if (p.qnw || p.knw) {
            launch_split<T, D, G, SQ, 2, M>(p, s);
            return;
        }
    }
    launch_split<T, D, G, SQ, F ? 1 : 0, M>(p, s);
}

template <typename T, int D, int G>
static int dispatch_sq(const DecodeParams &p, int sq, bool fused, hipStream_t s) {
    if (fused) {
        if constexpr (sizeof(T) == 2 && D == 128) {
            if (sq == 1) {
                if (p.has_mask) launch_decode<T, D, G, 1, true, true>(p, s);
                else launch_decode<T, D, G, 1, true, false>(p, s);
            } else if (sq == 2) {
                if (p.has_mask) launch_decode<T, D, G, 2, true, true>(p, s);
                else launch_decode<T, D, G, 2, true, false>(p, s);
            } else {
                return Q3T_EUNSUPPORTED;
            }
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

// Host-side validation and parameter set-up shared by every decode entry point; the device
// workspace (counter region, then the partial states) starts at `ws`.
static int decode_params(const q3t_decode_args *a, char *ws, DecodeParams &p) {
    if (!decode_sizes_ok(a)) return Q3T_EINVAL;
    if (a->kv_heads * a->batch > kMaxCounters) return Q3T_EUNSUPPORTED;
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
    const int grid = decode_grid(a);
    if (grid < 0) return Q3T_EUNSUPPORTED;
    const int64_t splits = grid == Q3T_GRID_BALANCED ? balanced_splits(a) : 0;
    const int64_t nchunks = chunk_count(a->batch, a->kv_heads, a->ctx, a->max_chunks);
    if (splits > 0 ? splits * a->kv_heads > INT32_MAX : a->batch * a->kv_heads * nchunks > INT32_MAX)
        return Q3T_EUNSUPPORTED;
    p.B = (int)a->batch;
    p.Hq = (int)a->q_heads;
    p.Hkv = (int)a->kv_heads;
    p.ctx = (int)a->ctx;
    p.nchunks = (int)nchunks;
    p.splits = (int)splits;
    p.bundles = grid == Q3T_GRID_BUNDLED ? (int)bundle_count(a) : 0;
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
    p.plan = grid == Q3T_GRID_BUNDLED ? a->plan : nullptr;  // read by the bundled grid's two kernels
    if (a->q_norm_weight || a->k_norm_weight) {
        if (!fused || !(a->norm_eps >= 0.f)) return Q3T_EINVAL;
        if ((a->q_norm_weight && !aligned(a->q_norm_weight, 16)) ||
            (a->k_norm_weight && !aligned(a->k_norm_weight, 16)))
            return Q3T_EINVAL;
        p.qnw = (const char *)a->q_norm_weight;
        p.knw = (const char *)a->k_norm_weight;
    }
    return Q3T_OK;
}

static int decode_launch(const q3t_decode_args *a, const DecodeParams &p, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    const int g = (int)(a->q_heads / a->kv_heads);
    const int sq = (int)a->query_len;
    const bool fused = a->fused != 0;
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

// Zero the counter region with vector stores (a kernel, not a memset node, so a caller may
// capture it in a graph).
__global__ void __launch_bounds__(256) reset_counters_kernel(int4 *counters, int64_t n16) {
    for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
        counters[i] = int4{0, 0, 0, 0};
}

extern "C" int q3t_decode_reset_workspace(void *workspace, int64_t workspace_bytes, void *stream) {
    if (!workspace || !aligned(workspace, 16) || workspace_bytes < counters_bytes()) return Q3T_EWORKSPACE;
    const int64_t n16 = counters_bytes() / 16;
    hipLaunchKernelGGL(reset_counters_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (int4 *)workspace, n16);
    return launch_status();
}

// ---- the allocation-free variant --------------------------------------------------------
// For callers that cannot allocate device memory (code under graph capture that may not call
// hipMalloc, serving loops, harnesses that forbid it): the workspace is a file-scope device
// array of a fixed size, one copy per GPU, held until the process ends.  Its device address
// is looked up once per device (with that device current) and kept; the array's name itself
// is only a host-side stand-in and is never passed to a kernel.  Every call on one GPU uses
// the same array: calls that overlap in time on one GPU (two streams) race.
constexpr int64_t kScratchBytes = 8 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex scratch_mutex;
static char *scratch_ptr[kMaxDevices];

// Device address of this device's scratch array (nullptr on failure).  The first call on a
// device also clears its counter region, on `stream`, before any decode launch that uses it.
static char *device_scratch(hipStream_t stream) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        const int64_t n16 = counters_bytes() / 16;
        hipLaunchKernelGGL(reset_counters_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, stream,
                           (int4 *)ptr, n16);
        if (hipGetLastError() != hipSuccess) return nullptr;
        scratch_ptr[dev] = (char *)ptr;
    }
    return scratch_ptr[dev];
}

extern "C" int q3t_decode_attention_static(const q3t_decode_args *a, void *stream) {
    if (!a) return Q3T_EINVAL;
    if (!decode_sizes_ok(a)) return Q3T_EINVAL;
    if (a->batch == 0) return Q3T_OK;
    if (q3t_decode_workspace_bytes(a) > kScratchBytes) return Q3T_EWORKSPACE;
    char *ws = device_scratch((hipStream_t)stream);
    if (!ws) return (int)hipErrorInvalidDevicePointer;
    DecodeParams p;
    const int st = decode_params(a, ws, p);
    if (st != Q3T_OK) return st;
    return decode_launch(a, p, stream);
}

extern "C" int q3t_decode_attention(const q3t_decode_args *a, void *stream) {
    if (!a) return Q3T_EINVAL;
    if (!decode_sizes_ok(a)) return Q3T_EINVAL;
    if (a->batch == 0) return Q3T_OK;
    DecodeParams p;
    const int st = decode_params(a, (char *)a->workspace, p);
    if (st != Q3T_OK) return st;
    const int64_t need = q3t_decode_workspace_bytes(a);
    if (need > 0 && (!a->workspace || a->workspace_bytes < need || !aligned(a->workspace, 16)))
        return Q3T_EWORKSPACE;
    return decode_launch(a, p, stream);
}

static bool plan_shape_ok(int64_t batch, int64_t ctx, int64_t q_heads, int64_t kv_heads) {
    return batch >= 0 && batch <= kBundleMaxBatch && ctx >= 1 && ctx <= (1 << 20) && kv_heads >= 1 &&
           q_heads >= kv_heads && q_heads % kv_heads == 0 && q_heads / kv_heads <= 4;
}

extern "C" int64_t q3t_decode_plan_bytes(int64_t batch, int64_t q_heads, int64_t kv_heads) {
    if (!plan_shape_ok(batch, 1, q_heads, kv_heads)) return -1;
    return plan_ints(batch, kv_heads) * 4;
}

extern "C" int q3t_decode_plan(const int64_t *positions, int64_t batch, int64_t ctx, int64_t q_heads,
                               int64_t kv_heads, int32_t *plan, void *stream) {
    if (!plan_shape_ok(batch, ctx, q_heads, kv_heads)) return Q3T_EINVAL;
    if (batch == 0) return Q3T_OK;
    if (!positions || !plan || !aligned(positions, 8) || !aligned(plan, 16)) return Q3T_EINVAL;
    return plan_launch(positions, (int)batch, (int)ctx, (int)plan_bundle_count(batch, kv_heads), plan,
                       (hipStream_t)stream);
}
