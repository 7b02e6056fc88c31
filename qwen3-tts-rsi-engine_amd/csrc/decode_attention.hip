// Ragged grouped-query decode attention over the slot arena: a per-step work plan and the
// attention kernel that follows it.
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
// Plan (one small launch per decode step; every layer of the step reuses it, as
// SlotCache.prepare runs once per step, continuous.py:189):
//   * a request longer than the mean bin load is cut into near-equal pieces; the pieces are
//     ranked by length and dealt to `bins` bins in snake order (0..n-1, n-1..0, ...), which
//     pairs long pieces with short ones, so bins carry near-equal key counts and, with
//     uniform-ish lengths, no request is split at all.
// Attention (one launch per layer):
//   * grid = kv_heads x bins workgroups of 8 waves; workgroup x serves KV head x % kv_heads,
//     so with 8 KV heads every head maps onto one XCD under the round-robin dispatch (its
//     partial states stay in that XCD's L2), and one workgroup occupies one CU.
//   * the workgroup's pieces are concatenated and each wave streams its own contiguous
//     eighth of that key range, crossing piece boundaries without barriers; within a wave
//     8 lanes share one key (16 bytes of each 128-byte half row per lane) and each 8-lane
//     group keeps its own online-softmax state.
//   * per piece, the group states merge with lane swaps (VALU) and the wave states through
//     LDS (the "LDS-staged online-softmax merge") after one barrier.  A split request
//     publishes device-scope partials; the last workgroup to arrive (atomic counter) merges
//     them in piece order, writes the output and re-zeroes the counter, so results are
//     deterministic and every launch can be replayed from a graph.
#include "q3t_common.hpp"

namespace q3t {

constexpr int kMaxBatch = 1024;
constexpr int kMaxBins = 1024;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kEmpty = -1.0e30f;  // finite "no key yet" running max

// Plan layout (int32): header [nbins, npieces, batch, slot_pieces, ctx, 0 x 3], piece counts per bin
// (padded to a multiple of 8), then per bin a fixed slot of slot_pieces 8-int records
// [b, j0, j1, L_b, slot, nsplit, first_slot, 0], so a workgroup reads its count and its
// records in one round trip.  A bin never holds more than batch / bins + 2 pieces.
constexpr int kPlanHeader = 8;
constexpr int kPieceInts = 8;
inline int64_t plan_slot_pieces(int64_t batch, int64_t bins) { return batch / bins + 2; }
inline int64_t plan_counts_ints(int64_t bins) { return (bins + 7) / 8 * 8; }
inline int64_t plan_ints(int64_t batch, int64_t bins) {
    return kPlanHeader + plan_counts_ints(bins) + bins * plan_slot_pieces(batch, bins) * kPieceInts;
}

struct DecodeParams {
    int B, Hq, Hkv, ctx, nbins, max_slots;
    float scale_log2;
    int has_mask, mask_dtype;
    const int *plan;
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

// Sum over each aligned group of LPK (8 or 16) lanes; every lane of the group gets the total.
template <int LPK>
Q3T_DEVICE float group_sum(float x) {
    x = sum8(x);
    if constexpr (LPK == 16) x += xor8(x);
    return x;
}

// One online-softmax step of a lane group over UU keys held in registers.
// key_idx[u] is the key's index within its request (for query-row causal limits and the
// mask); valid[u] excludes keys outside the piece.
template <typename T, int R, int G, int SQ, int NCH, int EPL, int UU, int LPK, bool MASK>
Q3T_DEVICE void softmax_step(const DecodeParams &p, const U4 (&qr)[R][NCH], const U4 (&kr)[UU][NCH],
                             const U4 (&vr)[UU][NCH], const bool (&valid)[UU],
                             const int (&key_idx)[UU], int last_pos, const char *mask_row,
                             float (&m)[R], float (&l)[R], float (&acc)[R][EPL]) {
    float s[UU][R];
#pragma unroll
    for (int u = 0; u < UU; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r) s[u][r] = group_sum<LPK>(lane_dot<T, NCH>(qr[r], kr[u]));
#pragma unroll
    for (int u = 0; u < UU; ++u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int qi = r / G;
            bool ok = valid[u];
            // with no explicit mask, several queries of a request are causal among the last keys
            if constexpr (SQ > 1 && !MASK) ok = ok && key_idx[u] <= last_pos - (SQ - 1) + qi;
            float x = s[u][r] * p.scale_log2;
            if (MASK && ok) {
                const char *mp = mask_row + (qi * p.m_ss + (int64_t)key_idx[u] * p.m_st) *
                                                (p.mask_dtype == Q3T_F32 ? 4 : p.mask_dtype == Q3T_BOOL ? 1 : 2);
                x += load_mask(mp, p.mask_dtype) * kLog2e;
            }
            s[u][r] = ok ? x : -INFINITY;
        }
    }
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
        for (int e = 0; e < EPL; ++e) acc[r][e] *= alpha;
#pragma unroll
        for (int u = 0; u < UU; ++u) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const uint32_t w[4] = {vr[u][c].x, vr[u][c].y, vr[u][c].z, vr[u][c].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (sizeof(T) == 2) {
                        acc[r][c * 8 + 2 * i] += pu[u] * bf16_lo(w[i]);
                        acc[r][c * 8 + 2 * i + 1] += pu[u] * bf16_hi(w[i]);
                    } else {
                        acc[r][c * 4 + i] += pu[u] * __uint_as_float(w[i]);
                    }
                }
            }
        }
    }
}


// Cross-workgroup partial states are written and read with device-scope (sc1) accesses,
// which are coherent across the XCDs' L2 caches without an L2 write-back.  A writer waits
// for its device-scope stores to complete (vmcnt 0) before the workgroup barrier that
// precedes the counter increment; the last workgroup reads the partials only after its
// increment returned, again with device-scope loads.
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

// ---- the plan --------------------------------------------------------------------------

constexpr int kPlanThreads = 256;
constexpr int kMaxPieces = kMaxBatch + kMaxBins;

// Exclusive block scan of one int per thread slot group (kPlanThreads threads, `per` values
// each, values in v[]); returns the block total.
template <int PER>
Q3T_DEVICE int block_exclusive_scan(int (&v)[PER], int *sm_wave) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tsum = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) tsum += v[i];
    int incl = tsum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
    }
    if (lane == 63) sm_wave[wave] = incl;
    __syncthreads();
    int excl = incl - tsum, total = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
        if (w < wave) excl += sm_wave[w];
        total += sm_wave[w];
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int x = v[i];
        v[i] = excl;
        excl += x;
    }
    __syncthreads();
    return total;
}

__global__ void __launch_bounds__(kPlanThreads)
decode_plan_kernel(const int64_t *__restrict__ pos, int B, int ctx, int nbins, int *__restrict__ plan) {
    constexpr int PER = kMaxBatch / kPlanThreads;
    __shared__ int sm_wave[kPlanThreads / 64];
    __shared__ int sm_piece[kMaxPieces][4];  // b, j0, j1, rank-key length
    __shared__ int sm_split[kMaxPieces][3];  // slot, nsplit, first_slot
    __shared__ int sm_order[kMaxPieces];
    const int tid = threadIdx.x;

    int L[PER], n[PER], slots[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int b = tid * PER + i;
        L[i] = 0;
        if (b < B) {
            const int64_t pp = pos[b];
            L[i] = (pp >= 0 && pp < ctx) ? (int)pp + 1 : 0;
        }
        n[i] = L[i];
    }
    const int total = block_exclusive_scan<PER>(n, sm_wave);  // n[] now holds key offsets (unused)
    const int target = total > 0 ? (total + nbins - 1) / nbins : 1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        n[i] = L[i] > 0 ? (L[i] + target - 1) / target : 0;
        slots[i] = n[i] > 1 ? n[i] : 0;
    }
    int base[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) base[i] = n[i];
    const int npieces = block_exclusive_scan<PER>(base, sm_wave);
    const int nslots = block_exclusive_scan<PER>(slots, sm_wave);
    (void)nslots;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int b = tid * PER + i;
        for (int k = 0; k < n[i]; ++k) {
            const int idx = base[i] + k;
            const int j0 = (int)((int64_t)L[i] * k / n[i]), j1 = (int)((int64_t)L[i] * (k + 1) / n[i]);
            sm_piece[idx][0] = b;
            sm_piece[idx][1] = j0;
            sm_piece[idx][2] = j1;
            sm_piece[idx][3] = L[i];
            sm_split[idx][0] = n[i] > 1 ? slots[i] + k : -1;
            sm_split[idx][1] = n[i];
            sm_split[idx][2] = slots[i];
        }
    }
    __syncthreads();
    // rank by length, longest first; ties keep request order
    for (int i = tid; i < npieces; i += kPlanThreads) {
        const int li = sm_piece[i][2] - sm_piece[i][1];
        int rank = 0;
        for (int j = 0; j < npieces; ++j) {
            const int lj = sm_piece[j][2] - sm_piece[j][1];
            rank += (lj > li) || (lj == li && j < i);
        }
        sm_order[rank] = i;
    }
    __syncthreads();
    // snake deal: rank r goes to round t = r / nbins, bin t even ? r % nbins : nbins-1 - r % nbins
    const int full = npieces / nbins, rem = npieces % nbins;
    const int slot_pieces = B / nbins + 2;
    if (tid < kPlanHeader)
        plan[tid] = tid == 0 ? nbins : tid == 1 ? npieces : tid == 2 ? B : tid == 3 ? slot_pieces : tid == 4 ? ctx : 0;
    auto bin_count = [&](int k) {
        const bool extra = rem > 0 && ((full & 1) == 0 ? k < rem : k >= nbins - rem);
        return full + (extra ? 1 : 0);
    };
    for (int k = tid; k < nbins; k += kPlanThreads) plan[kPlanHeader + k] = bin_count(k);
    int *bins = plan + kPlanHeader + (nbins + 7) / 8 * 8;
    for (int r = tid; r < npieces; r += kPlanThreads) {
        const int t = r / nbins, j = r % nbins;
        const int k = (t & 1) == 0 ? j : nbins - 1 - j;
        const int i = sm_order[r];
        int *rec = bins + ((int64_t)k * slot_pieces + t) * kPieceInts;
        rec[0] = sm_piece[i][0];
        rec[1] = sm_piece[i][1];
        rec[2] = sm_piece[i][2];
        rec[3] = sm_piece[i][3];
        rec[4] = sm_split[i][0];
        rec[5] = sm_split[i][1];
        rec[6] = sm_split[i][2];
        rec[7] = 0;
    }
}

// ---- the attention kernel ----------------------------------------------------------------

// Launch shape of a kernel variant: lanes per key (a 16-byte chunk per lane), waves per
// workgroup and keys per lane group per block, chosen so that the variant stays within
// 128 (16 waves) or 256 (8 waves) VGPRs.
constexpr int decode_waves(int rows) { return rows <= 2 ? 16 : 8; }

template <typename T, int D, int R>
struct DecodeShape {
    static constexpr int ES = sizeof(T);
    static constexpr int ROW = D * ES;                        // bytes per key row
    static constexpr int LPK = ROW >= 256 ? 16 : 8;
    static constexpr int WAVES = decode_waves(R);
    static constexpr int U = R <= 2 ? (ROW > 256 ? 4 : 8) : (R <= 4 ? 4 : 2);
    static constexpr int MAXP = R <= 2 ? 4 : (R <= 4 ? 4 : 2);  // pieces per batch
};

template <typename T, int D, int G, int SQ, bool FUSED, bool MASK>
__global__ void __launch_bounds__(decode_waves(G * SQ) * 64) decode_attention_kernel(DecodeParams p) {
    constexpr int R = G * SQ;
    using Shape = DecodeShape<T, D, R>;
    constexpr int LPK = Shape::LPK, WAVES = Shape::WAVES, U = Shape::U, MAXP = Shape::MAXP;
    constexpr int CW = ElemInfo<T>::CW;
    constexpr int QCH = D / CW;         // 16-byte chunks of a row
    constexpr int NCH = QCH / LPK;      // chunks per lane
    constexpr int EPL = NCH * CW;       // elements per lane
    constexpr int GPW = 64 / LPK;       // lane groups (keys in flight per step) per wave
    constexpr int KPW = GPW * U;        // keys per wave block
    constexpr int ES = sizeof(T);
    static_assert(!FUSED || (ES == 2 && D == 128 && SQ == 1), "fused path: bf16, D=128, one query");

    __shared__ int sm_rec[MAXP][kPieceInts];
    __shared__ int sm_off[MAXP + 1];
    __shared__ U4 sm_q[MAXP][R][QCH];                 // query rows (rotated when fused)
    __shared__ U4 sm_new[FUSED ? MAXP : 1][2][16];    // fused: rotated new key, new value
    __shared__ float sm_state[MAXP][WAVES][R][D + 2];
    __shared__ int sm_last[MAXP];
    __shared__ int sm_count;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane / LPK, cl = lane % LPK;
    const int h = blockIdx.x % p.Hkv;
    const int bin = blockIdx.x / p.Hkv;
    const int B = p.B;

    // a plan for another batch, bin count or context is never followed (nothing is written)
    if (p.plan[0] != p.nbins || p.plan[2] != B || p.plan[4] != p.ctx) return;
    const int slot_pieces = p.plan[3];
    const int *records = p.plan + kPlanHeader + (p.nbins + 7) / 8 * 8 + (int64_t)bin * slot_pieces * kPieceInts;

    // the bin's piece count and its first records in one round trip
    if (tid == 0) sm_count = p.plan[kPlanHeader + bin];
    if (tid < MAXP * kPieceInts && tid < slot_pieces * kPieceInts) sm_rec[tid / kPieceInts][tid % kPieceInts] = records[tid];

    // Requests without a valid position attend nothing; their rows are written as zeros
    // (one position per thread; such requests are rare, so the rows are written serially).
    if (bin == 0) {
        for (int b = tid; b < B; b += blockDim.x) {
            const int64_t pp = p.pos[b];
            if (pp >= 0 && pp < p.ctx) continue;
            for (int t = 0; t < R * D; ++t) {
                const int r = t / D, d = t % D;
                const int qi = r / G, hq = h * G + r % G;
                store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, 0.f);
            }
        }
    }
    __syncthreads();
    const int npieces = sm_count;

    for (int batch0 = 0; batch0 < npieces; batch0 += MAXP) {
        const int np = npieces - batch0 < MAXP ? npieces - batch0 : MAXP;
        if (batch0 > 0) {
            if (tid < np * kPieceInts)
                sm_rec[tid / kPieceInts][tid % kPieceInts] = records[(int64_t)batch0 * kPieceInts + tid];
            __syncthreads();
        }
        // batch-local key offsets of the pieces
        if (tid == 0) {
            int o = 0;
            for (int i = 0; i < np; ++i) {
                sm_off[i] = o;
                o += sm_rec[i][2] - sm_rec[i][1];
            }
            sm_off[np] = o;
        }
        __syncthreads();
        const int *off = sm_off;
        const int span = off[np];
        const int ws = span * wave / WAVES, we = span * (wave + 1) / WAVES;

        // this wave's part of piece i, in key indices of its request: [ja, je); the new key
        // (fused, last piece of a request) is attended separately after the arena keys
        auto part_of = [&](int i, int &ja, int &je, int &jend, bool &with_new) {
            const int ps = ws > off[i] ? ws : off[i], pe = we < off[i + 1] ? we : off[i + 1];
            if (ps >= pe) return false;
            ja = sm_rec[i][1] + (ps - off[i]);
            je = sm_rec[i][1] + (pe - off[i]);
            with_new = FUSED && je == sm_rec[i][3];
            jend = with_new ? je - 1 : je;
            return true;
        };
        auto next_part = [&](int i) {
            int ja, je, jend;
            bool wn;
            for (++i; i < np; ++i)
                if (part_of(i, ja, je, jend, wn)) return i;
            return np;
        };
        auto row_base = [&](int i, const char *base_ptr, int64_t sb, int64_t sh) {
            const int b = sm_rec[i][0];
            const int64_t off_b = p.offs ? p.offs[b] : (int64_t)b * sb;
            return base_ptr + (off_b + h * sh) * ES;
        };

        U4 ka[U][NCH], va[U][NCH];
        // K/V rows of a piece start at wave-uniform bases (kept in scalar registers); each key
        // is a 32-bit byte offset from them, shared by K and V when their strides agree
        const bool same_stride = p.k_st == p.v_st;
        auto load_block = [&](int i, int base, int jend) {
            const char *kb = row_base(i, p.k, p.k_sb, p.k_sh);
            const char *vb = row_base(i, p.v, p.v_sb, p.v_sh);
            kb = uniform_ptr(kb);
            vb = uniform_ptr(vb);
            const int kst = (int)(p.k_st * ES), vst = (int)(p.v_st * ES);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = base + grp + GPW * u;
                const int js = j < jend ? j : base;
                const uint32_t ko = (uint32_t)(js * kst) + cl * 16;
                const uint32_t vo = same_stride ? ko : (uint32_t)(js * vst) + cl * 16;
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    ka[u][c] = load16(kb + ko + c * LPK * 16);
                    va[u][c] = load16(vb + vo + c * LPK * 16);
                }
            }
        };

        const int i_first = next_part(-1);

        // ---- prologue: query rows of every piece into LDS (rotated when fused); fused: the new
        //      key/value rows of pieces ending a request, rotated, written to the arena and LDS ----
        if constexpr (FUSED) {
            for (int t = tid; t < np * (R + 1) * 8; t += blockDim.x) {
                const int c = t & 7, rr = (t >> 3) % (R + 1), i = (t >> 3) / (R + 1);
                const int b = sm_rec[i][0];
                const bool ends = sm_rec[i][2] == sm_rec[i][3];
                if (rr == R && !ends) continue;
                const char *crow = p.cs + b * p.cs_sb * 2, *srow = p.sn + b * p.cs_sb * 2;
                const U4 c1 = load16(crow + c * 16), c2 = load16(crow + 128 + c * 16);
                const U4 s1 = load16(srow + c * 16), s2 = load16(srow + 128 + c * 16);
                if (rr < R) {
                    const char *row = p.q + (b * p.q_sb + (h * G + rr) * p.q_sh) * ES;
                    U4 x1 = load16(row + c * 16), x2 = load16(row + 128 + c * 16), y1, y2;
                    rope8(&x1.x, &x2.x, &c1.x, &c2.x, &s1.x, &s2.x, &y1.x, &y2.x);
                    sm_q[i][rr][c] = y1;
                    sm_q[i][rr][c + 8] = y2;
                } else {
                    const int64_t last = sm_rec[i][3] - 1;
                    const char *nkrow = p.nk + (b * p.nk_sb + h * p.nk_sh) * ES;
                    const char *nvrow = p.nv + (b * p.nv_sb + h * p.nv_sh) * ES;
                    U4 x1 = load16(nkrow + c * 16), x2 = load16(nkrow + 128 + c * 16), y1, y2;
                    const U4 v1 = load16(nvrow + c * 16), v2 = load16(nvrow + 128 + c * 16);
                    rope8(&x1.x, &x2.x, &c1.x, &c2.x, &s1.x, &s2.x, &y1.x, &y2.x);
                    sm_new[i][0][c] = y1;
                    sm_new[i][0][c + 8] = y2;
                    sm_new[i][1][c] = v1;
                    sm_new[i][1][c + 8] = v2;
                    char *dk = (char *)row_base(i, p.k, p.k_sb, p.k_sh) + last * p.k_st * ES;
                    char *dv = (char *)row_base(i, p.v, p.v_sb, p.v_sh) + last * p.v_st * ES;
                    store16(dk + c * 16, y1);
                    store16(dk + 128 + c * 16, y2);
                    store16(dv + c * 16, v1);
                    store16(dv + 128 + c * 16, v2);
                }
            }
        } else {
            for (int t = tid; t < np * R * QCH; t += blockDim.x) {
                const int c = t % QCH, r = (t / QCH) % R, i = t / (QCH * R);
                const int qi = r / G, hq = h * G + r % G;
                sm_q[i][r][c] = load16(p.q + (sm_rec[i][0] * p.q_sb + qi * p.q_ss + hq * p.q_sh) * ES + c * 16);
            }
        }
        __syncthreads();

        // ---- stream this wave's keys, piece by piece, KPW keys per block ----
        for (int i = i_first; i < np; i = next_part(i)) {
            int ja, je, jend;
            bool with_new;
            part_of(i, ja, je, jend, with_new);
            const int last_pos = sm_rec[i][3] - 1;
            const int b = sm_rec[i][0];
            const char *mask_row = MASK ? p.mask + b * p.m_sb * (p.mask_dtype == Q3T_F32 ? 4 : p.mask_dtype == Q3T_BOOL ? 1 : 2) : nullptr;
            U4 qr[R][NCH];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < NCH; ++c) qr[r][c] = sm_q[i][r][c * LPK + cl];
            float m[R], l[R], acc[R][EPL];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                m[r] = kEmpty;
                l[r] = 0.f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[r][e] = 0.f;
            }
            for (int base = ja; base < jend; base += KPW) {
                load_block(i, base, jend);
                bool valid[U];
                int kidx[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    kidx[u] = base + grp + GPW * u;
                    valid[u] = kidx[u] < jend;
                }
                softmax_step<T, R, G, SQ, NCH, EPL, U, LPK, MASK>(p, qr, ka, va, valid, kidx, last_pos,
                                                            mask_row, m, l, acc);
            }
            if constexpr (FUSED) {
                if (with_new) {  // attend the new key at position pos[b], rotated in the prologue
                    U4 k1[1][NCH], v1[1][NCH];
                    bool valid[1] = {grp == 0};
                    int kidx[1] = {last_pos};
#pragma unroll
                    for (int c = 0; c < NCH; ++c) {
                        k1[0][c] = sm_new[i][0][c * LPK + cl];
                        v1[0][c] = sm_new[i][1][c * LPK + cl];
                    }
                    softmax_step<T, R, G, SQ, NCH, EPL, 1, LPK, MASK>(p, qr, k1, v1, valid, kidx, last_pos,
                                                                mask_row, m, l, acc);
                }
            }

            // merge the lane-group states of the wave (lanes differing in the bits above the
            // group), VALU only
#pragma unroll
            for (int step = (LPK == 16 ? 1 : 0); step < 3; ++step) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float mo = step == 0 ? xor8(m[r]) : step == 1 ? xor16(m[r]) : xor32(m[r]);
                    const float lo2 = step == 0 ? xor8(l[r]) : step == 1 ? xor16(l[r]) : xor32(l[r]);
                    const float mn = fmaxf(m[r], mo);
                    const float a = fexp2(m[r] - mn), bb = fexp2(mo - mn);
                    l[r] = l[r] * a + lo2 * bb;
                    m[r] = mn;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        const float x = acc[r][e];
                        const float xo = step == 0 ? xor8(x) : step == 1 ? xor16(x) : xor32(x);
                        acc[r][e] = x * a + xo * bb;
                    }
                }
            }
            if (grp == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
#pragma unroll
                    for (int c = 0; c < NCH; ++c)
#pragma unroll
                        for (int e = 0; e < CW; ++e)
                            sm_state[i][wave][r][(c * LPK + cl) * CW + e] = acc[r][c * CW + e];
                    if (cl == 0) {
                        sm_state[i][wave][r][D] = m[r];
                        sm_state[i][wave][r][D + 1] = l[r];
                    }
                }
            }
        }
        __syncthreads();

        // ---- merge the waves of every piece; publish partials of split requests ----
        for (int i = 0; i < np; ++i) {
            const int b = sm_rec[i][0];
            const int slot = sm_rec[i][4];
            float *part = slot >= 0 ? p.partials + ((int64_t)h * p.max_slots + slot) * (R * (D + 2)) : nullptr;
            int live[WAVES];
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const int a0 = span * w / WAVES, a1 = span * (w + 1) / WAVES;
                live[w] = (a0 > off[i] ? a0 : off[i]) < (a1 < off[i + 1] ? a1 : off[i + 1]);
            }
            for (int t = tid; t < R * D; t += blockDim.x) {
                const int r = t / D, d = t % D;
                float M = kEmpty;
#pragma unroll
                for (int w = 0; w < WAVES; ++w)
                    if (live[w]) M = fmaxf(M, sm_state[i][w][r][D]);
                float Ls = 0.f, A = 0.f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) {
                    if (live[w]) {
                        const float wt = fexp2(sm_state[i][w][r][D] - M);
                        Ls += sm_state[i][w][r][D + 1] * wt;
                        A += sm_state[i][w][r][d] * wt;
                    }
                }
                if (!part) {
                    const int qi = r / G, hq = h * G + r % G;
                    store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, A / Ls);
                } else {
                    publish(&part[r * (D + 2) + d], A);
                    if (d == 0) {
                        publish(&part[r * (D + 2) + D], M);
                        publish(&part[r * (D + 2) + D + 1], Ls);
                    }
                }
            }
        }

        // ---- split requests: count arrivals; the last workgroup merges every partial in order ----
        bool any_split = false;
        for (int i = 0; i < np; ++i) any_split |= sm_rec[i][4] >= 0;
        if (any_split) {
            wait_stores();
            __syncthreads();
            if (tid < np) {
                int last = 0;
                if (sm_rec[tid][4] >= 0) {
                    const int old = __hip_atomic_fetch_add(&p.counters[h * B + sm_rec[tid][0]], 1,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    last = old == sm_rec[tid][5] - 1;
                }
                sm_last[tid] = last;
            }
            __syncthreads();
            for (int i = 0; i < np; ++i) {
                if (!sm_last[i]) continue;
                const int b = sm_rec[i][0], n = sm_rec[i][5], first = sm_rec[i][6];
                for (int t = tid; t < R * D; t += blockDim.x) {
                    const int r = t / D, d = t % D;
                    float M = kEmpty;
                    for (int k = 0; k < n; ++k) {
                        const float *pp = p.partials + ((int64_t)h * p.max_slots + first + k) * (R * (D + 2));
                        M = fmaxf(M, collect(pp + r * (D + 2) + D));
                    }
                    float Ls = 0.f, A = 0.f;
                    for (int k = 0; k < n; ++k) {
                        const float *pp = p.partials + ((int64_t)h * p.max_slots + first + k) * (R * (D + 2));
                        const float wt = fexp2(collect(pp + r * (D + 2) + D) - M);
                        Ls += collect(pp + r * (D + 2) + D + 1) * wt;
                        A += collect(pp + r * (D + 2) + d) * wt;
                    }
                    const int qi = r / G, hq = h * G + r % G;
                    store_out<T>(p.out + (b * p.o_sb + qi * p.o_ss + hq * p.o_sh + d) * ES, A / Ls);
                }
                if (tid == 0)
                    __hip_atomic_store(&p.counters[h * B + b], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();  // LDS is reused by the next batch
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

// One workgroup per CU: CUs / kv_heads bins per head.
static int64_t default_bins(int64_t kv_heads) {
    int64_t bins = (int64_t)device_cus() / (kv_heads > 0 ? kv_heads : 1);
    if (bins < 1) bins = 1;
    if (bins > kMaxBins) bins = kMaxBins;
    return bins;
}

// The counter region has one fixed size, so that the counters of every launch sit on bytes
// that only ever hold counters (all zero between launches), whatever batch and head count
// earlier launches on the same workspace used.
constexpr int64_t kMaxCounters = 65536;  // kv_heads * batch
static int64_t counters_bytes() { return kMaxCounters * 4; }
static int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace q3t

using namespace q3t;

extern "C" int64_t q3t_decode_plan_bytes(int64_t batch, int64_t bins) {
    if (batch < 0 || batch > kMaxBatch) return -1;
    if (bins <= 0) bins = default_bins(8);
    if (bins > kMaxBins) return -1;
    return plan_ints(batch, bins) * 4;
}

extern "C" int q3t_decode_plan(const int64_t *positions, int64_t batch, int64_t ctx, int64_t bins,
                               void *plan, int64_t plan_bytes, void *stream) {
    if (!positions || !plan || batch < 1 || batch > kMaxBatch || ctx < 1 || ctx > (1 << 20) ||
        bins < 1 || bins > kMaxBins)
        return Q3T_EINVAL;
    if (plan_bytes < plan_ints(batch, bins) * 4 || !aligned(plan, 16)) return Q3T_EWORKSPACE;
    hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream,
                       positions, (int)batch, (int)ctx, (int)bins, (int *)plan);
    return launch_status();
}

extern "C" int64_t q3t_decode_workspace_bytes(int64_t batch, int64_t query_len, int64_t q_heads,
                                              int64_t kv_heads, int64_t head_dim, int64_t bins) {
    if (batch < 0 || batch > kMaxBatch || query_len < 1 || kv_heads < 1 || q_heads < kv_heads ||
        head_dim < 1)
        return -1;
    if (bins <= 0) bins = default_bins(kv_heads);
    if (bins > kMaxBins) return -1;
    const int64_t R = (q_heads / kv_heads) * query_len;
    return counters_bytes() + round256(plan_ints(batch, bins) * 4) +
           kv_heads * (batch + bins) * R * (head_dim + 2) * 4;
}

template <typename T, int D, int G, int SQ, bool F, bool M>
static void launch_decode(const DecodeParams &p, hipStream_t s) {
    hipLaunchKernelGGL((decode_attention_kernel<T, D, G, SQ, F, M>), dim3(p.Hkv * p.nbins),
                       dim3(decode_waves(G * SQ) * 64), 0, s, p);
}

template <typename T, int D, int G>
static int dispatch_sq(const DecodeParams &p, int sq, bool fused, hipStream_t s) {
    if (fused) {
        if constexpr (sizeof(T) == 2 && D == 128) {
            if (sq != 1 || p.has_mask) return Q3T_EUNSUPPORTED;
            launch_decode<T, D, G, 1, true, false>(p, s);
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
    // key rows are addressed by 32-bit byte offsets from a request's base
    const int64_t max_st = a->k_stride_t > a->v_stride_t ? a->k_stride_t : a->v_stride_t;
    if (max_st < 0 || a->ctx * max_st * es + a->head_dim * es > INT32_MAX) return Q3T_EUNSUPPORTED;
    const int64_t bins = a->bins > 0 ? a->bins : default_bins(a->kv_heads);
    if (bins > kMaxBins || a->kv_heads * bins > (int64_t)1 << 30) return Q3T_EINVAL;
    const int64_t need = q3t_decode_workspace_bytes(a->batch, a->query_len, a->q_heads, a->kv_heads,
                                                    a->head_dim, bins);
    if (!a->workspace || a->workspace_bytes < need || !aligned(a->workspace, 16)) return Q3T_EWORKSPACE;
    if (a->plan && (a->plan_bytes < plan_ints(a->batch, bins) * 4 || !aligned(a->plan, 16)))
        return Q3T_EWORKSPACE;

    hipStream_t s = (hipStream_t)stream;
    char *ws = (char *)a->workspace;
    const int *plan = (const int *)a->plan;
    if (!plan) {  // build this call's plan in the workspace
        int *own = (int *)(ws + counters_bytes());
        hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, a->positions,
                           (int)a->batch, (int)a->ctx, (int)bins, own);
        plan = own;
    }

    DecodeParams p;
    p.B = (int)a->batch;
    p.Hq = (int)a->q_heads;
    p.Hkv = (int)a->kv_heads;
    p.ctx = (int)a->ctx;
    p.nbins = (int)bins;
    p.max_slots = (int)(a->batch + bins);  // split pieces never exceed batch + bins
    p.scale_log2 = a->scale * kLog2e;
    p.has_mask = a->mask != nullptr;
    p.mask_dtype = (int)a->mask_dtype;
    p.plan = plan;
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
    p.counters = (int *)ws;
    p.partials = (float *)(ws + counters_bytes() + round256(plan_ints(a->batch, bins) * 4));

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
