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

// One wave per token; a lane's work item is 8 dims of each half of one of the token's head
// rows.  Heads [0, Hq) are query heads (rotated into q_out; absent when q_out is null, the
// attention kernel then rotates the queries itself); the Hkv heads after them rotate the key
// and copy the value into the arena at the token's position within its request (without value
// rows, p.v null, only the keys: the attention launch copies the values).  The token's
// request, position and slot are the same for the whole wave: 12.5 -> 12.0 us per layer on
// the 16-prompt workload (keys and values) against one item per thread with per-lane lookups,
// and 12.0 -> 11.0 us with the request found by one ballot instead of a binary search of
// dependent loads; keys only, 6.5 us.  (Two tokens per wave, the next one's rows requested
// before the current one's are stored, or non-temporal stores: no gain.)
__global__ void __launch_bounds__(256) prefill_rope_write_kernel(PrefillRopeWriteParams p) {
    const int vecs = p.D / 16;
    const int qh = p.qo ? p.Hq : 0;  // without q_out only the key/value rows are handled
    const int items = (qh + p.Hkv) * vecs;
    const int half = p.D / 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Up to 64 requests, lane i holds request i's first token and slot, loaded once per wave in
    // one round trip; a token's request is then a ballot (the count of requests starting at or
    // before it, less one), not a binary search of dependent loads.
    int start_l = 0x7fffffff;
    int64_t slot_l = 0;
    if (p.B <= 64 && lane < p.B) {
        start_l = p.cu[lane];
        slot_l = p.slots ? p.slots[lane] : lane;
    }
    // a token's request: the last one starting at or before it
    auto locate = [&](int t, int &pos, int64_t &slot) {
        if (p.B <= 64) {
            const int n = __builtin_popcountll(__builtin_amdgcn_ballot_w64(start_l <= t));
            const int b = n > 0 ? n - 1 : 0;
            pos = t - __builtin_amdgcn_readlane(start_l, b);
            slot = ((int64_t)__builtin_amdgcn_readlane((int)(slot_l >> 32), b) << 32) |
                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)slot_l, b);
        } else {
            const int b = request_of(p.cu, p.B, t);
            pos = t - p.cu[b];
            slot = p.slots ? p.slots[b] : b;
        }
    };
    for (int t = blockIdx.x * 4 + wave; t < (int)p.T; t += gridDim.x * 4) {
        int pos;
        int64_t slot;
        locate(t, pos, slot);
        const bool write_kv = pos >= 0 && pos < p.capacity;
        const char *crow = p.cs + (int64_t)t * p.cs_st * 2, *srow = p.sn + (int64_t)t * p.cs_st * 2;
        for (int it = lane; it < items; it += 64) {
            const int c = it % vecs, hd = it / vecs;
            U4 c1 = load16(crow + c * 16), c2 = load16(crow + (half + c * 8) * 2);
            U4 s1 = load16(srow + c * 16), s2 = load16(srow + (half + c * 8) * 2);
            if (hd < qh) {
                const char *row = p.q + ((int64_t)t * p.q_st + hd * p.q_sh) * 2;
                U4 x1 = load16(row + c * 16), x2 = load16(row + (half + c * 8) * 2), y1, y2;
                rope8(&x1.x, &x2.x, &c1.x, &c2.x, &s1.x, &s2.x, &y1.x, &y2.x);
                char *orow = p.qo + ((int64_t)t * p.qo_st + hd * p.qo_sh) * 2;
                store16(orow + c * 16, y1);
                store16(orow + (half + c * 8) * 2, y2);
            } else if (write_kv) {
                const int h = hd - qh;
                const char *krow = p.k + ((int64_t)t * p.k_st + h * p.k_sh) * 2;
                U4 x1 = load16(krow + c * 16), x2 = load16(krow + (half + c * 8) * 2), y1, y2;
                U4 w1 = {0u, 0u, 0u, 0u}, w2 = w1;
                if (p.v) {  // without value rows the attention launch copies them
                    const char *vrow = p.v + ((int64_t)t * p.v_st + h * p.v_sh) * 2;
                    w1 = load16(vrow + c * 16);
                    w2 = load16(vrow + (half + c * 8) * 2);
                }
                rope8(&x1.x, &x2.x, &c1.x, &c2.x, &s1.x, &s2.x, &y1.x, &y2.x);
                const int64_t a = (slot * p.a_sb + h * p.a_sh + pos * p.a_st) * 2;
                store16(p.ak + a + c * 16, y1);
                store16(p.ak + a + (half + c * 8) * 2, y2);
                if (p.v) {
                    store16(p.av + a + c * 16, w1);
                    store16(p.av + a + (half + c * 8) * 2, w2);
                }
            }
        }
    }
}


// ---- varlen causal attention on bf16 MFMA tiles ------------------------------------------
//
// One workgroup of 4 waves per (request, 64-query block, GH query heads of one KV head);
// wave w owns queries q0 + 16w ... q0 + 16w + 15 of every one of the GH heads, so each K and
// V read from LDS feeds the products of all GH heads (GH = 2: 168 VGPRs, 3 waves per SIMD,
// every workgroup of the 16-prompt workload resident at once).  Keys stream through
// a ring of kStages LDS stages of kTile keys (K rows then V rows), filled by buffer loads
// that write LDS directly (16 bytes per lane) kStages - 1 tiles ahead of the products, so
// the K/V reads never pass through registers.  Rows are stored unpadded with their 16-byte
// chunks XOR-swizzled (K chunk ch of row r at ch ^ (r & 15), V at ch ^ (2r & 15)), which
// keeps the 16-byte K reads of 16 rows and the transposing 8-byte V reads of 8 rows on
// distinct banks.  With v_mfma_f32_16x16x32_bf16 (lane l = 16g + c holds A[c][8g..8g+7],
// B[8g..8g+7][c] and D[4g..4g+3][c]), per 32 keys:
//   S^T (keys x queries) = K . Q^T   A = K rows from LDS, B = the wave's Q rows (registers);
//                                    lane (g, c) gets keys 4g..4g+3 and 16+4g..16+4g+3 of
//                                    query c;
//   O^T (dims x queries) += V^T . P^T   B = P^T straight from the S^T registers (K index
//                                    order {4g..4g+3, 16+4g..16+4g+3}); A = V^T read by
//                                    ds_read_b64_tr_b16: within a 16-lane group, lane c reads
//                                    4 dims of key row 4g + c/4 and receives, after the
//                                    transpose, keys 4g..4g+3 of dim c.
// Each lane keeps the online-softmax state of one query per head.  The causal mask is applied only
// on the steps that straddle the wave's diagonal or the end of the keys.  The running
// maximum moves only when a step's maximum exceeds it by more than kRescaleLog2 (log2
// units), so the accumulators are rescaled rarely and unnormalised weights stay below
// 2^kRescaleLog2 (well inside bf16 and fp32 range).
constexpr int kQBlock = 64;
constexpr int kXcds = 8;        // MI355X: 8 XCDs of 32 CUs
constexpr int kCusPerXcd = 32;
constexpr int kTile = 32;     // keys per LDS stage and per softmax step
constexpr int kStages = 3;    // LDS ring depth: loads run kStages - 1 tiles ahead
constexpr float kLog2eP = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;

struct PrefillParams {
    int B, Hq, Hkv, nqb, group;
    int64_t T;
    float scale_log2;
    const int32_t *cu;
    const char *q;
    int64_t q_st, q_sh;
    const char *k;
    char *v;  // written only with nv (the copy workgroups)
    int64_t k_sb, k_sh, k_st, v_sb, v_sh, v_st;
    int64_t cap;
    const int64_t *slots;
    char *out;
    int64_t o_st, o_sh;
    const char *cs, *sn;  // optional cos/sin rows per token: the query rows are rotated on load
    int64_t cs_st;
    const int32_t *kvl;   // optional keys per request (a right-padded batch): query i sees keys
                          // j <= i with j < kvl[b]
    const char *mask;     // optional (B, 1, Lq, capacity) additive mask: every key is scored
    int mdt;              // mask element type (Q3T_BF16, Q3T_F16 or Q3T_F32)
    int64_t m_sb, m_sq;   // mask strides (elements) of requests and query rows; keys unit-stride
    // optional value rows of the step's tokens as the projection wrote them: the products
    // read them (key j of request b is token cu[b] + j) and the workgroups past the
    // attention grid copy them into the arena view `v` at each token's position
    const char *nv;
    int64_t nv_st, nv_sh;
    int attn_wgs;         // workgroups of the attention grid (the copy workgroups follow)
};

constexpr int kCopyTokens = 16;  // value rows of 16 packed tokens per copy workgroup

// Copy workgroup `unit`: for each group of 16 of its packed tokens, wave w copies the value
// rows (every KV head) of tokens 4w ... 4w + 3 into the arena at their positions within their
// requests (rows past the capacity are not stored), all of a group's loads issued before its
// first store.
template <int D>
Q3T_DEVICE void copy_value_rows(const PrefillParams &p, int unit) {
    constexpr int CPR = D / 8;  // 16-byte chunks per row
    constexpr int PER = 8;      // chunks per lane in flight
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int start_l = 0x7fffffff;
    int64_t slot_l = 0;
    if (p.B <= 64 && lane < p.B) {
        start_l = p.cu[lane];
        slot_l = p.slots ? p.slots[lane] : lane;
    }
    const int chunks = p.Hkv * CPR;  // per token
    for (int group = 0; group < kCopyTokens / 16; ++group) {
        const int t0 = unit * kCopyTokens + group * 16 + 4 * wave;
        if (t0 >= p.T) break;
        // the four tokens' arena row offsets (elements), -1 for no row
        int64_t row[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + j;
            row[j] = -1;
            if (t >= p.T) continue;
            int start;
            int64_t slot;
            if (p.B <= 64) {
                const int n = __builtin_popcountll(__builtin_amdgcn_ballot_w64(start_l <= t));
                const int b = n > 0 ? n - 1 : 0;
                start = __builtin_amdgcn_readlane(start_l, b);
                slot = ((int64_t)__builtin_amdgcn_readlane((int)(slot_l >> 32), b) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)slot_l, b);
            } else {
                const int b = request_of(p.cu, p.B, t);
                start = p.cu[b];
                slot = p.slots ? p.slots[b] : b;
            }
            const int pos = t - start;
            if (pos >= 0 && pos < p.cap) row[j] = slot * p.v_sb + (int64_t)pos * p.v_st;
        }
        for (int f0 = 0; f0 < 4 * chunks; f0 += 64 * PER) {
            U4 buf[PER];
            int64_t dst[PER];
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int f = f0 + 64 * i + lane, j = f / chunks, it = f % chunks;
                const int hh = it / CPR, ch = it % CPR;
                const int64_t r = j == 0 ? row[0] : j == 1 ? row[1] : j == 2 ? row[2] : j == 3 ? row[3] : -1;
                dst[i] = r < 0 ? -1 : (r + hh * p.v_sh) * 2 + ch * 16;
                buf[i] = dst[i] < 0 ? U4{0u, 0u, 0u, 0u}
                                    : load16(p.nv + ((int64_t)(t0 + j) * p.nv_st + hh * p.nv_sh) * 2 + ch * 16);
            }
#pragma unroll
            for (int i = 0; i < PER; ++i)
                if (dst[i] >= 0) store16(p.v + dst[i], buf[i]);
        }
    }
}

constexpr float kEmptyP = -1.0e30f;  // finite running maximum before any visible key (masked)

// 16 bytes of a mask tile row in LDS -> 4 (2-byte types) or 2 x 2 (fp32: two reads) values in
// log2 units; positive infinity never occurs in an additive mask, -inf (and finfo.min, which
// overflows to -inf once scaled) gives a zero weight.
template <int MB>
Q3T_DEVICE void mask_values(uint32_t addr, int mdt, float (&mv)[4]) {
    if constexpr (MB == 2) {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t w = *(__attribute__((address_space(3))) const u32x2_t *)(uintptr_t)addr;
        const uint32_t h[4] = {w.x & 0xffffu, w.x >> 16, w.y & 0xffffu, w.y >> 16};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = mdt == Q3T_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)h[i])
                                           : bf16_to_float(h[i]);
            mv[i] = v * kLog2eP;
        }
    } else {
        const U4 w = lds_read16(addr);
        const uint32_t f[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) mv[i] = __uint_as_float(f[i]) * kLog2eP;
    }
}

// MB: bytes per mask element (0: no mask, 2: bf16 / fp16, 4: fp32).  Without a mask the
// causal rule (and the optional per-request key counts) bounds the key tiles of each query
// block; with a mask every key tile of the view is scored and the mask alone decides, its
// tile (64 query rows x 32 keys) staged through the same LDS ring as the keys and values.
template <int D, int GH, int MB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GH == 1 ? 4 : 3)))
prefill_attention_kernel(PrefillParams p) {
    constexpr int NT = 256;                       // threads
    constexpr int KK = D / 32;                    // MFMA steps over the head dimension
    constexpr int DB = D / 16;                    // 16-row blocks of O^T
    constexpr int CPR = D / 8;                    // 16-byte chunks per row
    constexpr int ROW = D * 2;                    // bytes per row
    constexpr int KBYTES = kTile * ROW;           // K part of a stage
    constexpr int RB = kTile * MB;                // mask bytes per query row of a tile
    constexpr int MBYTES = kQBlock * RB;          // mask tile of a stage
    constexpr int SBYTES = 2 * KBYTES + MBYTES;   // stage: K rows, V rows, mask rows
    constexpr int LPT = 2 * kTile * CPR / NT;     // 16-byte loads per thread per tile
    constexpr int LPR = MB ? RB / 16 : 1;         // lanes per mask row
    constexpr int RPI = 64 / LPR;                 // mask rows per wave load
    constexpr int LPTM = MB ? 16 / RPI : 0;       // mask loads per wave per tile (16 rows)
    constexpr int WAIT = LPT + LPTM;              // loads of one tile per thread
    static_assert(LPT >= 1 && (2 * kTile * CPR) % NT == 0, "a tile is whole loads per thread");
    static_assert(KBYTES % 1024 == 0, "a wave's load never straddles K and V");
    __shared__ __attribute__((aligned(1024))) uint8_t ring[kStages * SBYTES];

    // the wave index through readfirstlane: wave-uniform for the compiler too, so that the
    // per-wave load resources stay in scalar registers
    if ((int)blockIdx.x >= p.attn_wgs) {  // past the attention grid: value rows to copy
        if constexpr (MB == 0) copy_value_rows<D>(p, (int)blockIdx.x - p.attn_wgs);
        return;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int hgroups = p.Hq / GH;
    // Placement: the hardware deals workgroup i to XCD i % 8 and, within an XCD, to its 32 CUs
    // in turn, so CU k of an XCD holds the XCD's workgroups k, k + 32, k + 64 at once (three
    // per CU).  Work items are numbered longest first; reversing the order within the second
    // and third of every four rounds of 32 puts a short item next to every long one on a CU.
    // Measured on the 16-prompt workload (seed 0): the most loaded CU from 27 to 20 tiles.
    const int wg = [&] {
        const int xcd = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
        const int rounds = p.attn_wgs / (kXcds * kCusPerXcd);  // complete rounds on every XCD
        if (j >= rounds * kCusPerXcd) return (int)blockIdx.x;
        const int r = j / kCusPerXcd, pos = j % kCusPerXcd;
        const bool flip = (r & 3) == 1 || (r & 3) == 2;
        return (r * kCusPerXcd + (flip ? kCusPerXcd - 1 - pos : pos)) * kXcds + xcd;
    }();
    const int hq0 = (wg % hgroups) * GH;  // the workgroup's first query head
    const int h = hq0 / p.group;          // the workgroup's KV head
    const int rest = wg / hgroups;
    // Work item `rest` of this head group: a (64-query block qb, request b) pair, numbered with
    // the longest blocks first.  Up to 64 requests the numbering is dense: only pairs with
    // rows exist, so the grid's round-robin placement over shader engines sees real work
    // evenly (empty slots in between would pile long blocks onto some engines and stall the
    // in-order dispatch behind them).  Lane i holds request i's row range; each level counts
    // the requests with a block there (ballot) and the item's request is picked by rank
    // (mbcnt), all wave-uniform, with no memory access beyond the row offsets.
    int b, qb, t0, n, kn;
    int64_t slot;
    if (p.B <= 64) {
        int start = 0, rows = 0, klen = 0;
        int64_t slot_l = 0;  // the request's arena slot, loaded with its rows (no later round trip)
        if (lane < p.B) {
            start = p.cu[lane];
            rows = (start < 0 || start >= p.T) ? 0 : (int)min((int64_t)(p.cu[lane + 1] - start), p.T - start);
            klen = p.kvl ? p.kvl[lane] : rows;
            slot_l = p.slots ? p.slots[lane] : lane;
        }
        const int blocks = rows > 0 ? (rows + kQBlock - 1) / kQBlock : 0;
        int remaining = rest;
        qb = -1;
        b = 0;
        for (int level = p.nqb - 1; level >= 0; --level) {
            const uint64_t has = __builtin_amdgcn_ballot_w64(blocks > level);
            const int count = __builtin_popcountll(has);
            if (remaining < count) {
                const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(has >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)has, 0u));
                const uint64_t pick = __builtin_amdgcn_ballot_w64(blocks > level && (int)rank == remaining);
                b = __builtin_ctzll(pick);
                qb = level;
                break;
            }
            remaining -= count;
        }
        if (qb < 0) return;  // past the last block with rows
        t0 = __builtin_amdgcn_readlane(start, b);
        n = __builtin_amdgcn_readlane(rows, b);
        kn = __builtin_amdgcn_readlane(klen, b);
        slot = ((int64_t)__builtin_amdgcn_readlane((int)(slot_l >> 32), b) << 32) |
               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)slot_l, b);
    } else {
        b = rest % p.B;
        qb = p.nqb - 1 - rest / p.B;  // the longest blocks are dispatched first
        t0 = p.cu[b];
        if (t0 < 0 || t0 >= p.T) return;
        n = (int)min((int64_t)(p.cu[b + 1] - t0), p.T - t0);  // rows past the packed tokens do not exist
        kn = p.kvl ? p.kvl[b] : n;
        slot = p.slots ? p.slots[b] : b;
    }
    const int q0 = qb * kQBlock;
    if (q0 >= n) return;
    // keys 0 ... kv_end-1 are visible to this block; the arena holds at most `cap` of them.
    // Causal: up to the block's last query and the request's key count; masked: every key.
    const int kv_end = MB ? (int)p.cap : (int)min((int64_t)min(min(n, kn), q0 + kQBlock), p.cap);
    const int ntiles = kv_end > 0 ? (kv_end + kTile - 1) / kTile : 0;
    const int wq0 = q0 + 16 * wave;              // first query of this wave
    // keys [0, wave_end) can be visible to the wave; steps reaching past mask_from need the
    // per-key rule (the diagonal or the end of the keys).  A wave whose queries all lie past
    // the request (the tail of its last block) scores nothing: it only loads its share of
    // every tile and joins the barriers.
    const int wave_end = wq0 >= n ? 0 : MB ? kv_end : min(wq0 + 16, kv_end);
    const int mask_from = MB ? kv_end : min(wq0 + 1, kv_end);
    const int qpos = wq0 + c;
    const bool qvalid = qpos < n;
    const int lim = MB ? kv_end - 1 : min(qpos, kv_end - 1);  // last key visible to this lane's query

    // tile loader: load i of a thread fills LDS slot s = i * NT + tid (16 bytes) of a stage:
    // row s / CPR (K rows first, then V rows), physical chunk s % CPR, holding logical chunk
    // (physical ^ swizzle(row)) of key tile * kTile + row
    const char *kbase = p.k + (slot * p.k_sb + h * p.k_sh) * 2;
    const char *vbase = MB == 0 && p.nv ? p.nv + ((int64_t)t0 * p.nv_st + h * p.nv_sh) * 2
                                        : p.v + (slot * p.v_sb + h * p.v_sh) * 2;
    const uint32_t kst = (uint32_t)(p.k_st * 2), vst = (uint32_t)((MB == 0 && p.nv ? p.nv_st : p.v_st) * 2);
    const i32x4_t krs = scalar_rsrc(kbase, kv_end > 0 ? (uint32_t)((kv_end - 1) * kst + D * 2) : 0u);
    const i32x4_t vrs = scalar_rsrc(vbase, kv_end > 0 ? (uint32_t)((kv_end - 1) * vst + D * 2) : 0u);
    // mask rows of the request's queries (rows past its queries read zeros)
    const uint32_t mrow = (uint32_t)(p.m_sq * MB);
    const i32x4_t mrs = scalar_rsrc(MB ? p.mask + b * p.m_sb * MB : kbase,
                                    MB ? (uint32_t)((n - 1) * (int64_t)mrow + p.cap * MB) : 0u);
    const uint32_t ring_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring;
    uint32_t row_off[LPT];
    int row_of[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
        const int s = i * NT + tid, rall = s / CPR, pc = s % CPR;
        const bool is_v = rall >= kTile;
        const int r = rall % kTile;
        const int ch = pc ^ ((is_v ? 2 * r : r) & (CPR - 1));
        row_of[i] = r;
        row_off[i] = (uint32_t)r * (is_v ? vst : kst) + ch * 16;
    }
    auto issue = [&](int kt, int stage) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int first_slot = i * NT + wave * 64;             // wave-uniform
            const bool is_v = first_slot / CPR >= kTile;
            const int key0 = kt * kTile;
            const uint32_t off = row_of[i] < kv_end - key0
                                     ? row_off[i] + (uint32_t)key0 * (is_v ? vst : kst)
                                     : 0xfffffff0u;
            load_to_lds16(is_v ? vrs : krs, off,
                          (uint32_t)__builtin_amdgcn_readfirstlane((int)(ring_base + stage * SBYTES + first_slot * 16)));
        }
        if constexpr (MB > 0) {
            // the wave's own 16 query rows of the mask tile: load i covers rows RPI i ... + RPI - 1
#pragma unroll
            for (int i = 0; i < LPTM; ++i) {
                const int r = 16 * wave + i * RPI + lane / LPR;
                const uint32_t off = q0 + r < n ? (uint32_t)(q0 + r) * mrow + (uint32_t)(kt * RB + (lane % LPR) * 16)
                                                : 0xfffffff0u;
                load_to_lds16(mrs, off, (uint32_t)__builtin_amdgcn_readfirstlane(
                                            (int)(ring_base + stage * SBYTES + 2 * KBYTES + (16 * wave + i * RPI) * RB)));
            }
        }
    };

    // per-lane LDS read addresses within a stage
    uint32_t ka[KK], va[DB];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) ka[kk] = c * ROW + (((4 * kk + g) ^ (c & (CPR - 1))) * 16);
    {
        const int r = 4 * g + (c >> 2);  // key row of this lane's transposed read (+16 for keys 16..31)
        const int sw = (2 * r) & (CPR - 1);
#pragma unroll
        for (int db = 0; db < DB; ++db)
            va[db] = KBYTES + r * ROW + (((2 * db + ((c >> 1) & 1)) ^ sw) * 16) + 8 * (c & 1);
    }

    // the first tiles go out before anything else waits on memory
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
        if (s < ntiles) issue(s, s);

    // the wave's query rows as B operands: Q[query c][8g + 32kk ...], zeros past the request
    bf16x8_t qB[GH][KK];
    // with cos/sin: the lane's RoPE rows (its query token, dims 32kk + 8g ... + 7 and the same
    // dims D/2 further), shared by the GH heads
    U4 rc1[KK / 2], rc2[KK / 2], rs1[KK / 2], rs2[KK / 2];
    if (p.cs) {
        const int64_t tr = (int64_t)(t0 + (qvalid ? qpos : 0)) * p.cs_st * 2;
#pragma unroll
        for (int kk = 0; kk < KK / 2; ++kk) {
            const int d1 = (32 * kk + 8 * g) * 2, d2 = d1 + D;  // bytes of dims d and d + D/2
            rc1[kk] = load16(p.cs + tr + d1);
            rc2[kk] = load16(p.cs + tr + d2);
            rs1[kk] = load16(p.sn + tr + d1);
            rs2[kk] = load16(p.sn + tr + d2);
        }
    }
#pragma unroll
    for (int j = 0; j < GH; ++j) {
        const char *row = p.q + ((int64_t)(t0 + (qvalid ? qpos : 0)) * p.q_st + (hq0 + j) * p.q_sh) * 2;
        U4 qv[KK];
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qv[kk] = load16(row + (32 * kk + 8 * g) * 2);
        if (p.cs) {
            // rotate-half RoPE in registers (bf16-exact; the rotated rows are never stored, so
            // NaN payloads need no canonical form): the lane's dims 32kk + 8g ... + 7 pair with
            // the same dims of kk + KK/2, which the lane holds as well
#pragma unroll
            for (int kk = 0; kk < KK / 2; ++kk) {
                U4 y1, y2;
                rope8<false>(&qv[kk].x, &qv[kk + KK / 2].x, &rc1[kk].x, &rc2[kk].x, &rs1[kk].x, &rs2[kk].x,
                             &y1.x, &y2.x);
                qv[kk] = y1;
                qv[kk + KK / 2] = y2;
            }
        }
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            if (!qvalid) qv[kk] = U4{0u, 0u, 0u, 0u};
            qB[j][kk] = as_bf16x8(qv[kk]);
        }
    }

    f32x4_t acc[GH][DB];
    float m[GH], l[GH];  // running maximum (scaled log2 units) and this lane's weight sum
#pragma unroll
    for (int j = 0; j < GH; ++j) {
        m[j] = 0.f;
        l[j] = 0.f;
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[j][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    bool first = true;
    const float sl = p.scale_log2;

    auto step = [&](int kt, uint32_t sbase) {
        const int kb0 = kt * kTile;  // first key of the step
        if (kb0 >= wave_end) return;  // past this wave's keys
        const bool masked = kb0 + kTile > mask_from;  // the step reaches past the diagonal or the keys
        const int rel = lim - kb0;
        float mk[8];
        if constexpr (MB > 0) {
            const uint32_t mrow_lds = sbase + 2 * KBYTES + (16 * wave + c) * RB;
            float lo[4], hi[4];
            mask_values<MB>(mrow_lds + 4 * g * MB, p.mdt, lo);
            mask_values<MB>(mrow_lds + (16 + 4 * g) * MB, p.mdt, hi);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mk[i] = lo[i];
                mk[4 + i] = hi[i];
            }
        }
        bf16x8_t pB[GH];
#pragma unroll
        for (int j = 0; j < GH; ++j) {
            // S^T of head j for keys kb0 + 16kb + (4g..4g+3); a wave issuing products goes
            // first, the others do their softmax meanwhile
            f32x4_t st0 = {0.f, 0.f, 0.f, 0.f}, st1 = {0.f, 0.f, 0.f, 0.f};
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                const bf16x8_t a0 = as_bf16x8(lds_read16(sbase + ka[kk]));
                const bf16x8_t a1 = as_bf16x8(lds_read16(sbase + ka[kk] + 16 * ROW));
                st0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qB[j][kk], st0, 0, 0, 0);
                st1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qB[j][kk], st1, 0, 0, 0);
            }
            __builtin_amdgcn_s_setprio(0);
            float x[8] = {st0[0], st0[1], st0[2], st0[3], st1[0], st1[1], st1[2], st1[3]};
            if constexpr (MB > 0) {  // scores in log2 units with the mask added
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = __builtin_fmaf(x[e], sl, mk[e]);
            }
            if (masked) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (4 * g + i > rel) x[i] = -INFINITY;
                    if (16 + 4 * g + i > rel) x[4 + i] = -INFINITY;
                }
            }
            float mx = x[0];
#pragma unroll
            for (int e = 1; e < 8; ++e) mx = __builtin_amdgcn_fmed3f(mx, x[e], __builtin_inff());
            // the step maximum of a query is the largest of its four lanes' maxima (scaling is
            // monotonic, so it commutes with the maximum): some query exceeds its running maximum
            // by more than kRescaleLog2 exactly when some lane's own maximum does, and the
            // maximum across lanes is needed only to start and to rescale
            float mt = MB ? mx : mx * sl;
            if (first || __builtin_amdgcn_ballot_w64(mt > m[j] + kRescaleLog2) != 0) {
                mt = __builtin_amdgcn_fmed3f(mt, xor16(mt), __builtin_inff());
                mt = __builtin_amdgcn_fmed3f(mt, xor32(mt), __builtin_inff());
                if constexpr (MB > 0) mt = fmaxf(mt, kEmptyP);  // a fully masked step keeps m finite
                if (first) {
                    m[j] = mt;
                } else {
                    const float mn = fmaxf(m[j], mt);
                    const float alpha = fexp2(m[j] - mn);
                    m[j] = mn;
                    l[j] *= alpha;
#pragma unroll
                    for (int db = 0; db < DB; ++db) acc[j][db] *= alpha;
                }
            }
            float pv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[e] = MB ? fexp2(x[e] - m[j]) : fexp2(__builtin_fmaf(x[e], sl, -m[j]));
            l[j] += ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
            const U4 packed = {cvt_pk_bf16(pv[0], pv[1]), cvt_pk_bf16(pv[2], pv[3]),
                               cvt_pk_bf16(pv[4], pv[5]), cvt_pk_bf16(pv[6], pv[7])};
            pB[j] = as_bf16x8(packed);
        }
        first = false;
        // O^T += V^T . P^T, one V read for every head
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const uint2 lo = lds_read_tr16(sbase + va[db]), hi = lds_read_tr16(sbase + va[db] + 16 * ROW);
            const bf16x8_t av = as_bf16x8(U4{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
            for (int j = 0; j < GH; ++j)
                acc[j][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pB[j], acc[j][db], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    };
    // one ring position: wait for this tile's loads (later tiles stay in flight), barrier
    // (every wave is done with the stage the next load overwrites), issue the tile
    // kStages - 1 ahead into that stage, then the products
    auto ring_step = [&](int kt, int stage) {
        if (kt + 1 < ntiles) wait_loads<WAIT>();  // the one younger tile stays in flight
        else wait_loads<0>();
        lds_barrier();
        if (kt + kStages - 1 < ntiles) issue(kt + kStages - 1, (stage + kStages - 1) % kStages);
        step(kt, ring_base + stage * SBYTES);
    };
    static_assert(kStages == 3, "the waits above and the unrolled ring below assume three stages");
    for (int kt = 0; kt < ntiles; kt += kStages) {
        ring_step(kt, 0);
        if (kt + 1 < ntiles) ring_step(kt + 1, 1);
        if (kt + 2 < ntiles) ring_step(kt + 2, 2);
    }

    if (!qvalid) return;
#pragma unroll
    for (int j = 0; j < GH; ++j) {
        float lt = l[j] + xor16(l[j]);
        lt += xor32(lt);
        const float inv = lt > 0.f ? __builtin_amdgcn_rcpf(lt) : 0.f;  // no visible key: zero row
        char *orow = p.out + ((int64_t)(t0 + qpos) * p.o_st + (hq0 + j) * p.o_sh) * 2;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const uint2 v = {cvt_pk_bf16(acc[j][db][0] * inv, acc[j][db][1] * inv),
                             cvt_pk_bf16(acc[j][db][2] * inv, acc[j][db][3] * inv)};
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
    if (a->total_tokens > (1 << 30)) return Q3T_EUNSUPPORTED;  // 32-bit token indices
    if (a->total_tokens == 0) return Q3T_OK;
    // q_out == NULL: keys and values only (the attention kernel rotates the queries itself)
    const bool with_q = a->q_out != nullptr;
    // value == NULL: keys only (q3t_prefill_attention then copies the values, new_values)
    const bool with_v = a->value != nullptr;
    if (!a->cu_seqlens || (with_q && !a->query) || !a->key || !a->cos || !a->sin || !a->arena_keys ||
        (with_v && !a->arena_values))
        return Q3T_EINVAL;
    const int64_t st[] = {with_q ? a->q_stride_t : 0, with_q ? a->q_stride_h : 0, a->k_stride_t, a->k_stride_h,
                          with_v ? a->v_stride_t : 0, with_v ? a->v_stride_h : 0, a->cs_stride_t,
                          with_q ? a->qo_stride_t : 0, with_q ? a->qo_stride_h : 0, a->a_stride_b,
                          a->a_stride_h, a->a_stride_t};
    for (int64_t s : st)
        if ((s * 2) % 16) return Q3T_EINVAL;
    const void *ptrs[] = {with_q ? a->query : a->key, a->key, with_v ? a->value : a->key, a->cos, a->sin,
                          with_q ? a->q_out : a->key, a->arena_keys, with_v ? a->arena_values : a->key};
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
    p.ak = (char *)a->arena_keys; p.av = with_v ? (char *)a->arena_values : nullptr;
    p.a_sb = a->a_stride_b; p.a_sh = a->a_stride_h; p.a_st = a->a_stride_t;
    p.slots = a->kv_slots;
    int64_t blocks = (p.T + 3) / 4;  // one token per wave
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(prefill_rope_write_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, p);
    return launch_status();
}


template <int D, int GH>
static void launch_prefill(const PrefillParams &p, hipStream_t s) {
    const int64_t hgroups = p.Hq / GH;
    int64_t wgs = (int64_t)p.B * p.nqb * hgroups;
    if (p.B <= 64) {
        // items are numbered densely: a request of L rows has ceil(L / 64) blocks, so there are
        // at most (T + 63 B) / 64 of them; rounded up to whole rounds of one workgroup per CU,
        // which keeps the placement of every item as in the full grid
        const int64_t items = (p.T + (int64_t)(kQBlock - 1) * p.B) / kQBlock;
        const int64_t round = kXcds * kCusPerXcd;
        const int64_t bound = (items * hgroups + round - 1) / round * round;
        if (bound < wgs) wgs = bound;
    }
    PrefillParams q = p;
    q.attn_wgs = (int)wgs;
    if (p.nv) wgs += (p.T + kCopyTokens - 1) / kCopyTokens;
    const dim3 grid((uint32_t)wgs);
    if (!p.mask) hipLaunchKernelGGL((prefill_attention_kernel<D, GH, 0>), grid, dim3(256), 0, s, q);
    else if (p.mdt == Q3T_F32) hipLaunchKernelGGL((prefill_attention_kernel<D, GH, 4>), grid, dim3(256), 0, s, q);
    else hipLaunchKernelGGL((prefill_attention_kernel<D, GH, 2>), grid, dim3(256), 0, s, q);
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
    if ((a->cos != nullptr) != (a->sin != nullptr)) return Q3T_EINVAL;
    if (a->cos && (!aligned(a->cos, 16) || !aligned(a->sin, 16) || a->cs_stride_t < 0 || (a->cs_stride_t * 2) % 16))
        return Q3T_EINVAL;
    // key rows of one (slot, head) are addressed by 32-bit byte offsets
    const int64_t max_st = a->k_stride_t > a->v_stride_t ? a->k_stride_t : a->v_stride_t;
    if (a->capacity * max_st * 2 + a->head_dim * 2 > INT32_MAX) return Q3T_EUNSUPPORTED;
    if (a->mask) {
        // rows of 16-byte aligned keys, addressed by 32-bit offsets from a request's base
        if (a->mask_dtype != Q3T_BF16 && a->mask_dtype != Q3T_F16 && a->mask_dtype != Q3T_F32) return Q3T_EUNSUPPORTED;
        const int64_t es = a->mask_dtype == Q3T_F32 ? 4 : 2;
        if (!aligned(a->mask, 16) || a->mask_stride_q < 0 || a->mask_stride_b < 0 || (a->mask_stride_q * es) % 16 ||
            (a->mask_stride_b * es) % 16)
            return Q3T_EINVAL;
        if ((a->max_seqlen - 1) * a->mask_stride_q * es + a->capacity * es > INT32_MAX) return Q3T_EUNSUPPORTED;
    }
    if (a->new_values) {
        // value rows of the step's tokens: only for the causal rule (a mask scores every key
        // of the arena view, beyond the step's rows); 32-bit row offsets from a request's
        // first token
        if (a->mask) return Q3T_EINVAL;
        if (!aligned(a->new_values, 16) || a->nv_stride_t < 0 || a->nv_stride_h < 0 || (a->nv_stride_t * 2) % 16 ||
            (a->nv_stride_h * 2) % 16)
            return Q3T_EINVAL;
        const int64_t rows = a->capacity < a->max_seqlen ? a->capacity : a->max_seqlen;
        if (rows * a->nv_stride_t * 2 + a->head_dim * 2 > INT32_MAX) return Q3T_EUNSUPPORTED;
    }
    PrefillParams p;
    p.B = (int)a->batch; p.Hq = (int)a->q_heads; p.Hkv = (int)a->kv_heads;
    p.group = (int)G;
    p.nqb = (int)((a->max_seqlen + kQBlock - 1) / kQBlock);
    if ((int64_t)p.B * p.nqb * p.Hq + (a->total_tokens + kCopyTokens - 1) / kCopyTokens > INT32_MAX)
        return Q3T_EUNSUPPORTED;
    p.scale_log2 = a->scale * kLog2eP;
    p.cu = a->cu_seqlens;
    p.q = (const char *)a->query; p.q_st = a->q_stride_t; p.q_sh = a->q_stride_h;
    p.k = (const char *)a->keys; p.v = (char *)a->values;
    p.k_sb = a->k_stride_b; p.k_sh = a->k_stride_h; p.k_st = a->k_stride_t;
    p.v_sb = a->v_stride_b; p.v_sh = a->v_stride_h; p.v_st = a->v_stride_t;
    p.slots = a->kv_slots;
    p.cap = a->capacity;
    p.T = a->total_tokens;
    p.out = (char *)a->out; p.o_st = a->o_stride_t; p.o_sh = a->o_stride_h;
    p.cs = (const char *)a->cos; p.sn = (const char *)a->sin; p.cs_st = a->cs_stride_t;
    p.kvl = a->kv_lens;
    p.mask = (const char *)a->mask;
    p.mdt = (int)a->mask_dtype;
    p.m_sb = a->mask_stride_b; p.m_sq = a->mask_stride_q;
    p.nv = (const char *)a->new_values; p.nv_st = a->nv_stride_t; p.nv_sh = a->nv_stride_h;
    p.attn_wgs = 0;  // set at launch
    hipStream_t s = (hipStream_t)stream;
    // the query heads of a KV head pair up in one workgroup and share its staged K/V tiles
    if (G % 2 == 0) {
        if (a->head_dim == 128) launch_prefill<128, 2>(p, s);
        else launch_prefill<64, 2>(p, s);
    } else {
        if (a->head_dim == 128) launch_prefill<128, 1>(p, s);
        else launch_prefill<64, 1>(p, s);
    }
    return launch_status();
}
