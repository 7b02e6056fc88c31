// Ragged grouped-query decode attention on the shares grid: the talker step's launch.
//
// Reference behaviour (InferMatrixLab/qwen3-tts-rsi-engine), as on the other grids
// (decode_attention.hip):
//   out[b, hq] = softmax(q[b, hq] . K[b, hq/G, :L_b]^T * scale + mask) . V[b, hq/G, :L_b]
//   with L_b = pos[b] + 1 (SlotGraph.compute's mask `j <= pos[b]`, continuous.py:191-192,
//   dispatched from PackedAttention.forward, packed_attention.py:75-84, to
//   npu_attention.attention, npu_attention.py:11-26, which adds the layer's mask).
// Fused: RoPE of q and of the new key (packed_attention.py:46-51, rotary_triton_ascend.py:19-24)
// and the paired K/V write at pos[b] (continuous.py:152-166, kv_triton_ascend.py:24-36).
//
// Design.  One workgroup per CU: KV head h, bundle m of M.  The keys of all requests of a
// head, laid end to end in request order (a request's keys 0 ... L_b - 1), are cut into M
// shares of whole 64-key stages (the first r shares one stage longer, the last one taking
// the rest), so every workgroup streams the same number of stages whatever the spread of
// the lengths.  The cut is made once per step by the plan kernel (all layers of a talker
// step attend the same lengths) and read by every layer's launch in one scalar round trip.
//   * A share is a list of up to 8 segments (a request and a key range of it).  The share's
//     keys stream through a two-stage LDS ring as one packed sequence: a 64-key stage may hold
//     the end of one request and the start of the next, so no stage is partly empty except
//     the share's last.  K/V rows are loaded by global-to-LDS buffer loads (every request of
//     the head through one buffer resource, 32-bit row offsets), one stage ahead of the one
//     being scored, with explicit waits.
//   * Every segment of the share is a set of G columns of the 16 MFMA columns: S^T = K . Q^T
//     with v_mfma_f32_16x16x32_bf16 scores a wave's 16 keys against the query rows of all
//     the share's requests at once, a key counts only in the columns of its own segment, and
//     each column keeps its own online softmax and its O^T accumulator (O^T += V^T . P^T with
//     v_mfma_f32_16x16x16_bf16).  Request boundaries cost nothing inside the stream.
//   * A request cut between two or three shares is merged across workgroups.  A share
//     streams the part of the request it cuts first, so that part is finished early: its
//     waves publish their column states (device-scope stores) and, two stages later, when the
//     stores have completed, a flag per wave.  The share holding the request's last part
//     streams it last, reads the earlier parts' flags four stages before its stream ends and
//     their states two stages before, so both arrive with its last stages and the merge adds
//     no latency; it then clears the flags for the next launch.
//   * The plan falls back to whole requests paired longest with shortest (no cut) when a
//     share would hold more segments than MFMA columns or a request would span more than
//     three shares.
#include "decode_params.hpp"

namespace q3t {
namespace shares {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kSlots = 8;      // plan entries (segments) per share
constexpr int kPeers = 2;      // continuation parts a merging share reads
constexpr int kStageKeys = 64;
constexpr int kWaveKeys = 16;
constexpr int kRow = 256;                         // bf16 rows of D = 128
constexpr int kWaveStage = 2 * kWaveKeys * kRow;  // K rows then V rows of one wave: 8 KiB
constexpr int kStageBytes = kWaves * kWaveStage;  // 32 KiB
constexpr int kStageLoads = 8;                    // 1 KiB loads per wave and stage
constexpr int kGroups = 256;                      // workgroups of a launch: one per CU
constexpr int kMaxBatch = 128;
constexpr int kMaxBundles = 256;
constexpr float kRescaleLog2 = 8.0f;  // the running maximum moves when exceeded by more than this
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kEmpty = -1.0e30f;
// polls of a merging share for a flag (each a device-scope load, ~1-2 us, then a short sleep);
// the flags are set microseconds into the launch, so reaching the limit means a plan that lists
// a continued request without its later parts: the merged rows are then NaN
constexpr int kSpinLimit = 1 << 16;
// entry info bits: the segment holds the request's last key; it is the last part of a request
// cut between shares and merges the parts of the shares before (their count in bits 4-7); it
// is an earlier part of a cut request and publishes its state
constexpr int kLast = 1, kMerge = 2, kPublish = 4, kPeerShift = 4;

// Shares per KV head and segment columns of a launch shape.
inline int64_t bundle_count(int64_t batch, int64_t kv_heads) {
    const int64_t m = (kGroups + kv_heads - 1) / kv_heads;
    const int64_t least = (batch + 3) / 4;  // the fallback pairs at most four requests per share
    return m < least ? least : m;
}
inline int slot_cap(int64_t group) { return (int)(16 / group < kSlots ? 16 / group : kSlots); }
// floats of one wave's published state: G accumulator rows of 128, then (max, sum) per row
template <int G>
constexpr int record_floats() { return G * 128 + 8; }

typedef int i32x8_t __attribute__((ext_vector_type(8)));


// Global-to-LDS loads with the device-scope (sc1) policy, for states another workgroup wrote
// in this launch; 16 bytes or 4 bytes per lane at lds_base + size * lane.
Q3T_DEVICE void load_to_lds16_coherent(i32x4_t rsrc, uint32_t voffset, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\t" Q3T_VMEM_SGPR_WAIT "buffer_load_dwordx4 %1, %2, 0 offen sc1 lds"
                 :: "s"(lds_base), "v"(voffset), "s"(rsrc) : "memory", "m0");
}
Q3T_DEVICE void load_to_lds4_coherent(i32x4_t rsrc, uint32_t voffset, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\t" Q3T_VMEM_SGPR_WAIT "buffer_load_dword %1, %2, 0 offen sc1 lds"
                 :: "s"(lds_base), "v"(voffset), "s"(rsrc) : "memory", "m0");
}
Q3T_DEVICE void load_to_lds4(i32x4_t rsrc, uint32_t voffset, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\t" Q3T_VMEM_SGPR_WAIT "buffer_load_dword %1, %2, 0 offen lds"
                 :: "s"(lds_base), "v"(voffset), "s"(rsrc) : "memory", "m0");
}
// Stores issued from inline assembly, so that the loop knows exactly how many memory
// operations it has in flight besides the ring's loads (the wait for a stage may then leave
// them outstanding, see wait_slack); lanes with an offset outside the resource store nothing.
Q3T_DEVICE void store16_asm(i32x4_t rsrc, uint32_t voffset, U4 v) {
    asm volatile(Q3T_VMEM_SGPR_WAIT "buffer_store_dwordx4 %0, %1, %2, 0 offen\n\ts_nop 1"
                 :: "v"(__builtin_bit_cast(i32x4_t, v)), "v"(voffset), "s"(rsrc) : "memory");
}
Q3T_DEVICE void store16_asm_coherent(i32x4_t rsrc, uint32_t voffset, U4 v) {
    asm volatile(Q3T_VMEM_SGPR_WAIT "buffer_store_dwordx4 %0, %1, %2, 0 offen sc1\n\ts_nop 1"
                 :: "v"(__builtin_bit_cast(i32x4_t, v)), "v"(voffset), "s"(rsrc) : "memory");
}
Q3T_DEVICE void store8_asm_coherent(i32x4_t rsrc, uint32_t voffset, float a, float b) {
    typedef int i32x2_t __attribute__((ext_vector_type(2)));
    const i32x2_t v = {__float_as_int(a), __float_as_int(b)};
    asm volatile(Q3T_VMEM_SGPR_WAIT "buffer_store_dwordx2 %0, %1, %2, 0 offen sc1\n\ts_nop 1" :: "v"(v), "v"(voffset), "s"(rsrc) : "memory");
}
Q3T_DEVICE void store4_asm_coherent(i32x4_t rsrc, uint32_t voffset, int v) {
    asm volatile(Q3T_VMEM_SGPR_WAIT "buffer_store_dword %0, %1, %2, 0 offen sc1" :: "v"(v), "v"(voffset), "s"(rsrc) : "memory");
}
// The wait for a stage when `extra` memory operations went out after the stage's loads (in
// issue order: this stage, the extra operations, the next stage): vmcnt(B + extra) lets the
// extra ones and the next stage stay in flight; operations complete in issue order, so the
// stage itself has landed.  More than 24 extra operations: a stronger wait.
template <int B, int N = 0>
Q3T_DEVICE void wait_slack(int extra) {
    if constexpr (N >= 24) {
        wait_loads<B + 24>();
    } else {
        if (extra <= N) wait_loads<B + N>();
        else wait_slack<B, N + 1>(extra);
    }
}
constexpr int kPolicyCoherent = 16;  // sc1: device scope
// RMSNorm of one bf16 row of 128 spread over a 16-lane group (8 elements per lane), as the
// attention module's q_norm / k_norm compute it: fp32 sum of squares (lanes, then the DPP
// tree), x * rsqrt(mean + eps) rounded to bf16, times the bf16 weight, rounded to bf16.
Q3T_DEVICE U4 rms_norm_row(const U4 &x, const U4 &w, float eps) {
    const uint32_t v[4] = {x.x, x.y, x.z, x.w}, wt[4] = {w.x, w.y, w.z, w.w};
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = bf16_lo(v[i]), b = bf16_hi(v[i]);
        ss = __builtin_fmaf(a, a, ss);
        ss = __builtin_fmaf(b, b, ss);
    }
    ss = sum8(ss);
    ss += xor8(ss);
    const float r = __builtin_amdgcn_rsqf(ss * (1.0f / 128.0f) + eps);
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t n = cvt_pk_bf16(bf16_lo(v[i]) * r, bf16_hi(v[i]) * r);
        y[i] = cvt_pk_bf16_canon(bf16_lo(n) * bf16_lo(wt[i]), bf16_hi(n) * bf16_hi(wt[i]));
    }
    return U4{y[0], y[1], y[2], y[3]};
}

// A mask term (log2 units) from the 4-byte word holding it; `sub` = its byte offset in the word.
Q3T_DEVICE float mask_term(uint32_t word, uint32_t sub, int dtype) {
    const uint32_t x = word >> (8 * sub);
    switch (dtype) {
        case Q3T_BF16: return bf16_to_float(x & 0xffffu) * kLog2e;
        case Q3T_F16: return (float)__builtin_bit_cast(_Float16, (uint16_t)(x & 0xffffu)) * kLog2e;
        case Q3T_F32: return __uint_as_float(word) * kLog2e;
        default: return (x & 0xffu) ? 0.0f : -INFINITY;  // bool: True attends
    }
}

template <int G>
struct Lds {
    static constexpr int PEER_ACC = G * 128 < 256 ? 256 : G * 128;  // whole 1 KiB load runs
    char ring[2][kStageBytes];
    uint32_t maskw[2][kWaves][64];                // mask words of a stage's rows, per wave
    char head[kSlots][8][kRow];                   // per segment: query rows, cos, sin, new K, new V
    float acc[kWaves][16][132];                   // every wave's column states after the stream
                                                  // (rows padded: the 16 columns on distinct banks)
    float ml[kWaves][16][2];
    float peer_acc[kPeers][kWaves][PEER_ACC];     // published states of the next shares' parts
    float peer_ml[kPeers][kWaves][64];
    int flags[kWaves][64];
    int segb[kSlots];                             // request of each segment
    int fail[kWaves];
};

// NORM: the fused q/k RMSNorm is compiled in (a separate instance: the bundled kernel's norm
// code, even unexecuted, cost the talker step 1.8 us per launch).  MASK: an additive or bool
// (batch, 1, ctx) mask with unit key stride is added to the scores.
template <int G, bool FUSED, bool STREAM, bool NORM, bool MASK>
__global__ void __launch_bounds__(kThreads)
decode_shares_kernel(const int32_t *plan, int nb, int hkv, int M, DecodeParams p) {
    static_assert(G == 1 || G == 2 || G == 4, "query rows per KV head");
    constexpr int CAP = 16 / G < kSlots ? 16 / G : kSlots;
    constexpr int REC = record_floats<G>();
    constexpr int KL = kStageLoads + (MASK ? 1 : 0);  // loads per wave and stage
    __shared__ __attribute__((aligned(16))) Lds<G> s;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Share m of head h.  A merging share waits for the flags of the shares before it, which
    // have lower workgroup indices: they were dispatched before it, so it never waits for a
    // workgroup that is not yet resident.
    const int h = blockIdx.x % hkv, m = blockIdx.x / hkv;

    // fused norm weights (chunk c of the row): requested first and awaited before any ring load
    U4 qw = {0u, 0u, 0u, 0u}, kw = {0u, 0u, 0u, 0u};
    if constexpr (FUSED && NORM) {
        if (p.qnw) qw = load16(p.qnw + c * 16);
        if (p.knw) kw = load16(p.knw + c * 16);
    }
    // The share's eight plan entries, the plan header and one dword of every 64-byte line of
    // the argument block in one scalar round trip (the plan pointer and the sizes its
    // addresses need are the leading arguments, preloaded into scalar registers).
    i32x8_t e01, e23, e45, e67, hdr;
    {
        const uint64_t pa = reinterpret_cast<uint64_t>(plan) + (uint64_t)m * (kSlots * 16);
        const uint64_t ha = reinterpret_cast<uint64_t>(plan) + (uint64_t)M * (kSlots * 16);
        constexpr int BYTES = 32 + (int)sizeof(DecodeParams);
        static_assert(BYTES <= 8 * 64, "eight 64-byte lines at most");
        const uint64_t ka = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
        uint32_t d0, d1, d2, d3, d4, d5, d6, d7;
        asm volatile("s_load_dwordx8 %0, %13, 0x0\n\ts_load_dwordx8 %1, %13, 0x20\n\t"
                     "s_load_dwordx8 %2, %13, 0x40\n\ts_load_dwordx8 %3, %13, 0x60\n\t"
                     "s_load_dwordx8 %4, %14, 0x0\n\t"
                     "s_load_dword %5, %15, 0x0\n\ts_load_dword %6, %15, 0x40\n\t"
                     "s_load_dword %7, %15, 0x80\n\ts_load_dword %8, %15, 0xc0\n\t"
                     "s_load_dword %9, %15, %16\n\ts_load_dword %10, %15, %17\n\t"
                     "s_load_dword %11, %15, %18\n\ts_load_dword %12, %15, %19\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&s"(e01), "=&s"(e23), "=&s"(e45), "=&s"(e67), "=&s"(hdr), "=&s"(d0), "=&s"(d1),
                       "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7)
                     : "s"(pa), "s"(ha), "s"(ka), "n"(BYTES > 0x100 ? 0x100 : 0), "n"(BYTES > 0x140 ? 0x140 : 0),
                       "n"(BYTES > 0x180 ? 0x180 : 0), "n"(BYTES > 0x1c0 ? 0x1c0 : 0)
                     : "memory");
    }
    if constexpr (FUSED && NORM) asm volatile("" :: "v"(qw.x), "v"(kw.x) : "memory");
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the weights before any ring load

    const bool vec_out = ((reinterpret_cast<uintptr_t>(p.out) | (uintptr_t)(p.o_sb * 2) | (uintptr_t)(p.o_sh * 2)) & 15) == 0;
    auto store_row = [&](int b, int cc, const uint16_t *src, bool zero) {  // one output row, 16 lanes
        const int ch = tid & 15;
        U4 v = {0u, 0u, 0u, 0u};
        if (!zero) v = *reinterpret_cast<const U4 *>(src + ch * 8);
        char *dst = p.out + (b * p.o_sb + (h * G + cc) * p.o_sh) * 2;
        if (vec_out) {
            store16(dst + ch * 16, v);
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 8; ++i)
                *reinterpret_cast<uint16_t *>(dst + (ch * 8 + i) * 2) = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
        }
    };
    // A plan made for another batch or head shape: NaN rows for the requests b = m (mod M) (a
    // loud failure rather than stale outputs).  The plan's ctx only decided which positions
    // count; a launch over a narrower context (a mask's width) clamps the segments to it.
    if (hdr[0] != nb || hdr[1] != M || hdr[2] != CAP) {
        for (int b = m; b < nb; b += M)
            for (int t = tid; t < G * 128; t += kThreads)
                *reinterpret_cast<uint16_t *>(p.out + (b * p.o_sb + (h * G + t / 128) * p.o_sh + t % 128) * 2) = 0x7fc0;
        return;
    }

    // ---- the share's segments: lane k of every wave holds segment k ------------------------
    // Vector registers, read into scalars (v_readlane) only where the stream crosses a segment
    // boundary: as eight scalar tables live through the stream they spilled into lanes and
    // were reloaded on every stage.
    const int sl = lane & (kSlots - 1);
    int vb, vj0, vj1, vinf;
    {
        const int raw[kSlots][4] = {{e01[0], e01[1], e01[2], e01[3]}, {e01[4], e01[5], e01[6], e01[7]},
                                    {e23[0], e23[1], e23[2], e23[3]}, {e23[4], e23[5], e23[6], e23[7]},
                                    {e45[0], e45[1], e45[2], e45[3]}, {e45[4], e45[5], e45[6], e45[7]},
                                    {e67[0], e67[1], e67[2], e67[3]}, {e67[4], e67[5], e67[6], e67[7]}};
        vb = raw[0][0];
        vj0 = raw[0][1];
        vj1 = raw[0][2];
        vinf = raw[0][3];
#pragma unroll
        for (int k = 1; k < kSlots; ++k)
            if (sl == k) {
                vb = raw[k][0];
                vj0 = raw[k][1];
                vj1 = raw[k][2];
                vinf = raw[k][3];
            }
    }
    // entries are a prefix of the slots; one naming no request of the batch ends it
    const uint64_t unnamed = __builtin_amdgcn_ballot_w64(!(sl < CAP && vb >= 0 && vb < nb)) & 0xffull;
    const int nseg = unnamed ? (int)__builtin_ctzll(unnamed) : kSlots;
    const bool live = sl < nseg;
    vj1 = live ? min(max(vj1, 0), p.ctx) : 0;
    vj0 = live ? min(max(vj0, 0), vj1) : 0;
    vb = live ? vb : 0;
    vinf = live ? (vj1 > vj0 ? vinf : vinf & ~kLast) : 0;  // an empty segment has no new key
    // stream positions [vst, ven) of each segment: a scan over the 8 lanes of each lane group
    // (row shifts within each 16-lane row: lanes 0-7 hold the sums that are read)
    int ven = vj1 - vj0;
    ven += __builtin_amdgcn_update_dpp(0, ven, 0x111, 0xf, 0xf, true);  // row_shr:1
    ven += __builtin_amdgcn_update_dpp(0, ven, 0x112, 0xf, 0xf, true);  // row_shr:2
    ven += __builtin_amdgcn_update_dpp(0, ven, 0x114, 0xf, 0xf, true);  // row_shr:4
    const int vst = ven - (vj1 - vj0);
    auto rl = [](int v, int k) { return __builtin_amdgcn_readlane(v, k); };
    const int total_keys = rl(ven, kSlots - 1);
    const int total = (total_keys + kStageKeys - 1) / kStageKeys;
    // segments that write an output row: those holding a request's last key (a whole request,
    // or the last part of a cut one, merged with the parts published by the shares before)
    const int out_mask = (int)(__builtin_amdgcn_ballot_w64(live && (vinf & kLast)) & 0xffull);
    const bool publisher = nseg > 0 && (rl(vinf, 0) & kPublish) && rl(ven, 0) > 0;
    const int mk = nseg > 0 ? nseg - 1 : 0;
    const int minf = rl(vinf, mk);
    const bool merger = nseg > 0 && (minf & kMerge) && (minf & kLast);
    int npeers = merger ? min((minf >> kPeerShift) & 15, kPeers) : 0;
    npeers = min(npeers, m);  // the parts sit in shares m - 1, ..., m - npeers
    const bool merging = merger && npeers > 0;
    if (wave == 0 && lane < kSlots) s.segb[lane] = vb;  // read after the first barrier

    auto write_zero_rows = [&]() {
        // requests without a valid position (the header's bit mask): zero rows, written by
        // the share b % M of every head
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            uint32_t bits = (uint32_t)hdr[4 + wd];
            while (bits) {
                const int b = 32 * wd + __builtin_ctz(bits);
                bits &= bits - 1;
                if (b < nb && b % M == m && tid < 16 * G) store_row(b, tid / 16, nullptr, true);
            }
        }
    };
    if (total == 0) {
        write_zero_rows();
        return;
    }

    // ---- buffer resources and per-segment row addressing ---------------------------------
    const int kst = (int)(p.k_st * 2);
    const uint32_t range = (uint32_t)((int64_t)(nb - 1) * p.k_sb * 2 + (int64_t)(p.ctx - 1) * kst + kRow);
    const i32x4_t krs = scalar_rsrc(p.k + (int64_t)h * p.k_sh * 2, range);
    const i32x4_t vrs = scalar_rsrc(p.v + (int64_t)h * p.k_sh * 2, range);
    // stream position q of segment k is key j0 + q - vst of request b: its row sits at byte
    // vpa + q * kst; keys at or past vpe are not loaded (fused: the new key, placed in the
    // ring from LDS instead)
    const int vpa = (int)((uint32_t)((int64_t)vb * p.k_sb * 2) + (uint32_t)((vj0 - vst) * kst));
    const int vpe = live ? vst + (((FUSED && (vinf & kLast)) ? max(vj1 - 1, vj0) : vj1) - vj0) : 0;
    const int mes = MASK ? mask_elem_size(p.mask_dtype) : 0;
    i32x4_t mrs = {0, 0, 0, 0};
    if constexpr (MASK) {
        const uint32_t mbytes = (uint32_t)((((int64_t)(nb - 1) * p.m_sb + p.ctx) * mes + 3) & ~(int64_t)3);
        mrs = scalar_rsrc(p.mask, mbytes);
    }

    const uint32_t lds_ring = (uint32_t)(uintptr_t)&s.ring[0][0];
    const uint32_t lds_head = (uint32_t)(uintptr_t)&s.head[0][0][0];
    const uint32_t lds_mask = (uint32_t)(uintptr_t)&s.maskw[0][0][0];
    // the wave's producer segment (advances with the stream) and its scalars
    int pk = 0, pk_end = rl(ven, 0), pk_pe = rl(vpe, 0);
    uint32_t pk_pa = (uint32_t)rl(vpa, 0);
    auto issue = [&](int t) {
        const uint32_t base = lds_ring + (t & 1) * kStageBytes + wave * kWaveStage;
        const int P = t * kStageKeys + wave * kWaveKeys;  // stream position of the wave's first row
        while (pk + 1 < nseg && P >= pk_end) {
            ++pk;
            pk_end = rl(ven, pk);
            pk_pa = (uint32_t)rl(vpa, pk);
            pk_pe = rl(vpe, pk);
        }
        uint32_t a[4];
        int e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a[i] = pk_pa;
            e[i] = pk_pe;
        }
        if (P + kWaveKeys > pk_end) {
            // the wave's rows cross into later segments: each row takes the last segment
            // starting at or before it
            for (int k = pk + 1; k < nseg; ++k) {
                const int st = rl(vst, k);
                if (st >= P + kWaveKeys) break;
                const uint32_t ak = (uint32_t)rl(vpa, k);
                const int ek = rl(vpe, k);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (P + 4 * i + g >= st) {
                        a[i] = ak;
                        e[i] = ek;
                    }
            }
        }
#pragma unroll
        for (int i = 0; i < kWaveKeys / 4; ++i) {
            const int r = 4 * i + g, q = P + r;
            const bool ok = q < e[i];
            const uint32_t row = a[i] + (uint32_t)q * (uint32_t)kst;
            const uint32_t ko = ok ? row + ((c ^ r) & 15) * 16 : 0xfffffff0u;
            const uint32_t vo = ok ? row + ((c ^ (2 * r)) & 15) * 16 : 0xfffffff0u;
            const uint32_t kl = (uint32_t)__builtin_amdgcn_readfirstlane((int)(base + i * 1024));
            const uint32_t vl = (uint32_t)__builtin_amdgcn_readfirstlane((int)(base + kWaveKeys * kRow + i * 1024));
            if constexpr (STREAM) {
                load_to_lds16_stream(krs, ko, kl);
                load_to_lds16_stream(vrs, vo, vl);
            } else {
                load_to_lds16(krs, ko, kl);
                load_to_lds16(vrs, vo, vl);
            }
        }
        if constexpr (MASK) {
            // the mask word of each of the wave's 16 rows (lane r: row r), from the row's own
            // request; rows past the share read zeros
            const int q = P + (lane & 15);
            int mb = rl(vb, pk), mj = rl(vj0, pk), mst = rl(vst, pk), men = pk_end;
            for (int k = pk + 1; k < nseg; ++k) {
                const int st = rl(vst, k);
                if (st >= P + kWaveKeys) break;
                const int bk = rl(vb, k), jk = rl(vj0, k), ek = rl(ven, k);
                if (q >= st) {
                    mb = bk;
                    mj = jk;
                    mst = st;
                    men = ek;
                }
            }
            const int64_t elem = (int64_t)mb * p.m_sb + (mj + q - mst);
            const uint32_t off = (lane < 16 && q < men) ? (uint32_t)((elem * mes) & ~(int64_t)3) : 0xfffffff0u;
            load_to_lds4(mrs, off, (uint32_t)__builtin_amdgcn_readfirstlane((int)(lds_mask + ((t & 1) * kWaves + wave) * 256)));
        }
    };

    // ---- prologue: the first stage, every segment's rows, the second stage ---------------
    // Every wave issues its first stage at once (a wave that also loads a segment's rows would
    // otherwise start its stream behind the others and end behind them); the rows go out
    // next, and the rows' wait leaves the second stage in flight.
    int issued = 0;
    issue(0);
    ++issued;
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
        if (k >= nseg || wave != k % kWaves) continue;
        const int b = rl(vb, k);
        const uint32_t hk = (uint32_t)__builtin_amdgcn_readfirstlane((int)(lds_head + k * 8 * kRow));
        const i32x4_t qrs = scalar_rsrc(p.q + (b * p.q_sb + (int64_t)h * G * p.q_sh) * 2,
                                        (uint32_t)((G - 1) * p.q_sh * 2 + kRow));
        if (lane < 16 * G) load_to_lds16(qrs, (uint32_t)((lane >> 4) * p.q_sh * 2 + (lane & 15) * 16), hk);
        if constexpr (FUSED) {
            const i32x4_t crs = scalar_rsrc(p.cs + b * p.cs_sb * 2, kRow);
            const i32x4_t srs = scalar_rsrc(p.sn + b * p.cs_sb * 2, kRow);
            if (lane < 16) {
                load_to_lds16(crs, lane * 16, hk + 4 * kRow);
                load_to_lds16(srs, lane * 16, hk + 5 * kRow);
            }
            if (rl(vinf, k) & kLast) {
                const i32x4_t nkr = scalar_rsrc(p.nk + (b * p.nk_sb + h * p.nk_sh) * 2, kRow);
                const i32x4_t nvr = scalar_rsrc(p.nv + (b * p.nv_sb + h * p.nv_sh) * 2, kRow);
                if (lane < 16) {
                    load_to_lds16(nkr, lane * 16, hk + 6 * kRow);
                    load_to_lds16(nvr, lane * 16, hk + 7 * kRow);
                }
            }
        }
    }
    if (total > 1) {
        issue(1);
        ++issued;
    }
    // the first stage and the rows have landed (the second stage stays in flight)
    if (issued == 1) wait_loads<0>();
    else wait_loads<KL>();
    if constexpr (FUSED) {
        // rotations, each segment's in the wave that loaded its rows: lane group r < G holds
        // query row r and lane group G the new key (a second pass for G = 4), lane c chunk c
#pragma unroll
        for (int k = 0; k < kSlots; ++k) {
            if (k >= nseg || wave != k % kWaves) continue;
            const uint32_t hk = lds_head + k * 8 * kRow;
            const bool last = (rl(vinf, k) & kLast) != 0;
            const U4 cv = lds_read16(hk + 4 * kRow + c * 16), sv = lds_read16(hk + 5 * kRow + c * 16);
            auto rotate = [&](int row, bool is_key) {
                U4 x = lds_read16(hk + row * kRow + c * 16);
                if constexpr (NORM) {
                    if (is_key ? p.knw != nullptr : p.qnw != nullptr) x = rms_norm_row(x, is_key ? kw : qw, p.eps);
                }
                return rope_half8(x, xor8_u4(x), cv, sv, c < 8);
            };
            if constexpr (G < 4) {
                if (g < G) lds_write16(hk + g * kRow + c * 16, rotate(g, false));
                else if (g == G && last) lds_write16(hk + 6 * kRow + c * 16, rotate(6, true));
            } else {
                lds_write16(hk + g * kRow + c * 16, rotate(g, false));
                if (g == 0 && last) lds_write16(hk + 6 * kRow + c * 16, rotate(6, true));
            }
        }
    }
    lds_barrier();  // every segment's rows, rotated, visible to every wave

    // ---- the columns: segment c / G, query row c % G -------------------------------------
    const int cseg = c / G;
    const bool clive = cseg < nseg;
    const int cl = cseg & (kSlots - 1);
    // the column's stream range, request and first key
    const int lo = clive ? __shfl(vst, cl) : 0, hi = clive ? __shfl(ven, cl) : 0;
    const int cb = __shfl(vb, cl), cj0 = __shfl(vj0, cl);
    bf16x8_t qB[4];
    {
        const U4 zero = {0u, 0u, 0u, 0u};
        const uint32_t src = lds_head + cl * 8 * kRow + (c % G) * kRow;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const U4 x = lds_read16(src + (4 * kk + g) * 16);
            qB[kk] = as_bf16x8(clive ? x : zero);
        }
    }
    // per-lane LDS offsets within a wave's stage: K rows as the A operand of S^T (row c, dims
    // 32 kk + 8 g ...), V rows for the transposing read (row 4g + c/4, 4 dims)
    uint32_t ka[4], va[8];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) ka[kk] = c * kRow + (((4 * kk + g) ^ c) & 15) * 16;
    {
        const int r = 4 * g + (c >> 2);
#pragma unroll
        for (int db = 0; db < 8; ++db)
            va[db] = kWaveKeys * kRow + r * kRow + (((2 * db + ((c >> 1) & 1)) ^ (2 * r)) & 15) * 16 + 8 * (c & 1);
    }
    const float scale = p.scale_log2;

    // published states: per (head, share, wave) one record; flags in the counter region
    float *const recs = p.partials + (int64_t)h * M * kWaves * REC;
    const i32x4_t prs = scalar_rsrc(recs, (uint32_t)(M * kWaves * REC * 4));
    const i32x4_t frs = scalar_rsrc(p.counters + (int64_t)h * M * kWaves, (uint32_t)(M * kWaves * 4));
    auto load_peer_flags = [&]() {  // lane i < npeers: the flag of share m - 1 - i, this wave
        const uint32_t off = lane < npeers ? (uint32_t)(((m - 1 - lane) * kWaves + wave) * 4) : 0xfffffff0u;
        load_to_lds4_coherent(frs, off, (uint32_t)__builtin_amdgcn_readfirstlane((int)(uintptr_t)&s.flags[wave][0]));
    };
    auto load_peer_states = [&]() {  // wave w reads the records of wave w of the shares before
        for (int i = 0; i < npeers; ++i) {
            const uint32_t rec = (uint32_t)(((m - 1 - i) * kWaves + wave) * REC * 4);
#pragma unroll
            for (int r = 0; r < (G * 128 * 4 + 1023) / 1024; ++r) {
                const uint32_t o = (uint32_t)(r * 1024 + lane * 16);
                load_to_lds16_coherent(prs, o < (uint32_t)(G * 512) ? rec + o : 0xfffffff0u,
                                       (uint32_t)__builtin_amdgcn_readfirstlane((int)(uintptr_t)&s.peer_acc[i][wave][r * 256]));
            }
            load_to_lds4_coherent(prs, lane < 2 * G ? rec + G * 512 + lane * 4 : 0xfffffff0u,
                                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(uintptr_t)&s.peer_ml[i][wave][0]));
        }
    };
    auto peers_ready = [&]() {  // every flag this wave loaded is set
        const int f = lane < npeers ? s.flags[wave][lane] : 1;
        return __builtin_amdgcn_ballot_w64(f != 1) == 0;
    };

    // ---- the stream ------------------------------------------------------------------------
    float mx = kEmpty, l = 0.f;
    f32x4_t acc[8];
#pragma unroll
    for (int db = 0; db < 8; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int t_pub = publisher ? (rl(ven, 0) - 1) / kStageKeys : -1;
    // fused: the wave's next new key to place in the ring (segment ins_k, stream position
    // ins_pos); the segments holding a request's last key, in stream order
    int ins_k = -1, ins_pos = INT_MAX;
    auto next_insert = [&](int from) {
        ins_pos = INT_MAX;
        for (int k = from; k < nseg; ++k)
            if (rl(vinf, k) & kLast) {
                ins_k = k;
                ins_pos = rl(ven, k) - 1;
                break;
            }
    };
    if constexpr (FUSED) next_insert(0);
    // The memory operations besides the ring's loads go out after a stage's wait, and the next
    // stage's wait leaves them in flight (wait_slack); they have completed by the wait after
    // that.  So the flag of a published state is stored two stages after the state, and a
    // merging share reads the next shares' flags four stages before its stream ends, checks
    // them two stages later and reads their states then, in time for its last stage.
    const int t_flags = merging ? total - 4 : -1;
    const int t_flag_store = publisher ? t_pub + 2 : -1;
    bool have_peers = false;
    int slack = 0;  // operations the previous iteration issued after its wait
    const uint32_t flag_off = (uint32_t)((m * kWaves + wave) * 4);
    for (int t = 0; t < total; ++t) {
        // the next stage, into the slot scored last (the first two went out before the loop)
        if (issued < total && issued <= t + 1) {
            issue(issued);
            ++issued;
        }
        if (issued - 1 - t == 0) wait_loads<0>();  // this stage has landed (the next stays in flight)
        else wait_slack<KL>(slack);
        int extra = 0;
        if constexpr (FUSED) {
            if (t == 0) {
                // the step's keys and values into the arena, each segment's by the wave that
                // rotated them (lane group 0 stores, the others' offsets store nothing)
#pragma unroll
                for (int k = 0; k < kSlots; ++k) {
                    if (k >= nseg || wave != k % kWaves || !(rl(vinf, k) & kLast)) continue;
                    const uint32_t hk = lds_head + k * 8 * kRow;
                    const uint32_t row = (uint32_t)((int64_t)rl(vb, k) * p.k_sb * 2) + (uint32_t)((rl(vj1, k) - 1) * kst);
                    const uint32_t off = g == 0 ? row + c * 16 : 0xfffffff0u;
                    store16_asm(krs, off, lds_read16(hk + 6 * kRow + c * 16));
                    store16_asm(vrs, off, lds_read16(hk + 7 * kRow + c * 16));
                    extra += 2;
                }
            }
        }
        if (t == t_flag_store) {
            // the state stores of two stages ago have completed (the wait above covered them)
            store4_asm_coherent(frs, lane == 0 ? flag_off : 0xfffffff0u, 1);
            extra += 1;
        }
        if (t == t_flags) {
            load_peer_flags();
            extra += 1;
        }
        if (t == t_flags + 2 && t_flags >= 0 && peers_ready()) {
            load_peer_states();
            extra += npeers * ((G * 512 + 1023) / 1024 + 1);
            have_peers = true;
        }
        const uint32_t sbase = lds_ring + (t & 1) * kStageBytes + wave * kWaveStage;
        const int qbase = t * kStageKeys + wave * kWaveKeys;
        if constexpr (FUSED) {
            // a segment's new key and value enter the ring at its last stream position (the
            // loads left that row zero)
            while (ins_pos < qbase + kWaveKeys) {
                const int r = ins_pos - qbase;
                if (r >= 0 && g == 0) {
                    const uint32_t hk = lds_head + ins_k * 8 * kRow;
                    lds_write16(sbase + r * kRow + ((c ^ r) & 15) * 16, lds_read16(hk + 6 * kRow + c * 16));
                    lds_write16(sbase + kWaveKeys * kRow + r * kRow + ((c ^ (2 * r)) & 15) * 16,
                                lds_read16(hk + 7 * kRow + c * 16));
                }
                next_insert(ins_k + 1);
            }
        }

        // scores of the wave's 16 keys (rows of S^T) for the 16 columns
        f32x4_t st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(lds_read16(sbase + ka[kk])), qB[kk], st, 0, 0, 0);
        const int q0 = qbase + 4 * g;
        float x[4];
        if constexpr (MASK) {
            const U4 w4 = lds_read16(lds_mask + ((t & 1) * kWaves + wave) * 256 + 16 * g);
            const uint32_t wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = q0 + i;
                const int64_t elem = (int64_t)cb * p.m_sb + (cj0 + q - lo);
                const uint32_t sub = (uint32_t)(elem * mes) & 3u;
                x[i] = (q >= lo && q < hi) ? st[i] * scale + mask_term(wv[i], sub, p.mask_dtype) : -INFINITY;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = (q0 + i >= lo && q0 + i < hi) ? st[i] * scale : -INFINITY;
        }
        float mb = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        mb = fmaxf(mb, xor16(mb));
        mb = fmaxf(mb, xor32(mb));
        const bool up = mb > mx + kRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(up)) {
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
            acc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, lds_read_tr16(sbase + va[db])),
                                                               pb, acc[db], 0, 0, 0);
        if (t == t_pub) {
            // the first segment continues a request and ends in this stage: its columns are
            // final; this wave's state goes out now (lanes of the G columns) and its flag two
            // stages later
            float lt = l + xor16(l);
            lt += xor32(lt);
            const uint32_t rec = (uint32_t)((m * kWaves + wave) * REC * 4);
#pragma unroll
            for (int db = 0; db < 8; ++db)
                store16_asm_coherent(prs, c < G ? rec + (c * 128 + 16 * db + 4 * g) * 4 : 0xfffffff0u,
                                     U4{__float_as_uint(acc[db][0]), __float_as_uint(acc[db][1]),
                                        __float_as_uint(acc[db][2]), __float_as_uint(acc[db][3])});
            store8_asm_coherent(prs, c < G && g == 0 ? rec + G * 512 + c * 8 : 0xfffffff0u, mx, lt);
            extra += 9;
        }
        slack = extra;
    }
    wait_loads<0>();
    if (publisher && t_flag_store >= total)  // the state went out in one of the last two stages
        store4_asm_coherent(frs, lane == 0 ? flag_off : 0xfffffff0u, 1);

    // a merging share whose peers' states did not come with the stream: wait for their flags
    bool failed = false;
    if (merging && !have_peers) {
        for (int i = 0; i < npeers; ++i) {
            int v = 0, tries = 0;
            for (;; ++tries) {
                if (lane == 0)
                    v = __hip_atomic_load(p.counters + ((int64_t)h * M + m - 1 - i) * kWaves + wave, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
                if (__builtin_amdgcn_readfirstlane(v) == 1) break;
                if (tries >= kSpinLimit) {
                    failed = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        load_peer_states();
        wait_loads<0>();
    }

    // ---- the merge: every wave's columns and the published parts, four dims per thread -----
    // One barrier: the waves' (max, sum, accumulator) states go to LDS as they are, and each
    // thread combines four dims of one output row with the weights of the waves (and of the
    // earlier parts' waves, for the merged request) computed from the column's (max, sum)s.
    {
        float lt = l + xor16(l);
        lt += xor32(lt);
        if (g == 0) {
            s.ml[wave][c][0] = mx;
            s.ml[wave][c][1] = lt;
        }
        if (lane == 0) s.fail[wave] = failed ? 1 : 0;
#pragma unroll
        for (int db = 0; db < 8; ++db) *reinterpret_cast<f32x4_t *>(&s.acc[wave][c][16 * db + 4 * g]) = acc[db];
    }
    lds_barrier();
    const bool merge_failed = (s.fail[0] | s.fail[1] | s.fail[2] | s.fail[3]) != 0;
    const bool vec_out8 = ((reinterpret_cast<uintptr_t>(p.out) | (uintptr_t)(p.o_sb * 2) | (uintptr_t)(p.o_sh * 2)) & 7) == 0;
    for (int e4 = tid; e4 < nseg * G * 32; e4 += kThreads) {
        const int k = e4 / (G * 32), r = (e4 / 32) % G, d = (e4 & 31) * 4, col = k * G + r;
        if (!((out_mask >> k) & 1)) continue;
        const bool with_peers = merging && k == mk;
        float m4[kWaves], l4[kWaves];
        float mm = kEmpty;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            m4[w] = s.ml[w][col][0];
            l4[w] = s.ml[w][col][1];
            mm = fmaxf(mm, m4[w]);
        }
        if (with_peers)
            for (int i = 0; i < npeers; ++i)
#pragma unroll
                for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, s.peer_ml[i][w][2 * r]);
        f32x4_t sum = {0.f, 0.f, 0.f, 0.f};
        float sl = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float wt = fexp2(m4[w] - mm);
            sl += l4[w] * wt;
            sum += *reinterpret_cast<const f32x4_t *>(&s.acc[w][col][d]) * wt;
        }
        if (with_peers)
            for (int i = 0; i < npeers; ++i)
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float wt = fexp2(s.peer_ml[i][w][2 * r] - mm);
                    sl += s.peer_ml[i][w][2 * r + 1] * wt;
                    sum += *reinterpret_cast<const f32x4_t *>(&s.peer_acc[i][w][r * 128 + d]) * wt;
                }
        sum *= (with_peers && merge_failed) ? __builtin_nanf("") : __builtin_amdgcn_rcpf(sl);
        const uint32_t lo = cvt_pk_bf16_canon(sum[0], sum[1]), hi2 = cvt_pk_bf16_canon(sum[2], sum[3]);
        char *dst = p.out + ((int64_t)s.segb[k] * p.o_sb + (h * G + r) * p.o_sh + d) * 2;
        if (vec_out8) {
            *reinterpret_cast<uint2 *>(dst) = uint2{lo, hi2};
        } else {
            reinterpret_cast<uint16_t *>(dst)[0] = (uint16_t)lo;
            reinterpret_cast<uint16_t *>(dst)[1] = (uint16_t)(lo >> 16);
            reinterpret_cast<uint16_t *>(dst)[2] = (uint16_t)hi2;
            reinterpret_cast<uint16_t *>(dst)[3] = (uint16_t)(hi2 >> 16);
        }
    }
    write_zero_rows();
    // the flags this share consumed, cleared for the next launch on this workspace
    if (merging && lane < npeers)
        __hip_atomic_store(p.counters + ((int64_t)h * M + m - 1 - lane) * kWaves + wave, 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// ---- the plan: one launch per step, read by every layer ---------------------------------
// plan[(m * 8 + k) * 4 ...] = (b, j0, j1, info) for segment k of share m (b = -1: none), and
// after the M shares a header of 32 ints (batch, M, segment cap, ctx, four words of the bit
// mask of requests without a valid position, zeros), then the bundle section that the
// whole-request kernel of an unmasked launch reads: (batch, 0) and, for each of the M bundles,
// four (b, L_b) pairs ((-1, 0): none), every request of the batch in one of them.  L_b = pos[b] + 1 for a position
// in [0, ctx), else 0.
constexpr int kPlanThreads = kMaxBatch;

Q3T_DEVICE int inclusive_scan128(int x, int *part) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (lane == 63) part[w] = x;
    __syncthreads();
    return w ? x + part[0] : x;
}

__global__ void __launch_bounds__(kPlanThreads)
decode_shares_plan_kernel(const int64_t *pos, int B, int ctx, int M, int cap, int32_t *plan) {
    // the entries are built in LDS and stored once: two waves' stores to one global address
    // are not ordered by a workgroup barrier
    __shared__ int4 ent[kMaxBundles * kSlots];
    __shared__ int sL[kMaxBatch], pre[kMaxBatch + 1], ne[kMaxBatch + 1];
    __shared__ int first[kMaxBundles], count[kMaxBundles], cut[kMaxBundles];
    __shared__ __attribute__((aligned(16))) int keys[kMaxBatch];
    __shared__ int sorted_b[kMaxBatch], sorted_l[kMaxBatch];
    __shared__ int part[2][2];
    __shared__ int fallback;
    __shared__ uint32_t zmask[4];
    const int t = threadIdx.x;
    int L = 0;
    if (t < B) {
        const int64_t pb = pos[t];
        L = (pb >= 0 && pb < ctx) ? (int)pb + 1 : 0;
    }
    sL[t] = L;
    if (t < 4) zmask[t] = 0;
    if (t == 0) fallback = 0;
    for (int i = t; i < M; i += kPlanThreads) count[i] = 0;
    for (int i = t; i < M * kSlots; i += kPlanThreads) ent[i] = int4{-1, 0, 0, 0};
    const int incl = inclusive_scan128(L, part[0]);
    const int incl_ne = inclusive_scan128(L > 0 ? 1 : 0, part[1]);
    pre[t + 1] = incl;
    ne[t + 1] = incl_ne;
    if (t == 0) pre[0] = ne[0] = 0;
    keys[t] = t < B ? (L << 7) | (kMaxBatch - 1 - t) : -1;
    __syncthreads();
    if (t < B && L == 0) atomicOr(&zmask[t / 32], 1u << (t % 32));

    const int T = pre[B];
    const int TS = (T + kStageKeys - 1) / kStageKeys;
    const int q = TS / M, r = TS % M;
    auto start = [&](int mm) { return min(kStageKeys * (mm * q + min(mm, r)), T); };
    auto end = [&](int mm) { return mm == M - 1 ? T : min(kStageKeys * ((mm + 1) * q + min(mm + 1, r)), T); };
    auto share_of = [&](int x) {
        const int X = x / kStageKeys;
        int mm;
        if (X < r * (q + 1)) mm = X / (q + 1);
        else mm = q > 0 ? r + (X - r * (q + 1)) / q : M - 1;
        return min(mm, M - 1);
    };
    // the request holding each share's first key: the last b with pre[b] <= start
    for (int mm = t; mm < M; mm += kPlanThreads) {
        const int s0 = start(mm);
        int f = -1;
        if (s0 < end(mm)) {
            int a = 0, z = B - 1;
            while (a < z) {
                const int mid = (a + z + 1) >> 1;
                if (pre[mid] <= s0) a = mid;
                else z = mid - 1;
            }
            f = a;
        }
        first[mm] = f;
        // the share starts inside a request (bit 0) / ends inside one (bit 1)
        int k = 0;
        if (f >= 0) {
            if (pre[f] < s0) k |= 1;
            const int e0 = end(mm) - 1;
            int a = f, z = B - 1;
            while (a < z) {
                const int mid = (a + z + 1) >> 1;
                if (pre[mid] <= e0) a = mid;
                else z = mid - 1;
            }
            if (pre[a + 1] > end(mm)) k |= 2;
        }
        cut[mm] = k;
    }
    int m0 = 0, m1 = -1, P = 0;
    if (t < B && L > 0) {
        P = pre[t];
        m0 = share_of(P);
        m1 = share_of(P + L - 1);
        if (m1 - m0 > kPeers) atomicOr(&fallback, 1);
        for (int mm = m0; mm <= m1; ++mm) atomicAdd(&count[mm], 1);
    }
    __syncthreads();
    for (int mm = t; mm < M; mm += kPlanThreads)
        if (count[mm] > cap) atomicOr(&fallback, 1);
    __syncthreads();
    if (!fallback) {
        if (t < B && L > 0) {
            for (int mm = m0; mm <= m1; ++mm) {
                // processing order in the share: the part of the request it cuts first (published
                // early), its whole requests, the continued request's last part last (merged at
                // the end with the parts published long before)
                const int n = count[mm], ri = mm == m0 ? ne[t] - ne[first[mm]] : 0;
                const bool cont = cut[mm] & 1, head = cut[mm] & 2;
                int slot = ri + (head ? 1 : 0) - (cont ? 1 : 0);
                if (head && ri == n - 1) slot = 0;
                if (cont && ri == 0) slot = n - 1;
                if (n == 1) slot = 0;
                const int j0 = max(start(mm) - P, 0), j1 = min(end(mm) - P, L);
                int info = j1 == L ? kLast : 0;
                if (m1 > m0) info |= j1 == L ? kMerge | ((m1 - m0) << kPeerShift) : kPublish;
                if (slot >= 0 && slot < kSlots) ent[mm * kSlots + slot] = int4{t, j0, j1, info};
            }
        }
    }
    if (t < B) {
        // whole requests ranked by length (longest first, ties by index); without a cut, share
        // m takes ranks m, 2M-1-m, 2M+m, 4M-1-m
        const int key = keys[t];
        int rank = 0;
        for (int j = 0; j < B; j += 4) {
            const int4 k4 = *reinterpret_cast<const int4 *>(&keys[j]);  // keys past B are -1
            rank += (k4.x > key) + (k4.y > key) + (k4.z > key) + (k4.w > key);
        }
        sorted_b[rank] = t;
        sorted_l[rank] = L;
        if (fallback && L > 0) {
            const int round = rank / M, within = rank % M;
            const int mm = (round & 1) ? M - 1 - within : within;
            if (round < 4 && round < kSlots) ent[mm * kSlots + round] = int4{t, 0, L, kLast};
        }
    }
    __syncthreads();
    int4 *entries = reinterpret_cast<int4 *>(plan);
    for (int i = t; i < M * kSlots; i += kPlanThreads) entries[i] = ent[i];
    // whole requests: bundle m takes ranks m, 2M-1-m, 2M+m, 4M-1-m (longest with shortest)
    int2 *bundles = reinterpret_cast<int2 *>(plan + (M + 1) * kSlots * 4);
    for (int i = t; i < M * 4; i += kPlanThreads) {
        const int mm = i / 4, k = i % 4;
        const int r = (k >> 1) * 2 * M + ((k & 1) ? 2 * M - 1 - mm : mm);
        bundles[1 + i] = r < B ? int2{sorted_b[r], sorted_l[r]} : int2{-1, 0};
    }
    if (t == 0) {
        bundles[0] = int2{B, 0};
        int32_t *hd = plan + M * kSlots * 4;
        hd[0] = B;
        hd[1] = M;
        hd[2] = cap;
        hd[3] = ctx;
        for (int i = 0; i < 4; ++i) hd[4 + i] = (int32_t)zmask[i];
        for (int i = 8; i < kSlots * 4; ++i) hd[i] = 0;
    }
}

template <int G, bool F, bool N, bool MK>
static void launch(const DecodeParams &p, hipStream_t s) {
    const dim3 grid((uint32_t)p.bundles * p.Hkv);
    if (p.stream)
        hipLaunchKernelGGL((decode_shares_kernel<G, F, true, N, MK>), grid, dim3(kThreads), 0, s, p.plan, p.B, p.Hkv,
                           p.bundles, p);
    else
        hipLaunchKernelGGL((decode_shares_kernel<G, F, false, N, MK>), grid, dim3(kThreads), 0, s, p.plan, p.B, p.Hkv,
                           p.bundles, p);
}

template <int G>
static void launch_g(const DecodeParams &p, bool fused, bool norm, bool mask, hipStream_t s) {
    if (fused) {
        if (norm) {
            if (mask) launch<G, true, true, true>(p, s);
            else launch<G, true, true, false>(p, s);
        } else {
            if (mask) launch<G, true, false, true>(p, s);
            else launch<G, true, false, false>(p, s);
        }
    } else {
        if (mask) launch<G, false, false, true>(p, s);
        else launch<G, false, false, false>(p, s);
    }
}

}  // namespace shares

// Entry points used by decode_attention.hip.
int64_t shares_bundle_count(int64_t batch, int64_t kv_heads) { return shares::bundle_count(batch, kv_heads); }
int shares_slot_cap(int64_t group) { return shares::slot_cap(group); }
int64_t shares_rank_offset(int64_t batch, int64_t kv_heads) {
    return (shares::bundle_count(batch, kv_heads) + 1) * shares::kSlots * 4;
}
int64_t shares_plan_ints(int64_t batch, int64_t kv_heads) {
    return shares_rank_offset(batch, kv_heads) + 2 + 8 * shares::bundle_count(batch, kv_heads);
}
int64_t shares_partial_floats(int64_t batch, int64_t kv_heads, int64_t group) {
    return kv_heads * shares::bundle_count(batch, kv_heads) * shares::kWaves * (group * 128 + 8);
}
int64_t shares_flag_count(int64_t batch, int64_t kv_heads) {
    return kv_heads * shares::bundle_count(batch, kv_heads) * shares::kWaves;
}
int shares_launch(const DecodeParams &p, int group, bool fused, bool norm, bool mask, hipStream_t s) {
    switch (group) {  // the caller reads the launch status
        case 1: shares::launch_g<1>(p, fused, norm, mask, s); return Q3T_OK;
        case 2: shares::launch_g<2>(p, fused, norm, mask, s); return Q3T_OK;
        case 4: shares::launch_g<4>(p, fused, norm, mask, s); return Q3T_OK;
        default: return Q3T_EUNSUPPORTED;
    }
}
int shares_plan_launch(const int64_t *pos, int batch, int ctx, int bundles, int cap, int32_t *plan, hipStream_t s) {
    hipLaunchKernelGGL(shares::decode_shares_plan_kernel, dim3(1), dim3(shares::kPlanThreads), 0, s, pos, batch, ctx,
                       bundles, cap, plan);
    return launch_status();
}

}  // namespace q3t
