// Shared device helpers for the gfx950 kernels: bf16 bit conversions with torch's
// rounding, DPP lane reductions and 16-byte vector access.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qwen3tts_amd.h"

#define Q3T_DEVICE __device__ __forceinline__

namespace q3t {

struct alignas(16) U4 { uint32_t x, y, z, w; };

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// bf16 (as raw 16 bits) -> fp32: exact.
Q3T_DEVICE float bf16_to_float(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
Q3T_DEVICE float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
Q3T_DEVICE float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 (lo, hi), round-to-nearest-even, by gfx950's v_cvt_pk_bf16_f32.
// For every non-NaN input this equals torch's integer rule bf16 = (u + 0x7fff + lsb) >> 16.
Q3T_DEVICE uint32_t cvt_pk_bf16(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
// Same, with NaN mapped to 0x7fc0 as c10::BFloat16 does.
Q3T_DEVICE uint32_t cvt_pk_bf16_canon(float lo, float hi) {
    uint32_t r = cvt_pk_bf16(lo, hi);
    if (lo != lo) r = (r & 0xffff0000u) | 0x7fc0u;
    if (hi != hi) r = (r & 0x0000ffffu) | 0x7fc00000u;
    return r;
}
// fp32 -> bf16 bits (canonical NaN), for single values.
Q3T_DEVICE uint32_t float_to_bf16(float f) { return cvt_pk_bf16_canon(f, 0.f) & 0xffffu; }
// Round through bf16 and back (one torch-eager bf16 op boundary).
Q3T_DEVICE float round_bf16(float f) { return bf16_to_float(float_to_bf16(f)); }

Q3T_DEVICE uint32_t pack_bf16(float lo, float hi) { return cvt_pk_bf16_canon(lo, hi); }

// a.lo*b.lo + a.hi*b.hi + c on packed bf16 pairs (v_dot2c_f32_bf16).
Q3T_DEVICE float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

Q3T_DEVICE float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane exchanges within rows of 16 lanes.
template <int CTRL>
Q3T_DEVICE float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8-lane half row

// Sum over each aligned group of 8 lanes; every lane of the group receives the total.
Q3T_DEVICE float sum8(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    return x;
}

// Value of the lane whose index differs in bit 3 / 4 / 5, without LDS traffic:
// DPP row_ror:8 inside each 16-lane row, then the gfx950 permlane16/32 swaps.
Q3T_DEVICE float xor8(float x) { return dpp<0x128>(x); }
Q3T_DEVICE float xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
Q3T_DEVICE float xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

Q3T_DEVICE uint32_t xor8u(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xf, 0xf, false);
}
// The 16-byte vector of the lane whose index differs in bit 3 (the other half of a 256-byte
// row spread over 16 lanes).
Q3T_DEVICE U4 xor8_u4(const U4 &v) {
    return U4{xor8u(v.x), xor8u(v.y), xor8u(v.z), xor8u(v.w)};
}

// A wave-uniform pointer moved to scalar registers.  readfirstlane is a 32-bit operation, so
// the two halves of the address go through it separately.
template <typename P>
Q3T_DEVICE P *uniform_ptr(P *ptr) {
    const uint64_t x = reinterpret_cast<uint64_t>(ptr);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
    return reinterpret_cast<P *>(((uint64_t)hi << 32) | lo);
}

// Buffer access through a wave-uniform resource: 32-bit byte offsets from the base, reads at
// or past `bytes` return zeros (the resource's range check).  0x00020000 is the gfx9-family
// descriptor word 3 for raw 32-bit dword data.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
Q3T_DEVICE __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
Q3T_DEVICE U4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(U4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// Streaming read: the cache-policy `nt` (non-temporal) bit, for data that this launch reads
// once and no later access will find in the caches.  On the talker arena's ragged K/V
// reads it measured 6-11% faster than the default policy at 8 to 128 requests.
constexpr int kPolicyNonTemporal = 2;
Q3T_DEVICE U4 buffer_load16_stream(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(U4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kPolicyNonTemporal));
}
Q3T_DEVICE void buffer_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, U4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, v), r, (int)off, 0, 0);
}

Q3T_DEVICE U4 load16(const void *p) { return *reinterpret_cast<const U4 *>(p); }
Q3T_DEVICE void store16(void *p, U4 v) { *reinterpret_cast<U4 *>(p) = v; }

// Rotate-half RoPE on one packed bf16 pair of the first half (x1) and the matching pair of
// the second half (x2), reproducing torch-eager bf16 rounding after every op
// (reference contract: rotary_triton_ascend.py:19-24):
//   y1 = bf16(bf16(x1*c1) + bf16(-x2*s1)),  y2 = bf16(bf16(x2*c2) + bf16(x1*s2)).
// Products of two bf16 values are exact in fp32; each sum rounds to fp32 and then to bf16,
// the same double rounding torch performs for a bf16 add.
// CANON = false leaves NaN payloads as the conversion produces them (for rotated values that
// are consumed in registers and never stored).
template <bool CANON = true>
Q3T_DEVICE void rope_pair(uint32_t x1, uint32_t x2, uint32_t c1, uint32_t c2, uint32_t s1,
                          uint32_t s2, uint32_t &y1, uint32_t &y2) {
    const float a0 = bf16_lo(x1), a1 = bf16_hi(x1), b0 = bf16_lo(x2), b1 = bf16_hi(x2);
    // intermediate roundings: a NaN only has to stay a NaN, its bits are canonicalised at the end
    const uint32_t l1 = cvt_pk_bf16(a0 * bf16_lo(c1), a1 * bf16_hi(c1));
    const uint32_t r1 = cvt_pk_bf16(-(b0 * bf16_lo(s1)), -(b1 * bf16_hi(s1)));
    y1 = CANON ? cvt_pk_bf16_canon(bf16_lo(l1) + bf16_lo(r1), bf16_hi(l1) + bf16_hi(r1))
               : cvt_pk_bf16(bf16_lo(l1) + bf16_lo(r1), bf16_hi(l1) + bf16_hi(r1));
    const uint32_t l2 = cvt_pk_bf16(b0 * bf16_lo(c2), b1 * bf16_hi(c2));
    const uint32_t r2 = cvt_pk_bf16(a0 * bf16_lo(s2), a1 * bf16_hi(s2));
    y2 = CANON ? cvt_pk_bf16_canon(bf16_lo(l2) + bf16_lo(r2), bf16_hi(l2) + bf16_hi(r2))
               : cvt_pk_bf16(bf16_lo(l2) + bf16_lo(r2), bf16_hi(l2) + bf16_hi(r2));
}

// RoPE on 8 consecutive dims of each half (one 16-byte vector per half).
template <bool CANON = true>
Q3T_DEVICE void rope8(const uint32_t *x1, const uint32_t *x2, const uint32_t *c1, const uint32_t *c2,
                      const uint32_t *s1, const uint32_t *s2, uint32_t *y1, uint32_t *y2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) rope_pair<CANON>(x1[i], x2[i], c1[i], c2[i], s1[i], s2[i], y1[i], y2[i]);
}

// RoPE of one 16-byte vector (8 dims) of a row, as rope_pair computes it: `own` holds the
// lane's dims of one half, `partner` the same dims of the other half, c/s the cos/sin values
// at own's dims.  First half: bf16(bf16(own*c) + bf16(-(partner*s))); second half:
// bf16(bf16(own*c) + bf16(partner*s)).
Q3T_DEVICE U4 rope_half8(U4 own, U4 partner, U4 c, U4 s, bool first) {
    const uint32_t o[4] = {own.x, own.y, own.z, own.w}, q[4] = {partner.x, partner.y, partner.z, partner.w};
    const uint32_t cc[4] = {c.x, c.y, c.z, c.w}, ss[4] = {s.x, s.y, s.z, s.w};
    const uint32_t sign = first ? 0x80000000u : 0u;
    uint32_t y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = cvt_pk_bf16(bf16_lo(o[i]) * bf16_lo(cc[i]), bf16_hi(o[i]) * bf16_hi(cc[i]));
        const uint32_t b = cvt_pk_bf16(__uint_as_float(__float_as_uint(bf16_lo(q[i]) * bf16_lo(ss[i])) ^ sign),
                                       __uint_as_float(__float_as_uint(bf16_hi(q[i]) * bf16_hi(ss[i])) ^ sign));
        y[i] = cvt_pk_bf16_canon(bf16_lo(a) + bf16_lo(b), bf16_hi(a) + bf16_hi(b));
    }
    return U4{y[0], y[1], y[2], y[3]};
}

inline bool aligned(const void *p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? Q3T_OK : static_cast<int>(e);
}

// ---- MFMA operands and global-to-LDS loads -------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

Q3T_DEVICE bf16x8_t as_bf16x8(const U4 &v) { return __builtin_bit_cast(bf16x8_t, v); }

// 8 bytes of LDS per lane, transposed across each 16-lane group as 16-bit elements.
Q3T_DEVICE uint2 lds_read_tr16(uint32_t byte_addr) {
    const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t *)(uintptr_t)byte_addr);
    return __builtin_bit_cast(uint2, r);
}
Q3T_DEVICE void lds_write16(uint32_t byte_addr, const U4 &v) {
    *(__attribute__((address_space(3))) i32x4_t *)(uintptr_t)byte_addr = __builtin_bit_cast(i32x4_t, v);
}
Q3T_DEVICE U4 lds_read16(uint32_t byte_addr) {
    const i32x4_t v = *(__attribute__((address_space(3))) const i32x4_t *)(uintptr_t)byte_addr;
    return __builtin_bit_cast(U4, v);
}

// A buffer resource in scalar registers (for inline assembly): base, 32-bit range, raw dwords.
Q3T_DEVICE i32x4_t scalar_rsrc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4_t r;
    r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
    r.z = __builtin_amdgcn_readfirstlane((int)bytes);
    r.w = 0x00020000;
    return r;
}
// 16 bytes per lane from global memory straight into LDS at lds_base + 16 * lane (the wave's
// lanes fill one contiguous 1 KiB run); offsets past the resource's range write zeros.  The
// load is issued from inline assembly so that the compiler does not insert a wait for it in
// front of unrelated LDS reads; completion is awaited explicitly with wait_loads.
// Every memory instruction issued from inline assembly is preceded by five wait states
// (Q3T_VMEM_SGPR_WAIT): a VMEM instruction reading an SGPR that a VALU instruction wrote
// (v_readlane / v_readfirstlane, which is how the compiler reloads spilled or lane-derived
// resource words) needs them, the compiler does not insert them in front of inline assembly,
// and without them the instruction can read a stale resource word: a store then lands nowhere
// (out of range) and a load fills LDS with zeros.  The s_mov to m0 counts as one of them.
#define Q3T_VMEM_SGPR_WAIT "s_nop 4\n\t"
Q3T_DEVICE void load_to_lds16(i32x4_t rsrc, uint32_t voffset, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\t" Q3T_VMEM_SGPR_WAIT "buffer_load_dwordx4 %1, %2, 0 offen lds"
                 :: "s"(lds_base), "v"(voffset), "s"(rsrc) : "memory", "m0");
}
// The same with the non-temporal cache policy, for rows a launch reads once.
Q3T_DEVICE void load_to_lds16_stream(i32x4_t rsrc, uint32_t voffset, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\t" Q3T_VMEM_SGPR_WAIT "buffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :: "s"(lds_base), "v"(voffset), "s"(rsrc) : "memory", "m0");
}
// Touch every 64-byte line of the kernel's argument segment (BYTES long) at once, so that the
// scalar loads the compiler issues later, near each argument's first use, hit the scalar cache
// instead of paying one memory round trip each: a fresh launch finds none of its arguments
// cached, and a chain of such misses delayed the first loads of the decode kernel by ~1.5 us.
// The loads are issued together and awaited inside one asm statement (the compiler, left to
// itself, split them into two waits).
template <int BYTES>
Q3T_DEVICE void prefetch_kernargs() {
    static_assert(BYTES <= 8 * 64, "eight 64-byte lines at most");
    const uint64_t a = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
    uint32_t d0, d1, d2, d3, d4, d5, d6, d7;
    asm volatile("s_load_dword %0, %8, 0x0\n\t"
                 "s_load_dword %1, %8, 0x40\n\t"
                 "s_load_dword %2, %8, 0x80\n\t"
                 "s_load_dword %3, %8, 0xc0\n\t"
                 "s_load_dword %4, %8, %9\n\t"
                 "s_load_dword %5, %8, %10\n\t"
                 "s_load_dword %6, %8, %11\n\t"
                 "s_load_dword %7, %8, %12\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7)
                 : "s"(a), "n"(BYTES > 0x100 ? 0x100 : 0), "n"(BYTES > 0x140 ? 0x140 : 0),
                   "n"(BYTES > 0x180 ? 0x180 : 0), "n"(BYTES > 0x1c0 ? 0x1c0 : 0)
                 : "memory");
}
template <int N>
Q3T_DEVICE void wait_loads() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }
// Workgroup barrier after the wave's own LDS reads have returned.
Q3T_DEVICE void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace q3t
