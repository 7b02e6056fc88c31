// KV arena writes and strided copies: the byte-moving part of the slot arena.
//
// q3t_kv_write    - paired single/multi-token K/V write at per-request positions
//                   (reference: continuous.py:152-166, kv_triton_ascend.py:24-64,
//                    predictor.py:19-24).
// q3t_copy_strided - up-to-5-D strided copy used for the packed prefix copy, slot
//                   compaction and arena regrowth (packed_kv.py:6-31,
//                   continuous.py:118-128, 353-363).
// q3t_copy_bytes  - contiguous copy; also the calibration kernel for HBM counters.
//
// All three are HBM-bound byte moves: one work item moves one 16-byte vector when the
// row, pointers and strides allow it, else the widest power-of-two unit that divides them.
#include "q3t_common.hpp"

namespace q3t {

template <int V> struct Vec;
template <> struct Vec<16> { typedef U4 T; };
template <> struct Vec<8> { typedef uint2 T; };
template <> struct Vec<4> { typedef uint32_t T; };
template <> struct Vec<2> { typedef uint16_t T; };
template <> struct Vec<1> { typedef uint8_t T; };

struct KvWriteParams {
    const char *k, *v;
    char *tk, *tv;
    const int64_t *positions;
    int64_t heads, tokens, chunks;   // chunks of V bytes per row
    int64_t total;                   // batch*heads*tokens*chunks
    int64_t ks_b, ks_h, ks_t;        // source strides in bytes
    int64_t vs_b, vs_h, vs_t;
    int64_t ts_b, ts_h, ts_s;        // target strides in bytes
    int64_t capacity;
};

template <int V>
__global__ void __launch_bounds__(256) kv_write_kernel(KvWriteParams p) {
    typedef typename Vec<V>::T T;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < p.total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t c = i % p.chunks;
        int64_t r = i / p.chunks;
        int64_t t = r % p.tokens;
        r /= p.tokens;
        int64_t h = r % p.heads;
        int64_t b = r / p.heads;
        int64_t pos = p.positions[b] + t;
        if (pos < 0 || pos >= p.capacity) continue;
        int64_t off = c * V;
        T kval = *reinterpret_cast<const T *>(p.k + b * p.ks_b + h * p.ks_h + t * p.ks_t + off);
        T vval = *reinterpret_cast<const T *>(p.v + b * p.vs_b + h * p.vs_h + t * p.vs_t + off);
        int64_t dst = b * p.ts_b + h * p.ts_h + pos * p.ts_s + off;
        *reinterpret_cast<T *>(p.tk + dst) = kval;
        *reinterpret_cast<T *>(p.tv + dst) = vval;
    }
}

struct CopyParams {
    char *dst;
    const char *src;
    int64_t n[5];          // n[4] counts vectors of the innermost dimension
    int64_t ds[5], ss[5];  // byte strides; ds[4]/ss[4] step one vector
    int64_t total;
};

template <int V>
__global__ void __launch_bounds__(256) copy_strided_kernel(CopyParams p) {
    typedef typename Vec<V>::T T;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < p.total;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t rem = i, doff = 0, soff = 0;
#pragma unroll
        for (int d = 4; d >= 0; --d) {
            int64_t idx = rem % p.n[d];
            rem /= p.n[d];
            doff += idx * p.ds[d];
            soff += idx * p.ss[d];
        }
        *reinterpret_cast<T *>(p.dst + doff) = *reinterpret_cast<const T *>(p.src + soff);
    }
}

static int pick_vec(int64_t row_bytes, int64_t esize, std::initializer_list<int64_t> byte_strides,
                    std::initializer_list<const void *> ptrs) {
    // Widest power-of-two unit (>= one element) dividing the row, every stride and pointer.
    for (int64_t v = 16; v >= esize; v >>= 1) {
        if (row_bytes % v) continue;
        bool ok = true;
        for (int64_t s : byte_strides) ok = ok && (s % v == 0);
        for (const void *q : ptrs) ok = ok && aligned(q, v);
        if (ok) return (int)v;
    }
    return 0;
}

static unsigned grid_for(int64_t total) {
    int64_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;  // grid-stride beyond this
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

}  // namespace q3t

using namespace q3t;

extern "C" const char *q3t_status_string(int status) {
    switch (status) {
        case Q3T_OK: return "success";
        case Q3T_EINVAL: return "invalid argument";
        case Q3T_EUNSUPPORTED: return "unsupported shape or dtype";
        case Q3T_EWORKSPACE: return "workspace missing or too small";
        default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
    }
}

extern "C" int q3t_abi_version(void) { return 8; }

extern "C" int q3t_kv_write(const void *keys, const void *values, void *target_keys,
                            void *target_values, const int64_t *positions, int64_t batch,
                            int64_t heads, int64_t tokens, int64_t width, int64_t elem_size,
                            const int64_t key_strides[3], const int64_t value_strides[3],
                            const int64_t target_strides[3], int64_t capacity, void *stream) {
    if (!keys || !values || !target_keys || !target_values || !positions || !key_strides ||
        !value_strides || !target_strides)
        return Q3T_EINVAL;
    if (batch < 0 || heads < 1 || tokens < 1 || width < 1 || capacity < 1) return Q3T_EINVAL;
    if (elem_size != 1 && elem_size != 2 && elem_size != 4 && elem_size != 8) return Q3T_EINVAL;
    if (batch == 0) return Q3T_OK;
    KvWriteParams p;
    p.k = (const char *)keys;
    p.v = (const char *)values;
    p.tk = (char *)target_keys;
    p.tv = (char *)target_values;
    p.positions = positions;
    p.heads = heads;
    p.tokens = tokens;
    p.capacity = capacity;
    p.ks_b = key_strides[0] * elem_size; p.ks_h = key_strides[1] * elem_size; p.ks_t = key_strides[2] * elem_size;
    p.vs_b = value_strides[0] * elem_size; p.vs_h = value_strides[1] * elem_size; p.vs_t = value_strides[2] * elem_size;
    p.ts_b = target_strides[0] * elem_size; p.ts_h = target_strides[1] * elem_size; p.ts_s = target_strides[2] * elem_size;
    int64_t row = width * elem_size;
    int v = pick_vec(row, elem_size,
                     {p.ks_b, p.ks_h, p.ks_t, p.vs_b, p.vs_h, p.vs_t, p.ts_b, p.ts_h, p.ts_s},
                     {keys, values, target_keys, target_values});
    if (!v) return Q3T_EINVAL;
    p.chunks = row / v;
    p.total = batch * heads * tokens * p.chunks;
    hipStream_t s = (hipStream_t)stream;
    dim3 grid(grid_for(p.total)), block(256);
    switch (v) {
        case 16: hipLaunchKernelGGL(kv_write_kernel<16>, grid, block, 0, s, p); break;
        case 8: hipLaunchKernelGGL(kv_write_kernel<8>, grid, block, 0, s, p); break;
        case 4: hipLaunchKernelGGL(kv_write_kernel<4>, grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL(kv_write_kernel<2>, grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL(kv_write_kernel<1>, grid, block, 0, s, p); break;
    }
    return launch_status();
}

extern "C" int q3t_copy_strided(void *dst, const void *src, int64_t elem_size, int ndim,
                                const int64_t *sizes, const int64_t *dst_strides,
                                const int64_t *src_strides, void *stream) {
    if (!dst || !src || !sizes || !dst_strides || !src_strides) return Q3T_EINVAL;
    if (ndim < 1 || ndim > 5) return Q3T_EINVAL;
    if (elem_size != 1 && elem_size != 2 && elem_size != 4 && elem_size != 8) return Q3T_EINVAL;
    CopyParams p;
    p.dst = (char *)dst;
    p.src = (const char *)src;
    int lead = 5 - ndim;
    for (int d = 0; d < 5; ++d) {
        if (d < lead) {
            p.n[d] = 1; p.ds[d] = 0; p.ss[d] = 0;
        } else {
            int64_t n = sizes[d - lead];
            if (n < 0) return Q3T_EINVAL;
            if (n == 0) return Q3T_OK;
            p.n[d] = n;
            p.ds[d] = dst_strides[d - lead] * elem_size;
            p.ss[d] = src_strides[d - lead] * elem_size;
        }
    }
    int v = (int)elem_size;
    if (p.ds[4] == elem_size && p.ss[4] == elem_size) {
        int64_t row = p.n[4] * elem_size;
        int w = pick_vec(row, elem_size, {p.ds[0], p.ds[1], p.ds[2], p.ds[3], p.ss[0], p.ss[1], p.ss[2], p.ss[3]},
                         {dst, src});
        if (w > v) {
            v = w;
            p.n[4] = row / v;
            p.ds[4] = v;
            p.ss[4] = v;
        }
    }
    if (!aligned(dst, elem_size) || !aligned(src, elem_size)) return Q3T_EINVAL;
    p.total = p.n[0] * p.n[1] * p.n[2] * p.n[3] * p.n[4];
    hipStream_t s = (hipStream_t)stream;
    dim3 grid(grid_for(p.total)), block(256);
    switch (v) {
        case 16: hipLaunchKernelGGL(copy_strided_kernel<16>, grid, block, 0, s, p); break;
        case 8: hipLaunchKernelGGL(copy_strided_kernel<8>, grid, block, 0, s, p); break;
        case 4: hipLaunchKernelGGL(copy_strided_kernel<4>, grid, block, 0, s, p); break;
        case 2: hipLaunchKernelGGL(copy_strided_kernel<2>, grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL(copy_strided_kernel<1>, grid, block, 0, s, p); break;
    }
    return launch_status();
}

namespace q3t {
__global__ void __launch_bounds__(256) copy_bytes16_kernel(U4 *dst, const U4 *src, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}
}  // namespace q3t

extern "C" int q3t_copy_bytes(void *dst, const void *src, int64_t nbytes, void *stream) {
    if (!dst || !src || nbytes < 0) return Q3T_EINVAL;
    if (nbytes == 0) return Q3T_OK;
    if (nbytes % 16 == 0 && aligned(dst, 16) && aligned(src, 16)) {
        int64_t n = nbytes / 16;
        int64_t blocks = (n + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        hipLaunchKernelGGL(copy_bytes16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                           (hipStream_t)stream, (U4 *)dst, (const U4 *)src, n);
        return launch_status();
    }
    int64_t one = 1;
    return q3t_copy_strided(dst, src, 1, 1, &nbytes, &one, &one, stream);
}
