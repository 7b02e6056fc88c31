// Rotary position embedding kernels.
//
// q3t_rotary      - exact bf16 rotate-half RoPE on BSND rows (reference:
//                   rotary_triton_ascend.py:8-44; torch eager apply_rotary_pos_emb).
// q3t_rope_tables - default-RoPE cos/sin rows for integer positions (reference: the
//                   talker rotary_emb called at continuous.py:193 / prefill_graph.py:38).
#include "q3t_common.hpp"

namespace q3t {

// One work item = 8 dims of the first half and the matching 8 dims of the second half
// of one (row, head): two 16-byte loads of x, four of cos/sin, two 16-byte stores.
__global__ void __launch_bounds__(256)
rotary_bf16_kernel(const uint16_t *__restrict__ x, const uint16_t *__restrict__ cosv,
                   const uint16_t *__restrict__ sinv, uint16_t *__restrict__ y, int64_t rows,
                   int heads, int width) {
    const int half = width >> 1;
    const int vecs = half >> 3;  // 16-byte vectors per half
    const int64_t total = rows * heads * vecs;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % vecs);
        const int64_t rh = i / vecs;
        const int64_t row = rh / heads;
        const int64_t xo = rh * width + c * 8;
        const int64_t co = row * width + c * 8;
        U4 x1 = load16(x + xo), x2 = load16(x + xo + half);
        U4 c1 = load16(cosv + co), c2 = load16(cosv + co + half);
        U4 s1 = load16(sinv + co), s2 = load16(sinv + co + half);
        U4 y1, y2;
        rope8(&x1.x, &x2.x, &c1.x, &c2.x, &s1.x, &s2.x, &y1.x, &y2.x);
        store16(y + xo, y1);
        store16(y + xo + half, y2);
    }
}

// fp32 rows: torch-eager fp32 semantics, every product and the sum rounded separately
// (no fused multiply-add): y1 = x1*c1 + (-x2*s1), y2 = x2*c2 + x1*s2.
__global__ void __launch_bounds__(256)
rotary_f32_kernel(const float *__restrict__ x, const float *__restrict__ cosv,
                  const float *__restrict__ sinv, float *__restrict__ y, int64_t rows, int heads,
                  int width) {
#pragma clang fp contract(off)
    const int half = width >> 1;
    const int64_t total = rows * heads * half;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int d = (int)(i % half);
        const int64_t rh = i / half;
        const int64_t row = rh / heads;
        const float x1 = x[rh * width + d], x2 = x[rh * width + d + half];
        const float c1 = cosv[row * width + d], c2 = cosv[row * width + d + half];
        const float s1 = sinv[row * width + d], s2 = sinv[row * width + d + half];
        const float a = x1 * c1, b = -(x2 * s1), c = x2 * c2, e = x1 * s2;
        y[rh * width + d] = a + b;
        y[rh * width + d + half] = c + e;
    }
}

template <typename OutT>
__global__ void __launch_bounds__(256)
rope_tables_kernel(const int64_t *__restrict__ positions, int64_t n,
                   const float *__restrict__ inv_freq, int half, float scaling,
                   OutT *__restrict__ cosv, OutT *__restrict__ sinv) {
    const int64_t total = n * half;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int f = (int)(i % half);
        const int64_t r = i / half;
        // fp32 product as the reference's (inv_freq @ position) with a K=1 contraction.
        const float angle = inv_freq[f] * (float)positions[r];
        const float cf = cosf(angle) * scaling, sf = sinf(angle) * scaling;
        OutT c, s;
        if constexpr (sizeof(OutT) == 2) {
            c = (OutT)float_to_bf16(cf);
            s = (OutT)float_to_bf16(sf);
        } else {
            c = cf;
            s = sf;
        }
        const int64_t o = r * 2 * half + f;
        cosv[o] = c;
        cosv[o + half] = c;
        sinv[o] = s;
        sinv[o + half] = s;
    }
}

}  // namespace q3t

using namespace q3t;

extern "C" int q3t_rotary(const void *x, const void *cos, const void *sin, void *y, int64_t rows,
                          int64_t heads, int64_t width, int64_t dtype, void *stream) {
    if (!x || !cos || !sin || !y || rows < 0 || heads < 1) return Q3T_EINVAL;
    if (width != 64 && width != 128) return Q3T_EUNSUPPORTED;
    if (dtype != Q3T_BF16 && dtype != Q3T_F32) return Q3T_EUNSUPPORTED;
    if (!aligned(x, 16) || !aligned(cos, 16) || !aligned(sin, 16) || !aligned(y, 16))
        return Q3T_EINVAL;
    if (rows == 0) return Q3T_OK;
    const int64_t total = dtype == Q3T_BF16 ? rows * heads * (width / 16) : rows * heads * (width / 2);
    int64_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    if (dtype == Q3T_BF16)
        hipLaunchKernelGGL(rotary_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t *)x, (const uint16_t *)cos, (const uint16_t *)sin,
                           (uint16_t *)y, rows, (int)heads, (int)width);
    else
        hipLaunchKernelGGL(rotary_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const float *)x, (const float *)cos, (const float *)sin, (float *)y,
                           rows, (int)heads, (int)width);
    return launch_status();
}

extern "C" int q3t_rope_tables(const int64_t *positions, int64_t n, const float *inv_freq,
                               int64_t half, float scaling, int64_t dtype, void *cos, void *sin,
                               void *stream) {
    if (!positions || !inv_freq || !cos || !sin || n < 0 || half < 1 || half > 4096)
        return Q3T_EINVAL;
    if (dtype != Q3T_BF16 && dtype != Q3T_F32) return Q3T_EUNSUPPORTED;
    if (n == 0) return Q3T_OK;
    const int64_t total = n * half;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    if (dtype == Q3T_BF16)
        hipLaunchKernelGGL(rope_tables_kernel<uint16_t>, dim3((unsigned)blocks), dim3(256), 0,
                           (hipStream_t)stream, positions, n, inv_freq, (int)half, scaling,
                           (uint16_t *)cos, (uint16_t *)sin);
    else
        hipLaunchKernelGGL(rope_tables_kernel<float>, dim3((unsigned)blocks), dim3(256), 0,
                           (hipStream_t)stream, positions, n, inv_freq, (int)half, scaling,
                           (float *)cos, (float *)sin);
    return launch_status();
}
