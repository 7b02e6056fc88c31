// The step plan of the bundled decode grid: which requests each workgroup (bundle) of a KV
// head attends, made once per step from the positions and read by every layer's launch (the
// talker's layers all attend the same lengths: SlotGraph.compute fixes the positions for a
// step, continuous.py:188-198).
//
// plan[0] = batch, plan[1] = M (bundles per KV head), then for bundle m = 0 ... M-1 four
// (b, L_b) pairs: the requests of length ranks m, 2M-1-m, 2M+m and 4M-1-m (longest first,
// ties by ascending index; (-1, 0) past the batch), so that the i-th longest request shares a
// workgroup with the i-th shortest.  L_b = pos[b] + 1 for a position in [0, ctx), else 0.
#include "decode_params.hpp"

namespace q3t {
namespace plan {

constexpr int kMaxBatch = 128;
constexpr int kGroups = 256;    // workgroups of a bundled launch: one per CU
constexpr int kPerBundle = 4;   // requests per bundle

// One workgroup, thread t for request t: its rank is the number of requests ranked before it
// (16-byte LDS reads of the keys L << 7 | (127 - b)); the bundles then read the ranks in order.
__global__ void __launch_bounds__(kMaxBatch) decode_plan_kernel(const int64_t *pos, int B, int ctx, int M, int32_t *plan) {
    __shared__ __attribute__((aligned(16))) int keys[kMaxBatch];
    __shared__ int sorted_b[kMaxBatch], sorted_l[kMaxBatch];
    const int t = threadIdx.x;
    int L = 0;
    if (t < B) {
        const int64_t pb = pos[t];
        L = (pb >= 0 && pb < ctx) ? (int)pb + 1 : 0;
    }
    // ctx <= 2^20 keeps L << 7 below 2^31; b < 128 fits the low 7 bits
    const int key = t < B ? (L << 7) | (kMaxBatch - 1 - t) : -1;
    keys[t] = key;
    __syncthreads();
    if (t < B) {
        int rank = 0;
        for (int j = 0; j < B; j += 4) {  // keys past B are -1
            const int4 k4 = *reinterpret_cast<const int4 *>(&keys[j]);
            rank += (k4.x > key) + (k4.y > key) + (k4.z > key) + (k4.w > key);
        }
        sorted_b[rank] = t;
        sorted_l[rank] = L;
    }
    __syncthreads();
    int2 *table = reinterpret_cast<int2 *>(plan + 2);
    for (int i = t; i < M * kPerBundle; i += kMaxBatch) {
        const int m = i / kPerBundle, k = i % kPerBundle;
        const int r = (k >> 1) * 2 * M + ((k & 1) ? 2 * M - 1 - m : m);
        table[i] = r < B ? int2{sorted_b[r], sorted_l[r]} : int2{-1, 0};
    }
    if (t == 0) {
        plan[0] = B;
        plan[1] = M;
    }
}

}  // namespace plan

int64_t plan_bundle_count(int64_t batch, int64_t kv_heads) {
    const int64_t m = (plan::kGroups + kv_heads - 1) / kv_heads;
    const int64_t least = (batch + plan::kPerBundle - 1) / plan::kPerBundle;
    return m < least ? least : m;
}
int64_t plan_ints(int64_t batch, int64_t kv_heads) {
    return 2 + 2 * plan::kPerBundle * plan_bundle_count(batch, kv_heads);
}
int plan_launch(const int64_t *pos, int batch, int ctx, int bundles, int32_t *plan, hipStream_t s) {
    hipLaunchKernelGGL(plan::decode_plan_kernel, dim3(1), dim3(plan::kMaxBatch), 0, s, pos, batch, ctx, bundles, plan);
    return launch_status();
}

}  // namespace q3t
