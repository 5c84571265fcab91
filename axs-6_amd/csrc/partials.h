// Fixed-order column sums of per-chunk partial rows (the bias gradient of the
// quantized linear), shared by the packing and GEMM translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace axs6 {
namespace {

// db[c] = sum of partial[k, c] over the chunks k, in a fixed order: a
// workgroup takes 16 columns, its 16 thread groups 16 consecutive ranges of
// chunks (each summed in order, eight loads in flight), then the ranges are
// added in order.
constexpr int kRedCols = 16, kRedRanges = 16;

// out[c] = sum_k partial[k, c] for the kRedCols columns of block `bx`: 16
// ranges of k summed by 16 thread groups, then the ranges added in order.
__device__ __forceinline__ void reduce_partials_block(const float* __restrict__ partial, int64_t chunks,
                                                      int64_t cols, float* __restrict__ out, int64_t bx) {
    __shared__ float part[kRedRanges][kRedCols + 1];
    const int lc = threadIdx.x % kRedCols, q = threadIdx.x / kRedCols;
    const int64_t c = bx * kRedCols + lc;
    const int64_t per = (chunks + kRedRanges - 1) / kRedRanges;
    const int64_t k0 = q * per, k1 = (k0 + per) < chunks ? k0 + per : chunks;
    float s = 0.0f;
    if (c < cols) {
        int64_t kk = k0;
        for (; kk + 8 <= k1; kk += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = partial[(kk + u) * cols + c];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += v[u];
        }
        for (; kk < k1; ++kk) s += partial[kk * cols + c];
    }
    part[q][lc] = s;
    __syncthreads();
    if (q == 0 && c < cols) {
        float t = part[0][lc];
#pragma unroll
        for (int r = 1; r < kRedRanges; ++r) t += part[r][lc];
        out[c] = t;
    }
}

}  // namespace
}  // namespace axs6
