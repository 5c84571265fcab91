// Gradient unscale + overflow check + global-norm clip over a list of
// tensors: the loss-scaling and clipping steps of the reference's training
// step (axs/unified/training_unified.py:224-257), which divides every
// gradient by the loss scale, checks every gradient for inf/NaN with two
// host-synchronising reductions per parameter, and calls clip_grad_norm_.
//
// Here three kernels, all on the device, no host synchronisation:
//   unscale_norm_kernel  g *= fl(1 / loss_scale) in place -- what torch's
//                        grad.div_(loss_scale) computes on the GPU (a scalar
//                        divisor becomes a multiply by its fp32 reciprocal;
//                        the same as a division for power-of-two scales);
//                        per workgroup, the sum of
//                        squares of the unscaled values and the count of
//                        non-finite ones -> partials (fixed summation order)
//   finalize_kernel      one workgroup: partials summed in order (fp64) ->
//                        result = {norm, min(max_norm / (norm + 1e-6), 1), nonfinite}
//   clip_kernel          g *= result[1] when nothing overflowed and the
//                        coefficient is below 1 (no writes otherwise)
// A launch covers up to kMTMax tensors of one dtype, their pointers and sizes
// passed by value in the kernel arguments; a workgroup handles kMTChunk
// elements of one tensor.  HBM-bound: 2 reads + 1 write of each gradient
// element when the clip applies, 1 read + 1 write otherwise (f32: 8-12 B).
#include <limits.h>
#include <math.h>

#include "nf5_device.h"

namespace axs6 {
namespace {

constexpr int kMTMax = 48;         // tensors per launch (kernel-argument table)
constexpr int kMTThreads = 256;
constexpr int kMTChunk = 16384;    // elements per workgroup

struct MTArgs {
    void* ptr[kMTMax];
    int64_t n[kMTMax];
    int32_t wg0[kMTMax + 1];       // first workgroup of each tensor; wg0[count] = workgroups
    int32_t count;
    int32_t part0;                 // this launch's first partial
};

// tensor and element range of workgroup w (count <= kMTMax, uniform scan)
__device__ __forceinline__ int mt_tensor(const MTArgs& a, int w) {
    int t = 0;
    while (t + 1 < a.count && a.wg0[t + 1] <= w) ++t;
    return t;
}

__device__ __forceinline__ float block_sum_fixed(float v, float* red) {
    // wave sums in a fixed butterfly order, then the waves in order
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kMTThreads / 64; ++w) s += red[w];
    return s;
}

// Both element kernels multiply in fp32 and round once to the tensor dtype.
// For 16-bit tensors the compiler folds a multiply followed by the narrowing
// conversion into a mixed-precision fma with a +0 addend, which turns a -0
// product into +0; the product goes through an empty asm first, so the
// multiply and the round-to-nearest conversion stay separate instructions.
template <int DT>
__device__ __forceinline__ float product(float a, float b) {
    float v = a * b;
    if constexpr (DT != AXS6_F32) asm volatile("" : "+v"(v));
    return v;
}

template <int DT>
__global__ __launch_bounds__(kMTThreads) void unscale_norm_kernel(MTArgs a, float inv, float* partials,
                                                                 int64_t total_wg) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int V = E::V;
    __shared__ float red[2][kMTThreads / 64];
    const int w = blockIdx.x;
    const int t = mt_tensor(a, w);
    const int64_t n = a.n[t];
    const int64_t b = (int64_t)(w - a.wg0[t]) * kMTChunk;
    const int64_t e = b + kMTChunk < n ? b + kMTChunk : n;
    S* p = reinterpret_cast<S*>(a.ptr[t]);
    const bool div = inv != 1.0f;
    float ss = 0.0f, nf = 0.0f;
    // 16-byte vectors where the pointer allows, then element by element
    const int64_t lead = ((uintptr_t)(p + b) % 16 == 0) ? 0 : (e - b);
    const int64_t nvec = (e - b - lead) / V;
    for (int64_t i = threadIdx.x; i < nvec; i += kMTThreads) {
        u32x4* q = reinterpret_cast<u32x4*>(p + b + i * V);
        float f[V];
        E::unpack(*q, f);
#pragma unroll
        for (int k = 0; k < V; ++k) {
            if (div) f[k] = E::to_f(E::from_f(product<DT>(f[k], inv)));
            ss += f[k] * f[k];
            nf += isfinite(f[k]) ? 0.0f : 1.0f;
        }
        if (div) *q = E::pack(f);
    }
    for (int64_t i = b + nvec * V + threadIdx.x; i < e; i += kMTThreads) {
        float f = E::to_f(p[i]);
        if (div) {
            const S s = E::from_f(product<DT>(f, inv));
            p[i] = s;
            f = E::to_f(s);
        }
        ss += f * f;
        nf += isfinite(f) ? 0.0f : 1.0f;
    }
    ss = block_sum_fixed(ss, red[0]);
    nf = block_sum_fixed(nf, red[1]);
    if (threadIdx.x == 0) {
        partials[a.part0 + w] = ss;
        partials[total_wg + a.part0 + w] = nf;
    }
}

__global__ __launch_bounds__(kMTThreads) void finalize_kernel(const float* partials, int64_t total_wg,
                                                             float max_norm, float* result) {
    __shared__ double red[2][kMTThreads];
    double ss = 0.0, nf = 0.0;
    for (int64_t i = threadIdx.x; i < total_wg; i += kMTThreads) {
        ss += (double)partials[i];
        nf += (double)partials[total_wg + i];
    }
    red[0][threadIdx.x] = ss;
    red[1][threadIdx.x] = nf;
    __syncthreads();
    for (int s = kMTThreads / 2; s >= 1; s >>= 1) {
        if ((int)threadIdx.x < s) {
            red[0][threadIdx.x] += red[0][threadIdx.x + s];
            red[1][threadIdx.x] += red[1][threadIdx.x + s];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float norm = (float)sqrt(red[0][0]);
        float coef = max_norm / (norm + 1e-6f);
        coef = coef > 1.0f ? 1.0f : coef;          // torch.clamp(clip_coef, max=1.0): NaN stays NaN
        result[0] = norm;
        result[1] = coef;
        result[2] = (float)red[1][0];
    }
}

template <int DT>
__global__ __launch_bounds__(kMTThreads) void clip_kernel(MTArgs a, const float* result) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int V = E::V;
    const float coef = result[1];
    if (result[2] != 0.0f || !(coef < 1.0f)) return;   // overflow, or nothing to clip
    const int w = blockIdx.x;
    const int t = mt_tensor(a, w);
    const int64_t n = a.n[t];
    const int64_t b = (int64_t)(w - a.wg0[t]) * kMTChunk;
    const int64_t e = b + kMTChunk < n ? b + kMTChunk : n;
    S* p = reinterpret_cast<S*>(a.ptr[t]);
    const int64_t lead = ((uintptr_t)(p + b) % 16 == 0) ? 0 : (e - b);
    const int64_t nvec = (e - b - lead) / V;
    for (int64_t i = threadIdx.x; i < nvec; i += kMTThreads) {
        u32x4* q = reinterpret_cast<u32x4*>(p + b + i * V);
        float f[V];
        E::unpack(*q, f);
#pragma unroll
        for (int k = 0; k < V; ++k) f[k] = product<DT>(f[k], coef);
        *q = E::pack(f);
    }
    for (int64_t i = b + nvec * V + threadIdx.x; i < e; i += kMTThreads) p[i] = E::from_f(product<DT>(E::to_f(p[i]), coef));
}

int64_t wg_of(int64_t n) { return (n + kMTChunk - 1) / kMTChunk; }

// Splits the list into launches of at most kMTMax tensors of one dtype.
template <typename F>
int for_each_launch(void* const* grads, const int64_t* numel, const int32_t* dtypes, int32_t count, F&& fn) {
    int32_t i = 0;
    int64_t part = 0;
    while (i < count) {
        MTArgs a{};
        const int dt = dtypes[i];
        int32_t wg = 0;
        while (i < count && a.count < kMTMax && dtypes[i] == dt) {
            if (numel[i] > 0) {
                a.ptr[a.count] = grads[i];
                a.n[a.count] = numel[i];
                a.wg0[a.count] = wg;
                wg += (int32_t)wg_of(numel[i]);
                ++a.count;
            }
            ++i;
        }
        if (a.count == 0) continue;
        a.wg0[a.count] = wg;
        a.part0 = (int32_t)part;
        int rc = fn(a, dt, wg);
        if (rc) return rc;
        part += wg;
    }
    return AXS6_OK;
}

}  // namespace
}  // namespace axs6

using namespace axs6;

extern "C" int64_t axs6_multi_tensor_workspace(const int64_t* numel, int32_t count) {
    if (count < 0 || (count > 0 && !numel)) return -1;
    int64_t wg = 0;
    for (int32_t i = 0; i < count; ++i)
        if (numel[i] > 0) wg += wg_of(numel[i]);
    return 2 * wg;
}

extern "C" int axs6_multi_tensor_unscale_clip(void* const* grads, const int64_t* numel, const int32_t* dtypes,
                                              int32_t count, float loss_scale, float max_norm, int32_t clip,
                                              float* partials, int64_t partials_len, float* result, void* stream) {
    const char* fn = "axs6_multi_tensor_unscale_clip";
    if (count < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative tensor count", fn);
    if (!result) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null result", fn);
    if (count > 0 && (!grads || !numel || !dtypes))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null tensor list", fn);
    int64_t wg = 0;
    for (int32_t i = 0; i < count; ++i) {
        if (numel[i] < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative element count", fn);
        if (!valid_dtype(dtypes[i])) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtypes[i]);
        if (numel[i] > 0 && !grads[i]) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null gradient %d", fn, i);
        if (numel[i] > 0 && (uintptr_t)grads[i] % (dtypes[i] == AXS6_F32 ? 4 : 2) != 0)
            return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: gradient %d is not element-aligned", fn, i);
        wg += wg_of(numel[i]);
    }
    if (wg > INT_MAX / 2) return fail(AXS6_ERR_UNSUPPORTED, "%s: too many elements", fn);
    // positive; +inf allowed: as in torch, its float reciprocal is 0 and the
    // overflow count then catches every non-finite gradient (inf * 0 = NaN)
    if (!(loss_scale > 0.0f)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: loss_scale must be positive", fn);
    if (wg > 0 && (!partials || partials_len < 2 * wg))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: workspace of %lld floats required, got %lld", fn,
                    (long long)(2 * wg), (long long)partials_len);
    hipStream_t st = (hipStream_t)stream;
    const float inv = 1.0f / loss_scale;          // host IEEE division, as torch forms the reciprocal
    int rc = for_each_launch(grads, numel, dtypes, count, [&](const MTArgs& a, int dt, int32_t nwg) {
        const dim3 grid((unsigned)nwg);
        if (dt == AXS6_F32) unscale_norm_kernel<AXS6_F32><<<grid, kMTThreads, 0, st>>>(a, inv, partials, wg);
        else if (dt == AXS6_BF16) unscale_norm_kernel<AXS6_BF16><<<grid, kMTThreads, 0, st>>>(a, inv, partials, wg);
        else unscale_norm_kernel<AXS6_F16><<<grid, kMTThreads, 0, st>>>(a, inv, partials, wg);
        return check_launch(fn);
    });
    if (rc) return rc;
    finalize_kernel<<<1, kMTThreads, 0, st>>>(partials, wg, max_norm, result);
    if ((rc = check_launch(fn))) return rc;
    if (!clip) return AXS6_OK;
    return for_each_launch(grads, numel, dtypes, count, [&](const MTArgs& a, int dt, int32_t nwg) {
        const dim3 grid((unsigned)nwg);
        if (dt == AXS6_F32) clip_kernel<AXS6_F32><<<grid, kMTThreads, 0, st>>>(a, result);
        else if (dt == AXS6_BF16) clip_kernel<AXS6_BF16><<<grid, kMTThreads, 0, st>>>(a, result);
        else clip_kernel<AXS6_F16><<<grid, kMTThreads, 0, st>>>(a, result);
        return check_launch(fn);
    });
}
