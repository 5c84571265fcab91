// LayerNorm over the last `cols` values of each row, forward and backward:
// the normalisation of AXSLayerNormUnified (the reference's module calls
// F.layer_norm, axs/unified/modules_unified.py:120-144), here as HBM-streaming
// kernels instead of torch's.
//
//   mean_r = p_r + sum_c (x - p_r) / cols  (p_r = x[r, 0]: rows far from zero
//   keep their digits),  var_r = sum_c (x - mean_r)^2 / cols  (biased),
//   rstd_r = 1 / sqrt(var_r + eps),  xhat = (x - mean_r) * rstd_r,
//   y = xhat * gamma[c] + beta[c]
//   backward (g = dy * gamma):  dx = rstd_r * (g - (sum_c g + xhat * sum_c g*xhat) / cols),
//   dgamma[c] = sum_r dy * xhat,  dbeta[c] = sum_r dy
//
// Vector form (rows of whole 16-byte vectors, 16-byte aligned, at most
// 8192 f32 / 16384 16-bit values): a row is held in registers -- one wave per
// row up to 1024 f32 / 2048 16-bit values (four rows per workgroup), else
// one 256-thread workgroup per row -- so the statistics take one HBM read.
// The backward reads x and dy once per row: each thread keeps its columns'
// dgamma/dbeta sums over the rows of its workgroup, the workgroup writes them
// as one partial row (dgamma rows, then dbeta rows, one per workgroup), and a
// second launch sums the partial rows in a fixed order (deterministic for a
// given shape).
//
// Generic form (any length, alignment or size): one 256-thread workgroup per
// row streams it (three passes forward, two backward; the passes after the
// first read the row back from cache); the parameter sums run as a column
// pass over row ranges (one partial row per range) before the same fixed-order
// reduction.
#include <math.h>

#include "axs6_internal.h"
#include "nf5_device.h"
#include "partials.h"

namespace axs6 {
namespace {

constexpr int kLnThreads = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over the NT threads of a row group (NT == 64: one wave; NT == 256: the
// workgroup, through `red`, which holds 2 * 4 floats); every thread gets it.
template <int NT>
__device__ __forceinline__ float2 group_sum2(float a, float b, float* red) {
    a = wave_sum(a);
    b = wave_sum(b);
    if constexpr (NT == 64) {
        return make_float2(a, b);
    } else {
        const int w = threadIdx.x >> 6;
        __syncthreads();   // red may still be read by the previous reduction
        if ((threadIdx.x & 63) == 0) { red[w] = a; red[4 + w] = b; }
        __syncthreads();
        return make_float2((red[0] + red[1]) + (red[2] + red[3]), (red[4] + red[5]) + (red[6] + red[7]));
    }
}

template <int DT>
__device__ __forceinline__ void load_vec(const void* p, int64_t i, float* f) {
    using E = Elem<DT>;
    E::unpack(reinterpret_cast<const u32x4*>(p)[i], f);
}

template <int DT>
__device__ __forceinline__ void store_vec(void* p, int64_t i, const float* f) {
    using E = Elem<DT>;
    reinterpret_cast<u32x4*>(p)[i] = E::pack(f);
}

struct LnArgs {
    const void* x; const void* dy; const void* gamma; const void* beta;
    void* y; void* dx; float* mean; float* rstd;
    float* part;          // backward: [chunks, cols] partial dgamma rows, then [chunks, cols] dbeta rows
    int64_t rows, cols;
    float eps;
};

// ---- vector form ---------------------------------------------------------------

// NT threads per row, NV 16-byte vectors each; RPW rows per workgroup
// (RPW > 1 only with NT == 64).  Thread t of a row group holds vectors
// t, t + NT, ..., t + (NV - 1) * NT of the row.
template <int DT, int NT, int NV>
__global__ __launch_bounds__(kLnThreads) void ln_fwd_vec_kernel(LnArgs a) {
    using E = Elem<DT>;
    constexpr int V = E::V, RPW = kLnThreads / NT;
    __shared__ float red[8];
    const int t = threadIdx.x % NT, g = threadIdx.x / NT;
    const int64_t nvec = a.cols / V;
    // a wave's row group keeps its columns' gamma and beta in registers across
    // rows; a workgroup row reads them at the store (cache hits), which leaves
    // registers for more rows in flight
    constexpr bool KEEP = NT == 64;
    constexpr int NK = KEEP ? NV : 1;
    float gm[NK][V], bt[NK][V];
    if constexpr (KEEP) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = t + (int64_t)j * NT;
#pragma unroll
            for (int e = 0; e < V; ++e) { gm[j][e] = 1.0f; bt[j][e] = 0.0f; }
            if (vi < nvec) {
                if (a.gamma) load_vec<DT>(a.gamma, vi, gm[j]);
                if (a.beta) load_vec<DT>(a.beta, vi, bt[j]);
            }
        }
    }
    for (int64_t r0 = (int64_t)blockIdx.x * RPW; r0 < a.rows; r0 += (int64_t)gridDim.x * RPW) {
        const int64_t r = r0 + g;
        // NT == 256 rows are workgroup-uniform; NT == 64 rows are wave-uniform,
        // so an out-of-range row group skips its reductions as a whole
        if (NT == 64 && r >= a.rows) break;
        const void* xr = reinterpret_cast<const char*>(a.x) + r * a.cols * (int64_t)sizeof(typename E::S);
        const float piv = E::to_f(*reinterpret_cast<const typename E::S*>(xr));
        float v[NV][V];
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = t + (int64_t)j * NT;
#pragma unroll
            for (int e = 0; e < V; ++e) v[j][e] = 0.0f;
            if (vi < nvec) {
                load_vec<DT>(xr, vi, v[j]);
#pragma unroll
                for (int e = 0; e < V; ++e) s += v[j][e] - piv;
            }
        }
        const float mean = piv + group_sum2<NT>(s, 0.0f, red).x / (float)a.cols;
        float q = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const bool in = t + (int64_t)j * NT < nvec;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const float d = v[j][e] - mean;
                q += in ? d * d : 0.0f;
            }
        }
        const float var = group_sum2<NT>(q, 0.0f, red).x / (float)a.cols;
        const float rstd = rsqrtf(var + a.eps);
        void* yr = reinterpret_cast<char*>(a.y) + r * a.cols * (int64_t)sizeof(typename E::S);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = t + (int64_t)j * NT;
            if (vi < nvec) {
                float o[V], gw[V], bw[V];
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    gw[e] = KEEP ? gm[KEEP ? j : 0][e] : 1.0f;
                    bw[e] = KEEP ? bt[KEEP ? j : 0][e] : 0.0f;
                }
                if constexpr (!KEEP) {
                    if (a.gamma) load_vec<DT>(a.gamma, vi, gw);
                    if (a.beta) load_vec<DT>(a.beta, vi, bw);
                }
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = (v[j][e] - mean) * rstd * gw[e] + bw[e];
                store_vec<DT>(yr, vi, o);
            }
        }
        if (t == 0) {
            if (a.mean) a.mean[r] = mean;
            if (a.rstd) a.rstd[r] = rstd;
        }
    }
}

template <int DT, int NT, int NV>
__global__ __launch_bounds__(kLnThreads) void ln_bwd_vec_kernel(LnArgs a) {
    using E = Elem<DT>;
    constexpr int V = E::V, RPW = kLnThreads / NT;
    __shared__ float red[8];
    __shared__ float cs[RPW > 1 ? RPW : 1][2][64 * V + 1];   // per-wave column sums (NT == 64)
    const int t = threadIdx.x % NT, g = threadIdx.x / NT;
    const int64_t nvec = a.cols / V;
    float gm[NV][V], pg[NV][V], pb[NV][V];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t vi = t + (int64_t)j * NT;
#pragma unroll
        for (int e = 0; e < V; ++e) { gm[j][e] = 1.0f; pg[j][e] = 0.0f; pb[j][e] = 0.0f; }
        if (a.gamma && vi < nvec) load_vec<DT>(a.gamma, vi, gm[j]);
    }
    const float inv_n = 1.0f / (float)a.cols;
    const size_t es = sizeof(typename E::S);
    for (int64_t r0 = (int64_t)blockIdx.x * RPW; r0 < a.rows; r0 += (int64_t)gridDim.x * RPW) {
        const int64_t r = r0 + g;
        if (NT == 64 && r >= a.rows) break;
        const void* xr = reinterpret_cast<const char*>(a.x) + r * a.cols * (int64_t)es;
        const void* dyr = reinterpret_cast<const char*>(a.dy) + r * a.cols * (int64_t)es;
        const float mean = a.mean[r], rstd = a.rstd[r];
        float xh[NV][V], gg[NV][V];
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = t + (int64_t)j * NT;
            float xv[V], dv[V];
#pragma unroll
            for (int e = 0; e < V; ++e) { xv[e] = 0.0f; dv[e] = 0.0f; }
            if (vi < nvec) {
                load_vec<DT>(xr, vi, xv);
                load_vec<DT>(dyr, vi, dv);
            }
            const bool in = vi < nvec;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                xh[j][e] = in ? (xv[e] - mean) * rstd : 0.0f;   // dy is 0 past the row too
                gg[j][e] = dv[e] * gm[j][e];
                s1 += gg[j][e];
                s2 += gg[j][e] * xh[j][e];
                pg[j][e] += dv[e] * xh[j][e];
                pb[j][e] += dv[e];
            }
        }
        const float2 s = group_sum2<NT>(s1, s2, red);
        void* dxr = reinterpret_cast<char*>(a.dx) + r * a.cols * (int64_t)es;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = t + (int64_t)j * NT;
            if (vi < nvec) {
                float o[V];
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = rstd * (gg[j][e] - (s.x + xh[j][e] * s.y) * inv_n);
                store_vec<DT>(dxr, vi, o);
            }
        }
    }
    // this workgroup's partial rows (grid = chunks): the row groups' column
    // sums added in order
    float* prow[2] = {a.part + (int64_t)blockIdx.x * a.cols, a.part + ((int64_t)gridDim.x + blockIdx.x) * a.cols};
    if constexpr (RPW == 1) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = t + (int64_t)j * NT;
            if (vi < nvec) {
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    prow[0][vi * V + e] = pg[j][e];
                    prow[1][vi * V + e] = pb[j][e];
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            __syncthreads();
#pragma unroll
            for (int e = 0; e < V; ++e) {
                cs[g][0][t * V + e] = pg[j][e];
                cs[g][1][t * V + e] = pb[j][e];
            }
            __syncthreads();
            // thread k of the workgroup adds column k % (64 V) of the staged
            // vectors over the row groups, in order
            for (int k = threadIdx.x; k < 2 * 64 * V; k += kLnThreads) {
                const int which = k / (64 * V), c = k % (64 * V);
                const int64_t col = (int64_t)j * 64 * V + c;
                if (col < a.cols) {
                    float sum = cs[0][which][c];
#pragma unroll
                    for (int q = 1; q < RPW; ++q) sum += cs[q][which][c];
                    prow[which][col] = sum;
                }
            }
        }
    }
}

// ---- generic form --------------------------------------------------------------

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
    return Elem<DT>::to_f(reinterpret_cast<const typename Elem<DT>::S*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
    reinterpret_cast<typename Elem<DT>::S*>(p)[i] = Elem<DT>::from_f(v);
}

template <int DT>
__global__ __launch_bounds__(kLnThreads) void ln_fwd_row_kernel(LnArgs a) {
    __shared__ float red[8];
    for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
        const int64_t base = r * a.cols;
        const float piv = ld<DT>(a.x, base);
        float s = 0.0f;
        for (int64_t c = threadIdx.x; c < a.cols; c += kLnThreads) s += ld<DT>(a.x, base + c) - piv;
        const float mean = piv + group_sum2<kLnThreads>(s, 0.0f, red).x / (float)a.cols;
        float q = 0.0f;
        for (int64_t c = threadIdx.x; c < a.cols; c += kLnThreads) {
            const float d = ld<DT>(a.x, base + c) - mean;
            q += d * d;
        }
        const float rstd = rsqrtf(group_sum2<kLnThreads>(q, 0.0f, red).x / (float)a.cols + a.eps);
        for (int64_t c = threadIdx.x; c < a.cols; c += kLnThreads) {
            const float gmv = a.gamma ? ld<DT>(a.gamma, c) : 1.0f, btv = a.beta ? ld<DT>(a.beta, c) : 0.0f;
            st<DT>(a.y, base + c, (ld<DT>(a.x, base + c) - mean) * rstd * gmv + btv);
        }
        if (threadIdx.x == 0) {
            if (a.mean) a.mean[r] = mean;
            if (a.rstd) a.rstd[r] = rstd;
        }
    }
}

// dx of rows b, b + gridDim.x, ... (two passes over each row: the sums, then dx).
template <int DT>
__global__ __launch_bounds__(kLnThreads) void ln_bwd_row_kernel(LnArgs a) {
    __shared__ float red[8];
    const float inv_n = 1.0f / (float)a.cols;
    for (int64_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
        const int64_t base = r * a.cols;
        const float mean = a.mean[r], rstd = a.rstd[r];
        float s1 = 0.0f, s2 = 0.0f;
        for (int64_t c = threadIdx.x; c < a.cols; c += kLnThreads) {
            const float xh = (ld<DT>(a.x, base + c) - mean) * rstd;
            const float gv = ld<DT>(a.dy, base + c) * (a.gamma ? ld<DT>(a.gamma, c) : 1.0f);
            s1 += gv;
            s2 += gv * xh;
        }
        const float2 s = group_sum2<kLnThreads>(s1, s2, red);
        for (int64_t c = threadIdx.x; c < a.cols; c += kLnThreads) {
            const float xh = (ld<DT>(a.x, base + c) - mean) * rstd;
            const float gv = ld<DT>(a.dy, base + c) * (a.gamma ? ld<DT>(a.gamma, c) : 1.0f);
            st<DT>(a.dx, base + c, rstd * (gv - (s.x + xh * s.y) * inv_n));
        }
    }
}

// Generic form's parameter sums: block (x, y) takes 256 columns and the y-th
// of gridDim.y consecutive row ranges; each thread sums its column's
// dy * xhat and dy over the range in row order into partial row y.
template <int DT>
__global__ __launch_bounds__(kLnThreads) void ln_bwd_cols_kernel(LnArgs a) {
    const int64_t c = (int64_t)blockIdx.x * kLnThreads + threadIdx.x;
    const int64_t per = (a.rows + gridDim.y - 1) / gridDim.y;
    const int64_t r0 = (int64_t)blockIdx.y * per;
    const int64_t r1 = (r0 + per) < a.rows ? r0 + per : a.rows;
    if (c >= a.cols) return;
    float pg = 0.0f, pb = 0.0f;
    for (int64_t r = r0; r < r1; ++r) {
        const float dv = ld<DT>(a.dy, r * a.cols + c);
        pg += dv * ((ld<DT>(a.x, r * a.cols + c) - a.mean[r]) * a.rstd[r]);
        pb += dv;
    }
    a.part[(int64_t)blockIdx.y * a.cols + c] = pg;
    a.part[((int64_t)gridDim.y + blockIdx.y) * a.cols + c] = pb;
}

// dgamma[c] (blocks [0, nb)) and dbeta[c] (blocks [nb, 2 nb)) from the
// partial rows, in a fixed order; chunks == 0 writes zeros.
__global__ __launch_bounds__(kLnThreads) void ln_reduce_kernel(const float* part, int64_t chunks, int64_t cols,
                                                               float* dgamma, float* dbeta, int64_t nb) {
    const bool beta = blockIdx.x >= nb;
    const int64_t b = beta ? blockIdx.x - nb : blockIdx.x;
    float* out = beta ? dbeta : dgamma;
    if (!out) return;   // block-uniform
    reduce_partials_block(part + (beta ? chunks * cols : 0), chunks, cols, out, b);
}

// ---- launch shapes ---------------------------------------------------------------

struct LnShape { int nt; int nv; bool vec; };

// Row groups of 64 threads (one wave per row) while a row has at most
// 64 * cap64 vectors, else 256 threads with at most cap256 vectors each;
// longer, ragged or unaligned rows take the generic form.  The caps keep the
// row in registers without spills (the backward holds five values per
// element, 16-bit rows twice as many elements per vector).
LnShape ln_shape(int dtype, int64_t cols, const void* const* ptrs, int nptr, bool bwd) {
    const int V = dtype == AXS6_F32 ? 4 : 8;
    const int cap64 = (bwd && V == 8) ? 2 : 4;
    const int cap256 = (V == 8) ? 4 : 8;
    LnShape s{0, 0, false};
    if (cols <= 0 || cols % V != 0) return s;
    for (int i = 0; i < nptr; ++i)
        if (ptrs[i] && (uintptr_t)ptrs[i] % 16 != 0) return s;
    const int64_t nvec = cols / V;
    if (nvec <= 64 * cap64) {
        s.nt = 64;
        s.nv = (int)((nvec + 63) / 64);
    } else if (nvec <= 256 * cap256) {
        s.nt = 256;
        s.nv = (int)((nvec + 255) / 256);
    } else {
        return s;
    }
    s.vec = true;
    return s;
}

template <int DT, int NT, int NV>
void launch_fwd_vec(const LnArgs& a, hipStream_t st) {
    constexpr int RPW = kLnThreads / NT;
    const int64_t groups = (a.rows + RPW - 1) / RPW;
    const unsigned grid = (unsigned)(groups < 65536 ? groups : 65536);
    ln_fwd_vec_kernel<DT, NT, NV><<<grid, kLnThreads, 0, st>>>(a);
}

template <int DT, int NT, int NV>
void launch_bwd_vec(const LnArgs& a, int64_t chunks, hipStream_t st) {
    ln_bwd_vec_kernel<DT, NT, NV><<<(unsigned)chunks, kLnThreads, 0, st>>>(a);
}

template <int DT>
int fwd_dispatch(const LnArgs& a, const LnShape& s, hipStream_t st) {
    if (!s.vec) {
        const unsigned grid = (unsigned)(a.rows < 65536 ? a.rows : 65536);
        ln_fwd_row_kernel<DT><<<grid, kLnThreads, 0, st>>>(a);
        return AXS6_OK;
    }
    if (s.nt == 64) {
        switch (s.nv) {
            case 1: launch_fwd_vec<DT, 64, 1>(a, st); break;
            case 2: launch_fwd_vec<DT, 64, 2>(a, st); break;
            case 3: launch_fwd_vec<DT, 64, 3>(a, st); break;
            default: launch_fwd_vec<DT, 64, 4>(a, st); break;
        }
    } else if constexpr (DT == AXS6_F32) {
        switch (s.nv) {
            case 1: case 2: launch_fwd_vec<DT, 256, 2>(a, st); break;
            case 3: launch_fwd_vec<DT, 256, 3>(a, st); break;
            case 4: launch_fwd_vec<DT, 256, 4>(a, st); break;
            case 5: case 6: launch_fwd_vec<DT, 256, 6>(a, st); break;
            default: launch_fwd_vec<DT, 256, 8>(a, st); break;
        }
    } else {
        switch (s.nv) {
            case 1: case 2: launch_fwd_vec<DT, 256, 2>(a, st); break;
            case 3: launch_fwd_vec<DT, 256, 3>(a, st); break;
            default: launch_fwd_vec<DT, 256, 4>(a, st); break;
        }
    }
    return AXS6_OK;
}

template <int DT>
int bwd_dispatch(const LnArgs& a, const LnShape& s, int64_t chunks, hipStream_t st) {
    if (!s.vec) {
        const unsigned grid = (unsigned)(a.rows < 65536 ? a.rows : 65536);
        ln_bwd_row_kernel<DT><<<grid, kLnThreads, 0, st>>>(a);
        const dim3 cgrid((unsigned)((a.cols + kLnThreads - 1) / kLnThreads), (unsigned)chunks);
        ln_bwd_cols_kernel<DT><<<cgrid, kLnThreads, 0, st>>>(a);
        return AXS6_OK;
    }
    if constexpr (DT == AXS6_F32) {
        if (s.nt == 64) {
            switch (s.nv) {
                case 1: launch_bwd_vec<DT, 64, 1>(a, chunks, st); break;
                case 2: launch_bwd_vec<DT, 64, 2>(a, chunks, st); break;
                case 3: launch_bwd_vec<DT, 64, 3>(a, chunks, st); break;
                default: launch_bwd_vec<DT, 64, 4>(a, chunks, st); break;
            }
        } else {
            switch (s.nv) {
                case 1: case 2: launch_bwd_vec<DT, 256, 2>(a, chunks, st); break;
                case 3: launch_bwd_vec<DT, 256, 3>(a, chunks, st); break;
                case 4: launch_bwd_vec<DT, 256, 4>(a, chunks, st); break;
                case 5: case 6: launch_bwd_vec<DT, 256, 6>(a, chunks, st); break;
                default: launch_bwd_vec<DT, 256, 8>(a, chunks, st); break;
            }
        }
    } else {
        if (s.nt == 64) {
            if (s.nv == 1) launch_bwd_vec<DT, 64, 1>(a, chunks, st);
            else launch_bwd_vec<DT, 64, 2>(a, chunks, st);
        } else {
            switch (s.nv) {
                case 1: launch_bwd_vec<DT, 256, 1>(a, chunks, st); break;
                case 2: launch_bwd_vec<DT, 256, 2>(a, chunks, st); break;
                case 3: launch_bwd_vec<DT, 256, 3>(a, chunks, st); break;
                default: launch_bwd_vec<DT, 256, 4>(a, chunks, st); break;
            }
        }
    }
    return AXS6_OK;
}

// Workgroups of the backward (= partial rows): about 16 rows each, at most 2048.
int64_t bwd_chunks(int64_t rows) {
    if (rows <= 0) return 0;
    const int64_t c = (rows + 15) / 16;
    return c < 2048 ? c : 2048;
}

int check_common(const char* fn, int dtype, int64_t rows, int64_t cols) {
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    if (rows < 0 || cols < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative dimension", fn);
    if (rows > ((int64_t)1 << 40) || cols > ((int64_t)1 << 31))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: dimension too large", fn);
    return AXS6_OK;
}

}  // namespace
}  // namespace axs6

using namespace axs6;

extern "C" int axs6_layer_norm_forward(const void* x, int32_t dtype, int64_t rows, int64_t cols, const void* gamma,
                                       const void* beta, float eps, void* y, float* mean, float* rstd,
                                       void* stream) {
    const char* fn = "axs6_layer_norm_forward";
    int rc = check_common(fn, dtype, rows, cols);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return AXS6_OK;
    if (!x || !y) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null input or output", fn);
    if (!(eps >= 0.0f)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: eps must be non-negative", fn);
    const size_t es = dtype == AXS6_F32 ? 4 : 2;
    const void* ptrs[] = {x, y, gamma, beta};
    for (const void* p : ptrs)
        if (p && (uintptr_t)p % es != 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: pointer not element-aligned", fn);
    LnShape s = ln_shape(dtype, cols, ptrs, 4, false);
    LnArgs a{x, nullptr, gamma, beta, y, nullptr, mean, rstd, nullptr, rows, cols, eps};
    hipStream_t st = (hipStream_t)stream;
    if (dtype == AXS6_F32) rc = fwd_dispatch<AXS6_F32>(a, s, st);
    else if (dtype == AXS6_BF16) rc = fwd_dispatch<AXS6_BF16>(a, s, st);
    else rc = fwd_dispatch<AXS6_F16>(a, s, st);
    return rc ? rc : check_launch(fn);
}

extern "C" int64_t axs6_layer_norm_backward_workspace(int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return -1;
    return bwd_chunks(rows) * 2 * cols * (int64_t)sizeof(float);
}

extern "C" int axs6_layer_norm_backward(const void* dy, const void* x, int32_t dtype, int64_t rows, int64_t cols,
                                        const float* mean, const float* rstd, const void* gamma, void* dx,
                                        float* dgamma, float* dbeta, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    const char* fn = "axs6_layer_norm_backward";
    int rc = check_common(fn, dtype, rows, cols);
    if (rc) return rc;
    if (cols == 0) return AXS6_OK;
    hipStream_t st = (hipStream_t)stream;
    const int64_t chunks = bwd_chunks(rows);
    const int64_t nb = (cols + kRedCols - 1) / kRedCols;
    if (rows > 0) {
        if (!dy || !x || !dx || !mean || !rstd)
            return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null dy, x, dx, mean or rstd", fn);
        const size_t need = (size_t)chunks * 2 * (size_t)cols * sizeof(float);
        if (!workspace || workspace_bytes < need)
            return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: workspace of %zu bytes required, got %zu", fn, need,
                        workspace_bytes);
        if ((uintptr_t)workspace % 4 != 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: workspace not aligned", fn);
        const size_t es = dtype == AXS6_F32 ? 4 : 2;
        const void* ptrs[] = {dy, x, dx, gamma};
        for (const void* p : ptrs)
            if (p && (uintptr_t)p % es != 0)
                return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: pointer not element-aligned", fn);
        LnShape s = ln_shape(dtype, cols, ptrs, 4, true);
        LnArgs a{x, dy, gamma, nullptr, nullptr, dx, const_cast<float*>(mean), const_cast<float*>(rstd),
                 reinterpret_cast<float*>(workspace), rows, cols, 0.0f};
        if (dtype == AXS6_F32) rc = bwd_dispatch<AXS6_F32>(a, s, chunks, st);
        else if (dtype == AXS6_BF16) rc = bwd_dispatch<AXS6_BF16>(a, s, chunks, st);
        else rc = bwd_dispatch<AXS6_F16>(a, s, chunks, st);
        if (rc) return rc;
    }
    if (dgamma || dbeta) {
        ln_reduce_kernel<<<(unsigned)(2 * nb), kLnThreads, 0, st>>>(reinterpret_cast<const float*>(workspace),
                                                                    chunks, cols, dgamma, dbeta, nb);
    }
    return check_launch(fn);
}
