// Operand packing for the quantized linear (gfx950).
//
// The linear contracts fake-quantized operands on fp16 MFMA.  An NF5 value
// is +-lut[i] * 2^e1 with a per-block exponent, and fp16 has only a 5-bit
// exponent, so each operand row is scaled by an exact power of two 2^-S
// chosen so that the row's largest value lands at <= 2^15; the GEMM epilogue
// multiplies the exponents back.  Relative to the fp32 reference only the
// fp16 rounding of each NF5 value remains (11 significant bits), which keeps
// the GEMM within rel-L2 ~3e-4 of the fp32 product -- bf16 operands (8 bits)
// land at ~2.5e-3.
//
// Kernels:
//   pack_rows_kernel    one workgroup per row, the row held in registers:
//                       FQ + row scale in a single HBM pass (forward X, W;
//                       backward dY for dX with the weight's row exponents
//                       folded in per column).
//   pack_global_kernel  column strips, one tensor-wide scale (read from a
//                       device scalar): backward dY for dW, plus fixed-order
//                       column partial sums for the bias gradient.
//   transpose_f16_kernel / reduce_partials_kernel / init_gmax_kernel.
#include <limits.h>

#include "nf5_device.h"
#include "linear_internal.h"

namespace axs6 {
namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kPackThreads = 256;
constexpr int kF16MaxExp = 15;   // largest packed magnitude is <= 2^15

enum PackMode { kRaw = 0, kNearest = 1, kStochastic = 2 };

// Unsigned max over groups of g neighbouring lanes (g uniform at runtime).
__device__ __forceinline__ uint32_t group_umax_rt(uint32_t v, int g) {
    if (g >= 2) v = group_umax<2>(v) ;
    if (g >= 4) {
        uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x4E, 0xF, 0xF, false);
        v = v > o ? v : o;
    }
    if (g >= 8) {
        uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x141, 0xF, 0xF, false);
        v = v > o ? v : o;
    }
    return v;
}

__device__ __forceinline__ uint32_t group_umax_shfl_rt(uint32_t v, int bs) {
    for (int off = 1; off < bs; off <<= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = v > o ? v : o;
    }
    return v;
}

__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        int o = __shfl_xor(v, off, 64);
        v = v > o ? v : o;
    }
    return v;
}

template <int V>
__device__ __forceinline__ void store_f16(_Float16* p, const float* v, int sh_base, const int* sh_col) {
    uint16_t h[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
        const int sh = sh_base + (sh_col ? sh_col[e] : 0);
        h[e] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(v[e], sh));
    }
    if constexpr (V == 8) {
        u32x4 w;
        w.x = h[0] | ((uint32_t)h[1] << 16); w.y = h[2] | ((uint32_t)h[3] << 16);
        w.z = h[4] | ((uint32_t)h[5] << 16); w.w = h[6] | ((uint32_t)h[7] << 16);
        *reinterpret_cast<u32x4*>(p) = w;
    } else {
        u32x2 w;
        w.x = h[0] | ((uint32_t)h[1] << 16); w.y = h[2] | ((uint32_t)h[3] << 16);
        *reinterpret_cast<u32x2*>(p) = w;
    }
}

struct PackRowsK {
    const void* x; int64_t rows; int64_t cols; int block;
    uint64_t seed; uint64_t offset;
    const int32_t* colx;
    _Float16* out; int64_t ld_out; int64_t cols_pad;
    int32_t* s_out; int32_t* rmax_out;
    const int32_t* rowx; int32_t* gmax;
    const float* lut; const uint8_t* band;
};

template <int DT, int MODE, bool COLX, int NV>
__global__ __launch_bounds__(kPackThreads) void pack_rows_kernel(PackRowsK k, PackRowsK k2) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int V = E::V;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ int red[2][kPackThreads / 64];
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    // two operands may share one launch: workgroups past k.rows take k2
    const bool second = blockIdx.x >= k.rows;
    const PackRowsK q = second ? k2 : k;      // by value: field-wise selects, no stack copy
    const int tid = threadIdx.x;
    const int64_t r = second ? blockIdx.x - k.rows : blockIdx.x;
    const int64_t nvec = q.cols / V;
    const int g = q.block / V;
    const S* xr = reinterpret_cast<const S*>(q.x) + r * q.cols;

    // the row's HBM loads go out before the LUT is staged
    float f[NV][V];
    int eb[NV];
    u32x4 raw[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t vi = tid + (int64_t)kPackThreads * j;
        raw[j] = vi < nvec ? *(reinterpret_cast<const u32x4*>(xr) + vi) : u32x4{0u, 0u, 0u, 0u};
    }
    stage_tables(lut_s, band_w, q.lut, q.band);
    int tmax = INT_MIN, rmax = INT_MIN;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t vi = tid + (int64_t)kPackThreads * j;
        E::unpack(raw[j], f[j]);
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < V; ++e) {
            uint32_t a = __float_as_uint(f[j][e]) & 0x7fffffffu;
            m = m > a ? m : a;
        }
        m = group_umax_rt(m, g);
        const FqScale s = fq_scale(m, band_s);
        if constexpr (MODE != kRaw) {
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const float u = (MODE == kStochastic)
                    ? dither_uniform(q.seed, q.offset + (uint64_t)(r * q.cols + vi * V + e)) : 0.0f;
                f[j][e] = fq_value(f[j][e], s, lut_s, MODE == kStochastic, u);
            }
        }
        const bool finite_block = !(s.nan_block || s.inf_scale || m == 0u);
        eb[j] = (vi < nvec && finite_block) ? s.e1 : INT_MIN;
        rmax = eb[j] > rmax ? eb[j] : rmax;
        if constexpr (COLX) {
            if (eb[j] != INT_MIN) {
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const int b = eb[j] + q.colx[vi * V + e];
                    tmax = b > tmax ? b : tmax;
                }
            }
        }
    }
    if constexpr (!COLX) tmax = rmax;

    // workgroup max of (tmax, rmax)
    tmax = wave_max_i32(tmax);
    rmax = wave_max_i32(rmax);
    if ((tid & 63) == 0) { red[0][tid >> 6] = tmax; red[1][tid >> 6] = rmax; }
    __syncthreads();
    tmax = red[0][0]; rmax = red[1][0];
#pragma unroll
    for (int w = 1; w < kPackThreads / 64; ++w) {
        tmax = red[0][w] > tmax ? red[0][w] : tmax;
        rmax = red[1][w] > rmax ? red[1][w] : rmax;
    }
    const int S_row = (tmax == INT_MIN) ? 0 : tmax - kF16MaxExp;

    if (q.out) {
        _Float16* orow = q.out + r * q.ld_out;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = tid + (int64_t)kPackThreads * j;
            if (vi < nvec) {
                int colx_v[V];
                if constexpr (COLX) {
#pragma unroll
                    for (int e = 0; e < V; ++e) colx_v[e] = q.colx[vi * V + e];
                }
                store_f16<V>(orow + vi * V, f[j], -S_row, COLX ? colx_v : nullptr);
            }
        }
        const int64_t zvec = (q.cols_pad - q.cols) / 8;   // 8-half zero chunks
        for (int64_t z = tid; z < zvec; z += kPackThreads)
            *reinterpret_cast<u32x4*>(orow + q.cols + z * 8) = u32x4{0u, 0u, 0u, 0u};
    }
    if (tid == 0) {
        q.s_out[r] = S_row;
        if (q.rmax_out) q.rmax_out[r] = rmax;
        if (q.gmax && rmax != INT_MIN) atomicMax(q.gmax, rmax + (q.rowx ? q.rowx[r] : 0));
    }
}

struct PackGlobalK {
    const void* x; int64_t rows; int64_t cols; int block;
    uint64_t seed; uint64_t offset;
    const int32_t* rowx; const int32_t* gmax;
    _Float16* out; int64_t ld_out; int64_t cols_pad;
    float* partial; int rows_per_chunk;
    const float* lut; const uint8_t* band;
};

template <int DT, int MODE>
__global__ __launch_bounds__(kPackThreads) void pack_global_kernel(PackGlobalK k) {
    using E = Elem<DT>;
    using S = typename E::S;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    stage_tables(lut_s, band_w, k.lut, k.band);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int64_t c = (int64_t)blockIdx.x * kPackThreads + threadIdx.x;
    const bool vc = c < k.cols;
    const int64_t r0 = (int64_t)blockIdx.y * k.rows_per_chunk;
    const int64_t r1 = r0 + k.rows_per_chunk < k.rows ? r0 + k.rows_per_chunk : k.rows;
    const int gm = *k.gmax;
    const int G = (gm == INT_MIN) ? 0 : gm - kF16MaxExp;
    const S* xs = reinterpret_cast<const S*>(k.x);
    float colsum = 0.0f;
#pragma unroll 4
    for (int64_t r = r0; r < r1; ++r) {
        const int64_t gi = r * k.cols + c;
        float f = vc ? E::to_f(xs[gi]) : 0.0f;
        const uint32_t m = group_umax_shfl_rt(__float_as_uint(f) & 0x7fffffffu, k.block);
        if constexpr (MODE != kRaw) {
            const FqScale s = fq_scale(m, band_s);
            const float u = (MODE == kStochastic) ? dither_uniform(k.seed, k.offset + (uint64_t)gi) : 0.0f;
            f = fq_value(f, s, lut_s, MODE == kStochastic, u);
        }
        if (k.out && c < k.cols_pad) {
            const int sh = (k.rowx ? k.rowx[r] : 0) - G;
            k.out[r * k.ld_out + c] = vc ? (_Float16)__builtin_amdgcn_ldexpf(f, sh) : (_Float16)0.0f;
        }
        colsum += f;
    }
    if (k.partial && vc) k.partial[(int64_t)blockIdx.y * k.cols + c] = colsum;
}

__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ partial, int64_t chunks,
                                                              int64_t cols, float* __restrict__ out) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= cols) return;
    float s = 0.0f;
    for (int64_t k = 0; k < chunks; ++k) s += partial[k * cols + c];
    out[c] = s;
}

__global__ __launch_bounds__(256) void transpose_f16_kernel(const uint16_t* __restrict__ in, int64_t rows,
                                                            int64_t cols, int64_t ld_in, uint16_t* __restrict__ out,
                                                            int64_t out_rows, int64_t rows_pad, int64_t ld_out) {
    __shared__ uint16_t tile[64][66];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * 64;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int64_t r = r0 + ty + 4 * i, c = c0 + tx;
        tile[ty + 4 * i][tx] = (r < rows && c < cols) ? in[r * ld_in + c] : (uint16_t)0;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int64_t oc = c0 + ty + 4 * i, orr = r0 + tx;
        if (oc < out_rows && orr < rows_pad) out[oc * ld_out + orr] = tile[tx][ty + 4 * i];
    }
}

__global__ void init_gmax_kernel(int32_t* p) { *p = INT_MIN; }

template <int DT, int MODE, bool COLX>
void dispatch_rows_nv(const PackRowsK& k, const PackRowsK& k2, int64_t rows, int nv, hipStream_t st) {
    const dim3 grid((unsigned)rows);
    switch (nv) {
        case 1: pack_rows_kernel<DT, MODE, COLX, 1><<<grid, kPackThreads, 0, st>>>(k, k2); break;
        case 2: pack_rows_kernel<DT, MODE, COLX, 2><<<grid, kPackThreads, 0, st>>>(k, k2); break;
        case 4: pack_rows_kernel<DT, MODE, COLX, 4><<<grid, kPackThreads, 0, st>>>(k, k2); break;
        case 8: pack_rows_kernel<DT, MODE, COLX, 8><<<grid, kPackThreads, 0, st>>>(k, k2); break;
        default: pack_rows_kernel<DT, MODE, COLX, 16><<<grid, kPackThreads, 0, st>>>(k, k2); break;
    }
}

template <int DT>
void dispatch_rows(const PackRowsK& k, const PackRowsK& k2, int64_t rows, int mode, bool colx, int nv,
                   hipStream_t st) {
    if (mode == kRaw) {
        if (colx) dispatch_rows_nv<DT, kRaw, true>(k, k2, rows, nv, st); else dispatch_rows_nv<DT, kRaw, false>(k, k2, rows, nv, st);
    } else if (mode == kNearest) {
        if (colx) dispatch_rows_nv<DT, kNearest, true>(k, k2, rows, nv, st); else dispatch_rows_nv<DT, kNearest, false>(k, k2, rows, nv, st);
    } else {
        if (colx) dispatch_rows_nv<DT, kStochastic, true>(k, k2, rows, nv, st); else dispatch_rows_nv<DT, kStochastic, false>(k, k2, rows, nv, st);
    }
}

template <int DT>
void dispatch_global(const PackGlobalK& k, int mode, dim3 grid, hipStream_t st) {
    if (mode == kRaw) pack_global_kernel<DT, kRaw><<<grid, kPackThreads, 0, st>>>(k);
    else if (mode == kNearest) pack_global_kernel<DT, kNearest><<<grid, kPackThreads, 0, st>>>(k);
    else pack_global_kernel<DT, kStochastic><<<grid, kPackThreads, 0, st>>>(k);
}

constexpr int kGlobalRowsPerChunk = 64;

}  // namespace

int64_t pack_global_chunks(int64_t rows) { return (rows + kGlobalRowsPerChunk - 1) / kGlobalRowsPerChunk; }

namespace {

int check_pack_rows(const PackRowsArgs& a, int* nv_out) {
    const int V = a.dtype == AXS6_F32 ? 4 : 8;
    if (a.cols % a.block != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: cols (%lld) must be a multiple of block_size", (long long)a.cols);
    if ((uintptr_t)a.x % 16 != 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: input not 16-byte aligned");
    if (a.out && (a.ld_out % 8 != 0 || (uintptr_t)a.out % 16 != 0 || a.cols_pad % 8 != 0 || a.cols_pad < a.cols))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: output must be 16-byte aligned with padded width >= cols");
    const int64_t nvec = a.cols / V;
    const int64_t per = (nvec + kPackThreads - 1) / kPackThreads;
    if (per > 16)
        return fail(AXS6_ERR_UNSUPPORTED, "pack_rows: rows of %lld elements exceed the register-resident limit (%d)",
                    (long long)a.cols, 16 * kPackThreads * V);
    *nv_out = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
    return AXS6_OK;
}

PackRowsK to_kernel_args(const PackRowsArgs& a, const DeviceTables& t) {
    return PackRowsK{a.x, a.rows, a.cols, a.block, a.seed, a.offset, a.colx, a.out, a.ld_out, a.cols_pad,
                     a.s_out, a.rmax_out, a.rowx, a.gmax, t.lut, t.band};
}

int pack_mode(const PackRowsArgs& a) { return a.fake_quant ? (a.stochastic ? kStochastic : kNearest) : kRaw; }

}  // namespace

int launch_pack_rows(const PackRowsArgs& a, const DeviceTables& t, hipStream_t st) {
    int nv = 0;
    int rc = check_pack_rows(a, &nv);
    if (rc) return rc;
    if (a.rows == 0) return AXS6_OK;
    const PackRowsK k = to_kernel_args(a, t);
    const bool colx = a.colx != nullptr;
    if (a.dtype == AXS6_F32) dispatch_rows<AXS6_F32>(k, k, a.rows, pack_mode(a), colx, nv, st);
    else if (a.dtype == AXS6_BF16) dispatch_rows<AXS6_BF16>(k, k, a.rows, pack_mode(a), colx, nv, st);
    else dispatch_rows<AXS6_F16>(k, k, a.rows, pack_mode(a), colx, nv, st);
    return check_launch("pack_rows");
}

int launch_pack_rows2(const PackRowsArgs& a, const PackRowsArgs& b, const DeviceTables& t, hipStream_t st) {
    int nva = 0, nvb = 0;
    int rc = check_pack_rows(a, &nva);
    if (rc) return rc;
    if ((rc = check_pack_rows(b, &nvb))) return rc;
    const bool same = a.dtype == b.dtype && pack_mode(a) == pack_mode(b) && nva == nvb &&
                      (a.colx != nullptr) == (b.colx != nullptr);
    if (!same || a.rows == 0 || b.rows == 0) {
        if ((rc = launch_pack_rows(a, t, st))) return rc;
        return launch_pack_rows(b, t, st);
    }
    const PackRowsK ka = to_kernel_args(a, t), kb = to_kernel_args(b, t);
    const bool colx = a.colx != nullptr;
    const int64_t rows = a.rows + b.rows;
    if (a.dtype == AXS6_F32) dispatch_rows<AXS6_F32>(ka, kb, rows, pack_mode(a), colx, nva, st);
    else if (a.dtype == AXS6_BF16) dispatch_rows<AXS6_BF16>(ka, kb, rows, pack_mode(a), colx, nva, st);
    else dispatch_rows<AXS6_F16>(ka, kb, rows, pack_mode(a), colx, nva, st);
    return check_launch("pack_rows");
}

int launch_pack_global(const PackGlobalArgs& a, const DeviceTables& t, hipStream_t st) {
    if (a.cols % a.block != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_global: cols must be a multiple of block_size");
    if (a.rows == 0) return AXS6_OK;
    PackGlobalK k{a.x, a.rows, a.cols, a.block, a.seed, a.offset, a.rowx, a.gmax, a.out, a.ld_out,
                  a.out ? a.cols_pad : a.cols, a.partial, kGlobalRowsPerChunk, t.lut, t.band};
    const int64_t width = a.out ? a.cols_pad : a.cols;
    const dim3 grid((unsigned)((width + kPackThreads - 1) / kPackThreads), (unsigned)pack_global_chunks(a.rows));
    const int mode = a.fake_quant ? (a.stochastic ? kStochastic : kNearest) : kRaw;
    if (a.dtype == AXS6_F32) dispatch_global<AXS6_F32>(k, mode, grid, st);
    else if (a.dtype == AXS6_BF16) dispatch_global<AXS6_BF16>(k, mode, grid, st);
    else dispatch_global<AXS6_F16>(k, mode, grid, st);
    return check_launch("pack_global");
}

int launch_reduce_partials(const float* partial, int64_t chunks, int64_t cols, float* out, hipStream_t st) {
    if (cols == 0) return AXS6_OK;
    reduce_partials_kernel<<<dim3((unsigned)((cols + 255) / 256)), 256, 0, st>>>(partial, chunks, cols, out);
    return check_launch("reduce_partials");
}

int launch_transpose_f16(const _Float16* in, int64_t rows, int64_t cols, int64_t ld_in, _Float16* out,
                         int64_t out_rows, int64_t rows_pad, int64_t ld_out, hipStream_t st) {
    if (out_rows == 0 || rows_pad == 0) return AXS6_OK;
    const dim3 grid((unsigned)((out_rows + 63) / 64), (unsigned)((rows_pad + 63) / 64));
    transpose_f16_kernel<<<grid, 256, 0, st>>>(reinterpret_cast<const uint16_t*>(in), rows, cols, ld_in,
                                               reinterpret_cast<uint16_t*>(out), out_rows, rows_pad, ld_out);
    return check_launch("transpose_f16");
}

int launch_init_gmax(int32_t* p, hipStream_t st) {
    init_gmax_kernel<<<1, 1, 0, st>>>(p);
    return check_launch("init_gmax");
}

}  // namespace axs6
