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
// With bf16 or f16 inputs the FQ values are first rounded to that type, as
// the reference's fake-quantize returns them before its 16-bit F.linear; a
// bf16 or f16 value times a power of two is exact in fp16 (down to its
// subnormal range), so the contraction then sees the reference's operands.
//
// Kernels:
//   pack_rows_kernel    one workgroup per row, the row held in registers:
//                       FQ + row scale in a single HBM pass (forward X, W;
//                       backward dY for dX with the weight's row exponents
//                       folded in per column).
//   pack_t_kernel       64 x 64 tiles, one tensor-wide scale (read from a
//                       device scalar), written transposed: backward dY ->
//                       the dW operand [N, Mp] directly, plus fixed-order
//                       column partial sums for the bias gradient; and/or
//                       the row-major operand with row shifts computed
//                       beforehand (backward dY -> the dX operand; forward
//                       rows too long for pack_rows_kernel's registers).
//   stats_tile_kernel + stats_finalize_kernel
//                       row shifts and the tensor-wide exponent, streamed
//                       over 2-D tiles (the backward's dY).
//   stats_row_kernel    row shifts of rows too long for pack_rows_kernel,
//                       one workgroup streaming each row.
//   transpose_f16_kernel / reduce_partials_kernel / init_gmax_kernel.
#include <limits.h>

#include <type_traits>

#include "nf5_device.h"
#include "linear_internal.h"
#include "partials.h"

namespace axs6 {
namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kPackThreads = 256;
constexpr int kF16MaxExp = 15;   // largest packed magnitude is <= 2^15

enum PackMode { kRaw = 0, kNearest = 1, kStochastic = 2 };

// Unsigned max over groups of g neighbouring lanes (g uniform at runtime).
__device__ __forceinline__ uint32_t group_umax_rt(uint32_t v, int g) {
    if (g >= 2) v = dpp_umax<0xB1>(v);
    if (g >= 4) v = dpp_umax<0x4E>(v);
    if (g >= 8) v = dpp_umax<0x141>(v);
    return v;
}

__device__ __forceinline__ uint32_t group_umax_shfl_rt(uint32_t v, int bs) {
    for (int off = 1; off < bs; off <<= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = v > o ? v : o;
    }
    return v;
}

__device__ __forceinline__ int wave_max_i32(int v) { return wave_imax(v); }

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

// fp16 of v[e] * factor (factor a power of two), V halves stored as one vector.
template <int V>
__device__ __forceinline__ void store_f16_mul(_Float16* p, const float* v, float factor) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    uint32_t w[V / 2];
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
        const f32x2 x = {v[2 * i] * factor, v[2 * i + 1] * factor};
        w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
    }
    if constexpr (V == 8) {
        *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
        *reinterpret_cast<u32x2*>(p) = u32x2{w[0], w[1]};
    }
}

struct PackRowsK {
    const void* x; int64_t rows; int64_t cols; int block;
    uint64_t seed; const uint64_t* seed_dev; uint64_t offset;   // dither seed (+ *seed_dev when set)
    const int32_t* colx;
    _Float16* out; int64_t ld_out; int64_t cols_pad;
    int32_t* s_out; int32_t* rmax_out;
    const int32_t* rowx; int32_t* gmax;
    const float* lut; const uint8_t* band;
};

// Row pack: rows of the concatenation of k's rows and k2's (two operands in
// one launch; k2 == k and total == k.rows for one).  NT threads hold a row in
// registers, NV 16-byte vectors each (rows_shape picks NT and NV by row
// length).  A workgroup holds RPW row groups and handles rows RPW*w + g,
// RPW*(w + gridDim.x) + g, ...; with NT == 64 a row is one wave and its
// reductions need no barrier, so short rows run several to a workgroup
// (RPW > 1 requires NT == 64).  The LUT and band table are staged once per
// workgroup (NT * RPW >= 256 threads).
//
// The row index is wave-uniform (taken from the block index, or read from the
// first lane), so row addresses and the choice between k and k2 are scalar.
//
// DEFER (nearest FQ without column exponents, f32 or bf16 input -- the
// forward's packing): the FQ leaves +-lut[i] per element and the block
// exponent e1 per vector (fq_vector_unscaled), and the store multiplies by
// 2^(e1 - S_row) -- the block scale and the row shift in one exact product
// instead of a product and an ldexp.  For bf16 input the LUT is read rounded
// to bf16 (the reference's FQ output rounding, which commutes with 2^e1 on
// this path).  Vectors whose wave met a special block keep full FQ values
// and the ldexp store.
template <int DT, int MODE, bool COLX, int NV, int NT, int RPW>
__global__ __launch_bounds__(NT * RPW) void pack_rows_kernel(PackRowsK k, PackRowsK k2, int64_t total) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int V = E::V;
    constexpr int NW = NT / 64;
    constexpr bool WAVE_ROW = NT == 64;
    constexpr bool DEFER = MODE == kNearest && !COLX && DT != AXS6_F16;
    constexpr bool ROUNDED_LUT = DEFER && DT == AXS6_BF16;
    static_assert(RPW == 1 || WAVE_ROW, "several rows per workgroup need one wave per row");
    static_assert(NT * RPW >= kLutSize / 4 && NT * RPW >= kBandSize / 4, "table staging takes one thread per word");
    __shared__ float lut_s[kLutSize];
    __shared__ float lutr_s[ROUNDED_LUT ? kLutSize : 1];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ int red[2][2][NW];         // [row parity][tmax, rmax][wave]
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);
    const int tid = threadIdx.x % NT;     // thread within the row group
    if constexpr (ROUNDED_LUT) {
        if (threadIdx.x < kLutSize / 4) {
            const float4 v = reinterpret_cast<const float4*>(k.lut)[threadIdx.x];
            float4 r;
            r.x = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.x)); r.y = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.y));
            r.z = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.z)); r.w = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.w));
            reinterpret_cast<float4*>(lutr_s)[threadIdx.x] = r;
        }
    }
    stage_tables(lut_s, band_w, k.lut, k.band);
    const float* lut_fast = ROUNDED_LUT ? lutr_s : lut_s;

    // wave-uniform row group index within the workgroup
    const int64_t g0 = RPW == 1 ? 0 : (int64_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x / NT));
    const int64_t stride = (int64_t)gridDim.x * RPW;

    int parity = 0;
    for (int64_t R = (int64_t)blockIdx.x * RPW + g0; R < total; R += stride, parity ^= 1) {
        const bool second = R >= k.rows;
        const PackRowsK q = second ? k2 : k;      // by value: field-wise selects, no stack copy
        const uint64_t key = MODE == kStochastic ? dither_key(q.seed + (q.seed_dev ? *q.seed_dev : 0ull)) : 0ull;
        const int64_t r = second ? R - k.rows : R;
        const int64_t nvec = q.cols / V;
        const int g = q.block / V;
        const S* xr = reinterpret_cast<const S*>(q.x) + r * q.cols;

        float f[NV][V];
        int cx[NV][V];
        int e1v[NV];          // DEFER: the vector's block exponent, or INT_MIN when f holds full FQ values
        u32x4 raw[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = tid + (int64_t)NT * j;
            raw[j] = vi < nvec ? *(reinterpret_cast<const u32x4*>(xr) + vi) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = tid + (int64_t)NT * j;
            if constexpr (COLX) {
                // V consecutive column exponents: one or two 16-byte loads
#pragma unroll
                for (int h = 0; h < V / 4; ++h) {
                    const u32x4 c4 = vi < nvec ? *(reinterpret_cast<const u32x4*>(q.colx + vi * V) + h)
                                               : u32x4{0u, 0u, 0u, 0u};
                    cx[j][4 * h] = (int)c4.x; cx[j][4 * h + 1] = (int)c4.y;
                    cx[j][4 * h + 2] = (int)c4.z; cx[j][4 * h + 3] = (int)c4.w;
                }
            }
        }
        int tmax = INT_MIN, rmax = INT_MIN;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t vi = tid + (int64_t)NT * j;
            E::unpack(raw[j], f[j]);
            uint32_t m = 0;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                uint32_t a = __float_as_uint(f[j][e]) & 0x7fffffffu;
                m = m > a ? m : a;
            }
            m = group_umax_rt(m, g);
            const FqScale s = fq_scale(m, band_s);
            if constexpr (DEFER) {
                const bool full = fq_vector_unscaled<V>(f[j], s, lut_s, lut_fast);
                if (full) round_to_elem<DT>(f[j]);
                e1v[j] = full ? INT_MIN : s.e1;
            } else if constexpr (MODE != kRaw) {
                const DitherVec dv = dither_vec(key, q.offset + (uint64_t)(r * q.cols + vi * V));
                float d[V];
#pragma unroll
                for (int e = 0; e < V; ++e) d[e] = (MODE == kStochastic) ? dither_step(dv, e) : 0.0f;
                fq_vector<V>(f[j], s, lut_s, MODE == kStochastic, d);
                round_to_elem<DT>(f[j]);
            }
            const bool finite_block = !(s.nan_block || s.inf_scale || m == 0u);
            const int eb = (vi < nvec && finite_block) ? s.e1 : INT_MIN;
            rmax = eb > rmax ? eb : rmax;
            if constexpr (COLX) {
                if (eb != INT_MIN) {
#pragma unroll
                    for (int e = 0; e < V; ++e) {
                        const int b = eb + cx[j][e];
                        tmax = b > tmax ? b : tmax;
                    }
                }
            }
        }
        if constexpr (!COLX) tmax = rmax;

        // row max of (tmax, rmax); across waves, the parity buffer lets the
        // next row's writes proceed while slower waves still read this row's
        tmax = wave_max_i32(tmax);
        rmax = COLX ? wave_max_i32(rmax) : tmax;
        if constexpr (!WAVE_ROW) {
            if ((tid & 63) == 0) { red[parity][0][tid >> 6] = tmax; red[parity][1][tid >> 6] = rmax; }
            __syncthreads();
            tmax = red[parity][0][0]; rmax = red[parity][1][0];
#pragma unroll
            for (int w = 1; w < NW; ++w) {
                tmax = red[parity][0][w] > tmax ? red[parity][0][w] : tmax;
                rmax = red[parity][1][w] > rmax ? red[parity][1][w] : rmax;
            }
        }
        const int S_row = (tmax == INT_MIN) ? 0 : tmax - kF16MaxExp;

        if (q.out) {
            _Float16* orow = q.out + r * q.ld_out;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int64_t vi = tid + (int64_t)NT * j;
                if (vi < nvec) {
                    if constexpr (DEFER) {
                        // e1v[j] <= row max, so 2^(e1 - S_row) <= 2^15: finite; below 2^-149 it is 0,
                        // as is the fp16 value of anything that small
                        if (e1v[j] != INT_MIN) store_f16_mul<V>(orow + vi * V, f[j], __builtin_amdgcn_ldexpf(1.0f, e1v[j] - S_row));
                        else store_f16<V>(orow + vi * V, f[j], -S_row, nullptr);
                    } else {
                        store_f16<V>(orow + vi * V, f[j], -S_row, COLX ? cx[j] : nullptr);
                    }
                }
            }
            // zeros up to cols_pad: a 4-half chunk first when cols % 8 == 4
            // (f32 rows of 4k + 4 values), then 8-half (16-byte) chunks
            int64_t zc = q.cols;
            if ((q.cols_pad - zc) % 8 != 0) {
                if (tid == 0) *reinterpret_cast<uint2*>(orow + zc) = uint2{0u, 0u};
                zc += 4;
            }
            const int64_t zvec = (q.cols_pad - zc) / 8;
            for (int64_t z = tid; z < zvec; z += NT)
                *reinterpret_cast<u32x4*>(orow + zc + z * 8) = u32x4{0u, 0u, 0u, 0u};
        }
        if (tid == 0) {
            q.s_out[r] = S_row;
            if (q.rmax_out) q.rmax_out[r] = rmax;
            if (q.gmax && rmax != INT_MIN) atomicMax(q.gmax, rmax + (q.rowx ? q.rowx[r] : 0));
        }
    }
}

// Transposed global pack: one workgroup per 64 x 64 tile of x (rows r, columns
// c).  Loads are 16-byte vectors along the rows, so an NF5 block is G = block/V
// neighbouring lanes and its amax is a DPP reduction; the value of element
// (r, c) is FQ(x)[r, c] with the same dither counter as the row pack, scaled
// by 2^(rowx[r] - G) (G = *gmax - 15) and written transposed through LDS:
// out[c, r] (ld_out halves per row, r up to the tile end: zeros past rows).
// With `partial`, the tile's column sums of FQ(x) go to partial[tile_row, c],
// summed in a fixed order (each thread over its rows in order, then the
// row groups in order), so the bias gradient is deterministic.
struct PackTK {
    const void* x; int64_t rows; int64_t cols; int block;
    uint64_t seed; const uint64_t* seed_dev; uint64_t offset;
    const int32_t* rowx; const int32_t* gmax;
    _Float16* out; int64_t ld_out;
    _Float16* out_r; int64_t ld_r; const int32_t* colx_r; const int32_t* shift_r;
    float* partial;
    const float* lut; const uint8_t* band;
    // with gtile: the tensor-wide maximum is folded here from the statistics
    // pass's per-band maxima (instead of read from gmax) and written to gmax_out
    const int32_t* gtile; int64_t ngtile; int32_t* gmax_out;
};

constexpr int kTile = 64;          // rows and columns of a transpose tile
constexpr int kTileLd = kTile + 8; // LDS row stride (halves) of the transposed tile

// C32: every dither counter offset .. offset + rows*cols - 1 has the same high
// word (the common case), so the draw needs only the 32-bit low word.
// One 64 x 64 tile per workgroup (tile blockIdx.x, column tiles fastest): its
// loads -- the tile of x, the column exponents and the rows' shifts -- go out
// first, so their latency overlaps the staging of the tables and the fold of
// the tensor-wide maximum.  Tiles wholly inside x (all but the last row band
// and column tile) skip the bounds tests; both forms compute the same values.
template <int DT, int MODE, int BS, bool C32>
__global__ __launch_bounds__(kPackThreads) void pack_t_kernel(PackTK k, int64_t ntx, int64_t ntiles) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int V = E::V;
    constexpr int GL = BS / V > 0 ? BS / V : 1;     // lanes per NF5 block
    constexpr int TPR = kTile / V;                  // threads per tile row
    constexpr int RPP = kPackThreads / TPR;         // tile rows per pass
    constexpr int PASSES = kTile / RPP;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ uint16_t tile[kTile * kTileLd];      // transposed: tile[c * kTileLd + r]
    __shared__ float csum[RPP][kTile + 1];
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int tid = threadIdx.x;
    const int tc = tid % TPR, tr = tid / TPR;
    const int64_t t = blockIdx.x;
    if (t >= ntiles) return;   // workgroup-uniform (the grid is the tile count)
    const int64_t ty = t / ntx, tx = t - ty * ntx;
    const bool full = (ty + 1) * kTile <= k.rows && (tx + 1) * kTile <= k.cols;   // workgroup-uniform
    const int64_t c0 = tx * kTile, r0 = ty * kTile;
    const int64_t c = c0 + tc * V;
    const bool cin = full || c < k.cols;            // cols % V == 0: vectors are whole
    const int64_t rt = r0 + tr;                     // this thread's row in pass 0
    const S* xp = reinterpret_cast<const S*>(k.x) + rt * k.cols + c;
    const int64_t x_pass = (int64_t)RPP * k.cols;

    // ---- the tile's loads ----
    u32x4 raw[PASSES];
    if (full) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) raw[p] = *reinterpret_cast<const u32x4*>(xp + p * x_pass);
    } else {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int64_t r = rt + RPP * p;
            raw[p] = (cin && r < k.rows) ? *reinterpret_cast<const u32x4*>(xp + p * x_pass) : u32x4{0u, 0u, 0u, 0u};
        }
    }
    // the column exponents of this thread's V columns, the rows' shifts and exponents
    int cx[V];
#pragma unroll
    for (int e = 0; e < V; ++e) cx[e] = 0;
    if (k.out_r && cin && k.colx_r) {
#pragma unroll
        for (int h = 0; h < V / 4; ++h) {
            const u32x4 c4 = *(reinterpret_cast<const u32x4*>(k.colx_r + c) + h);
            cx[4 * h] = (int)c4.x; cx[4 * h + 1] = (int)c4.y; cx[4 * h + 2] = (int)c4.z; cx[4 * h + 3] = (int)c4.w;
        }
    }
    int shr[PASSES], rxv[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int64_t r = rt + RPP * p;
        const bool rin = full || r < k.rows;
        shr[p] = (k.out_r && rin) ? k.shift_r[r] : 0;
        rxv[p] = (k.rowx && cin && rin) ? k.rowx[r] : INT_MIN;
    }

    // ---- tables and the tensor-wide maximum ----
    const uint64_t key = MODE == kStochastic ? dither_key(k.seed + (k.seed_dev ? *k.seed_dev : 0ull)) : 0ull;
    int gm = INT_MIN;
    if (k.gtile) {
        __shared__ int gred[kPackThreads / 64];
        for (int64_t i = tid; i < k.ngtile; i += kPackThreads) gm = max(gm, k.gtile[i]);
        gm = wave_max_i32(gm);
        if ((tid & 63) == 0) gred[tid >> 6] = gm;
        stage_tables(lut_s, band_w, k.lut, k.band);   // its barrier publishes gred
#pragma unroll
        for (int w = 0; w < kPackThreads / 64; ++w) gm = max(gm, gred[w]);
        if (blockIdx.x == 0 && tid == 0 && k.gmax_out) *k.gmax_out = gm;
    } else {
        stage_tables(lut_s, band_w, k.lut, k.band);
        if (k.gmax) gm = *k.gmax;
    }
    const int G = (gm == INT_MIN) ? 0 : gm - kF16MaxExp;
    int shx[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) shx[p] = rxv[p] == INT_MIN ? -G : rxv[p] - G;

    // ---- FQ and the two operands ----
    const uint32_t kh = (uint32_t)key ^ ((uint32_t)(k.offset >> 32) * 0x9E3779B9u + (uint32_t)(key >> 32));
    auto tile_body = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        // dither counters offset + r * cols + c (low words: pass p adds p * RPP * cols)
        const uint32_t lo0 = (uint32_t)k.offset + (uint32_t)rt * (uint32_t)k.cols + (uint32_t)c;
        const uint32_t lo_pass = (uint32_t)RPP * (uint32_t)k.cols;
        _Float16* orow = k.out_r ? k.out_r + rt * k.ld_r + c : nullptr;
        const int64_t o_pass = (int64_t)RPP * k.ld_r;
        float colsum[V];
#pragma unroll
        for (int e = 0; e < V; ++e) colsum[e] = 0.0f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int lr = tr + RPP * p;
            const int64_t r = r0 + lr;
            float f[V];
            E::unpack(raw[p], f);
            uint32_t m = 0;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
                m = m > a ? m : a;
            }
            m = group_umax<GL>(m);
            if constexpr (MODE != kRaw) {
                const FqScale s = fq_scale(m, band_s);
                float d[V];
                if constexpr (MODE == kStochastic && C32) {
                    const uint32_t lo = lo0 + (uint32_t)p * lo_pass;
#pragma unroll
                    for (int e = 0; e < V; ++e) d[e] = dither_step32(lo + (uint32_t)e, kh);
                } else if constexpr (MODE == kStochastic) {
                    const DitherVec dv = dither_vec(key, k.offset + (uint64_t)(r * k.cols + c));
#pragma unroll
                    for (int e = 0; e < V; ++e) d[e] = dither_step(dv, e);
                } else {
#pragma unroll
                    for (int e = 0; e < V; ++e) d[e] = 0.0f;
                }
                fq_vector<V>(f, s, lut_s, MODE == kStochastic, d);
                round_to_elem<DT>(f);
            }
            const bool live = FULL || (cin && r < k.rows);
            if (k.partial) {
#pragma unroll
                for (int e = 0; e < V; ++e) colsum[e] += live ? f[e] : 0.0f;
            }
            if (k.out_r && (FULL || r < k.rows)) {
                // row-major operand: fp16(v * 2^(colx[c] - shift[r])), zeros in the
                // padding columns cols <= c < 64 * ceil(cols / 64)
                float z[V];
#pragma unroll
                for (int e = 0; e < V; ++e) z[e] = cin ? f[e] : 0.0f;
                store_f16<V>(orow + p * o_pass, z, -shr[p], cx);
            }
            if (k.out) {
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const _Float16 h = live ? (_Float16)__builtin_amdgcn_ldexpf(f[e], shx[p]) : (_Float16)0.0f;
                    tile[(tc * V + e) * kTileLd + lr] = __builtin_bit_cast(uint16_t, h);
                }
            }
        }
        if (k.partial) {
#pragma unroll
            for (int e = 0; e < V; ++e) csum[tr][tc * V + e] = colsum[e];
        }
        __syncthreads();
        if (k.partial && tid < kTile && (FULL || c0 + tid < k.cols)) {
            float sum = 0.0f;
            for (int q = 0; q < RPP; ++q) sum += csum[q][tid];
            k.partial[ty * k.cols + c0 + tid] = sum;
        }
        if (k.out) {
            // 64 output rows (columns c of x) of 64 halves = 8 chunks of 16 bytes each
#pragma unroll
            for (int q = tid; q < kTile * 8; q += kPackThreads) {
                const int oc = q >> 3, j = q & 7;
                if (FULL || c0 + oc < k.cols)
                    *reinterpret_cast<u32x4*>(k.out + (c0 + oc) * k.ld_out + r0 + j * 8) =
                        *reinterpret_cast<const u32x4*>(&tile[oc * kTileLd + j * 8]);
            }
        }
    };
    if (full) tile_body(std::true_type{});
    else tile_body(std::false_type{});
}

// Rows longer than pack_rows_kernel holds in registers take two launches: this
// kernel, one workgroup per row streaming it (U 16-byte vectors in flight per
// thread), writes what pack_rows writes besides the packed values -- s_out,
// rmax_out, gmax -- and the zero columns of `out` from 64 * ceil(cols / 64) to
// cols_pad; then pack_t_kernel writes the row-major operand (values and the
// zero columns up to 64 * ceil(cols / 64)) with these shifts.  The shift rule
// is pack_rows_kernel's: S = max over the row's finite nonzero blocks of
// (e1 + colx[c]) - 15, 0 if there is none.
template <int DT, int BS>
__global__ __launch_bounds__(256) void stats_row_kernel(PackRowsK k) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int V = E::V;
    constexpr int G = BS / V > 0 ? BS / V : 1;     // lanes per NF5 block
    constexpr int U = 4;
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ int red[2][4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < kBandSize / 4) band_w[tid] = reinterpret_cast<const uint32_t*>(k.band)[tid];
    __syncthreads();
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);
    const int64_t r = blockIdx.x;
    const int64_t nvec = k.cols / V;
    const u32x4* xr = reinterpret_cast<const u32x4*>(reinterpret_cast<const S*>(k.x) + r * k.cols);

    int tm = INT_MIN, rm = INT_MIN;
    for (int64_t v0 = 0; v0 < nvec; v0 += 256 * U) {
        u32x4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t vi = v0 + u * 256 + tid;
            raw[u] = vi < nvec ? xr[vi] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t vi = v0 + u * 256 + tid;
            float f[V];
            E::unpack(raw[u], f);
            uint32_t m = 0;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
                m = m > a ? m : a;
            }
            // a block is G whole vectors at a multiple of G, so its lanes are
            // all inside the row or all past its end
            m = group_umax<G>(m);
            const FqScale s = fq_scale(m, band_s);
            if (vi < nvec && !(s.nan_block || s.inf_scale || m == 0u)) {
                rm = s.e1 > rm ? s.e1 : rm;
                int cm = 0;
                if (k.colx) {
                    cm = INT_MIN;
#pragma unroll
                    for (int h = 0; h < V / 4; ++h) {
                        const u32x4 c4 = *(reinterpret_cast<const u32x4*>(k.colx + vi * V) + h);
                        const int a = (int)c4.x > (int)c4.y ? (int)c4.x : (int)c4.y;
                        const int b = (int)c4.z > (int)c4.w ? (int)c4.z : (int)c4.w;
                        const int ab = a > b ? a : b;
                        cm = ab > cm ? ab : cm;
                    }
                }
                const int t = s.e1 + cm;
                tm = t > tm ? t : tm;
            }
        }
    }
    tm = wave_max_i32(tm);
    rm = wave_max_i32(rm);
    if (lane == 0) { red[0][wave] = tm; red[1][wave] = rm; }
    if (k.out) {
        _Float16* orow = k.out + r * k.ld_out;
        const int64_t z0 = ((k.cols + kTile - 1) / kTile) * kTile / 8, z1 = k.cols_pad / 8;   // 8-half chunks
        for (int64_t z = z0 + tid; z < z1; z += 256) *reinterpret_cast<u32x4*>(orow + z * 8) = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    if (tid == 0) {
        tm = red[0][0]; rm = red[1][0];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            tm = red[0][w] > tm ? red[0][w] : tm;
            rm = red[1][w] > rm ? red[1][w] : rm;
        }
        k.s_out[r] = tm == INT_MIN ? 0 : tm - kF16MaxExp;
        if (k.rmax_out) k.rmax_out[r] = rm;
        if (k.gmax && rm != INT_MIN) atomicMax(k.gmax, rm + (k.rowx ? k.rowx[r] : 0));
    }
}

// Row statistics of x for the packing shifts (block exponents only, no FQ
// values), streamed over tiles of RPP*PASSES rows x 256 columns.  For the
// blocks with a finite nonzero scale 2^e1 (every FQ value of the block is at
// most 2^e1 in magnitude) the workgroup of column tile tx writes, per row,
//   tmax[tx][r] = max over its blocks of (e1 + max colx over the block's columns)
//   rmax[tx][r] = max over its blocks of e1
// (INT_MIN when no block qualifies); stats_finalize_kernel folds the column
// tiles in order and writes shift[r] = max_tx tmax - 15 (0 if INT_MIN) and
// atomicMax(gmax, max_tx rmax + rowx[r]).  These are the quantities pack_rows
// derives for a whole row in one workgroup; a row-per-workgroup pass over
// long rows is latency-bound, this one streams.  Plain stores of per-tile
// maxima, not atomics on a zeroed array: no initialising launch.
//
// Rows of at most kStatsCols columns are one tile per row band (FINAL): the
// workgroup then holds whole rows and writes shift[r] itself, and for the
// tensor-wide shift gtile[band] = max over its rows of (max block e1 +
// rowx[r]) -- folded by the packing pass (pack_t) into gmax, so no folding
// launch runs (8192 x 256 f32 forward + backward 50.8 -> 48.3 us).  Wider rows
// in one tile per band were slower: 1024-column tiles leave too few
// workgroups (8192 x 1024: 90.0 -> 91.5 us, 2048 x 768: 93.1 -> 97.2 us).
struct StatsK {
    const void* x; int64_t rows; int64_t cols;
    const int32_t* colx; int32_t* tmax; int32_t* rmax;   // [ntx][rows] each
    const uint8_t* band; int32_t* gmax;                  // gmax set to INT_MIN by workgroup 0
    int32_t* shift; const int32_t* rowx; int32_t* gtile; // FINAL: per-row shifts, per-band maxima
};

constexpr int kStatsCols = 256;   // columns of a statistics tile

// Statistics tile `bid`; band_w: LDS for the band table, gred: 4 ints of LDS.
template <int DT, int BS, int PASSES, bool FINAL>
__device__ __forceinline__ void stats_tile_body(const StatsK& k, int64_t ntx, int64_t bid, uint32_t* band_w,
                                                int* gred) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int V = E::V;
    constexpr int G = BS / V > 0 ? BS / V : 1;
    constexpr int TPR = kTile / V;                  // threads per 64-column chunk of a row
    constexpr int RPP = 256 / TPR;                  // rows per pass
    constexpr int CH = kStatsCols / kTile;          // 64-column chunks per tile
    const int tid = threadIdx.x;
    if (tid < kBandSize / 4) band_w[tid] = reinterpret_cast<const uint32_t*>(k.band)[tid];
    const int tc = tid % TPR, tr = tid / TPR;
    const int64_t ty = bid / ntx, tx = bid - ty * ntx;
    const int64_t r0 = ty * (RPP * PASSES), c0 = tx * kStatsCols;
    if (!FINAL && bid == 0 && tid == 0 && k.gmax) *k.gmax = INT_MIN;
    const S* xs = reinterpret_cast<const S*>(k.x);

    u32x4 raw[PASSES][CH];
    int cm[CH];
#pragma unroll
    for (int h = 0; h < CH; ++h) {
        const int64_t c = c0 + h * kTile + tc * V;
        const bool cin = c < k.cols;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int64_t r = r0 + tr + RPP * p;
            raw[p][h] = (cin && r < k.rows) ? *reinterpret_cast<const u32x4*>(xs + r * k.cols + c)
                                            : u32x4{0u, 0u, 0u, 0u};
        }
        int m = INT_MIN;
        if (cin && k.colx) {
#pragma unroll
            for (int q = 0; q < V / 4; ++q) {
                const u32x4 c4 = *(reinterpret_cast<const u32x4*>(k.colx + c) + q);
                const int a = (int)c4.x > (int)c4.y ? (int)c4.x : (int)c4.y;
                const int b = (int)c4.z > (int)c4.w ? (int)c4.z : (int)c4.w;
                const int ab = a > b ? a : b;
                m = ab > m ? ab : m;
            }
        } else if (cin) {
            m = 0;
        }
        cm[h] = m;
    }
    __syncthreads();
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);
    int gband = INT_MIN;   // FINAL: max over this thread's rows of (max e1 + rowx)
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int64_t r = r0 + tr + RPP * p;
        int tm = INT_MIN, rm = INT_MIN;
#pragma unroll
        for (int h = 0; h < CH; ++h) {
            float f[V];
            E::unpack(raw[p][h], f);
            uint32_t a = 0;
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const uint32_t b = __float_as_uint(f[e]) & 0x7fffffffu;
                a = a > b ? a : b;
            }
            a = group_umax<G>(a);
            const FqScale s = fq_scale(a, band_s);
            if (!(s.nan_block || s.inf_scale || a == 0u) && cm[h] != INT_MIN) {
                rm = s.e1 > rm ? s.e1 : rm;
                const int t = s.e1 + cm[h];
                tm = t > tm ? t : tm;
            }
        }
        // max over the TPR lanes of this row (consecutive lanes)
#pragma unroll
        for (int off = 1; off < TPR; off <<= 1) {
            const int o1 = __shfl_xor(tm, off, 64), o2 = __shfl_xor(rm, off, 64);
            tm = o1 > tm ? o1 : tm;
            rm = o2 > rm ? o2 : rm;
        }
        if (tc == 0 && r < k.rows) {
            if constexpr (FINAL) {
                if (k.shift) k.shift[r] = tm == INT_MIN ? 0 : tm - kF16MaxExp;
                if (rm != INT_MIN) gband = max(gband, rm + (k.rowx ? k.rowx[r] : 0));
            } else {
                k.tmax[tx * k.rows + r] = tm;
                k.rmax[tx * k.rows + r] = rm;
            }
        }
    }
    if constexpr (FINAL) {
        if (k.gtile) {
            gband = wave_max_i32(gband);
            if ((tid & 63) == 0) gred[tid >> 6] = gband;
            __syncthreads();
            if (tid == 0) k.gtile[bid] = max(max(gred[0], gred[1]), max(gred[2], gred[3]));
        }
    }
}

template <int DT, int BS, int PASSES, bool FINAL = false>
__global__ __launch_bounds__(256) void stats_tile_kernel(StatsK k, int64_t ntx) {
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ int gred[4];
    stats_tile_body<DT, BS, PASSES, FINAL>(k, ntx, blockIdx.x, band_w, gred);
}

// A workgroup folds 64 rows: wave w takes the column tiles w, w + 4, ...
// (eight loads in flight per lane), the four waves meet in LDS.
constexpr int kFinRows = 64;

__global__ __launch_bounds__(256) void stats_finalize_kernel(const int32_t* __restrict__ tmax,
                                                             const int32_t* __restrict__ rmax, int64_t rows,
                                                             int64_t ntx, int32_t* shift, const int32_t* rowx,
                                                             int32_t* gmax) {
    __shared__ int part[2][4][kFinRows];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t r = (int64_t)blockIdx.x * kFinRows + lane;
    int t = INT_MIN, rm = INT_MIN;
    if (r < rows) {
        int64_t x = w;
        for (; x + 28 < ntx; x += 32) {
            int a[8], b[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) { a[u] = tmax[(x + 4 * u) * rows + r]; b[u] = rmax[(x + 4 * u) * rows + r]; }
#pragma unroll
            for (int u = 0; u < 8; ++u) { t = a[u] > t ? a[u] : t; rm = b[u] > rm ? b[u] : rm; }
        }
        for (; x < ntx; x += 4) {
            const int a = tmax[x * rows + r], b = rmax[x * rows + r];
            t = a > t ? a : t;
            rm = b > rm ? b : rm;
        }
    }
    part[0][w][lane] = t;
    part[1][w][lane] = rm;
    __syncthreads();
    if (w != 0) return;
    int g = INT_MIN;
    if (r < rows) {
#pragma unroll
        for (int v = 1; v < 4; ++v) {
            t = part[0][v][lane] > t ? part[0][v][lane] : t;
            rm = part[1][v][lane] > rm ? part[1][v][lane] : rm;
        }
        if (shift) shift[r] = t == INT_MIN ? 0 : t - kF16MaxExp;
        if (rm != INT_MIN) g = rm + (rowx ? rowx[r] : 0);
    }
    if (gmax) {
        g = wave_max_i32(g);
        if (lane == 0 && g != INT_MIN) atomicMax(gmax, g);
    }
}

// out[c] = sum over chunks k of partial[k, c], in the order k = 0, 1, ...
// split into 4 consecutive ranges combined in order: deterministic.
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ partial, int64_t chunks,
                                                              int64_t cols, float* __restrict__ out) {
    reduce_partials_block(partial, chunks, cols, out, blockIdx.x);
}

// out[c, r] = in[r, c] for r < rows, c < out_rows; zero for rows <= r < rows_pad.
// 64 x 64 tiles; 16-byte loads along input rows, 16-byte stores along output
// rows, the transpose done through LDS with 2-byte accesses.  One launch
// serves two independent transposes: blockIdx.y below ny0 tiles the first,
// the next ny1 rows the second (the backward's two operands; one launch
// less); rows past those, when red.blocks > 0, run the bias-gradient
// reduction (reduce_partials_block), block (y - ny0 - ny1) * gridDim.x + x.
struct ReduceJob { const float* partial; int64_t chunks; int64_t cols; float* out; int64_t blocks; };

__global__ __launch_bounds__(256) void transpose_f16_kernel(TransposeF16 j0, TransposeF16 j1, int ny0, int ny1,
                                                            ReduceJob red) {
    if ((int)blockIdx.y >= ny0 + ny1) {      // uniform per workgroup
        const int64_t rb = (int64_t)(blockIdx.y - ny0 - ny1) * gridDim.x + blockIdx.x;
        if (rb < red.blocks) reduce_partials_block(red.partial, red.chunks, red.cols, red.out, rb);
        return;
    }
    const bool second = (int)blockIdx.y >= ny0;
    const TransposeF16 j = second ? j1 : j0;
    const uint16_t* __restrict__ in = reinterpret_cast<const uint16_t*>(j.in);
    uint16_t* __restrict__ out = reinterpret_cast<uint16_t*>(j.out);
    const int64_t rows = j.rows, cols = j.cols, ld_in = j.ld_in, out_rows = j.out_rows, rows_pad = j.rows_pad,
                  ld_out = j.ld_out;
    __shared__ uint16_t tile[kTile * kTileLd];   // tile[c * kTileLd + r]
    const int tid = threadIdx.x;
    const int64_t c0 = (int64_t)blockIdx.x * kTile, r0 = (int64_t)(second ? blockIdx.y - ny0 : blockIdx.y) * kTile;
    const bool vec_in = (ld_in % 8 == 0) && ((uintptr_t)in % 16 == 0);
#pragma unroll
    for (int q = tid; q < kTile * 8; q += 256) {
        const int lr = q >> 3, j = q & 7;
        const int64_t r = r0 + lr, cb = c0 + j * 8;
        uint16_t h[8];
        if (r < rows && vec_in && cb + 8 <= cols) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(in + r * ld_in + cb);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) { h[2 * e] = (uint16_t)(ww[e] & 0xffffu); h[2 * e + 1] = (uint16_t)(ww[e] >> 16); }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (r < rows && cb + e < cols) ? in[r * ld_in + cb + e] : (uint16_t)0;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) tile[(j * 8 + e) * kTileLd + lr] = h[e];
    }
    __syncthreads();
    const bool vec_out = (ld_out % 8 == 0) && ((uintptr_t)out % 16 == 0);
#pragma unroll
    for (int q = tid; q < kTile * 8; q += 256) {
        const int oc = q >> 3, j = q & 7;
        const int64_t orow = c0 + oc, ocol = r0 + j * 8;
        if (orow >= out_rows) continue;
        const uint16_t* src = &tile[oc * kTileLd + j * 8];
        if (vec_out && ocol + 8 <= rows_pad) {
            *reinterpret_cast<u32x4*>(out + orow * ld_out + ocol) = *reinterpret_cast<const u32x4*>(src);
        } else {
            for (int e = 0; e < 8; ++e)
                if (ocol + e < rows_pad) out[orow * ld_out + ocol + e] = src[e];
        }
    }
}

// The same transposes in 128 x 128 tiles when every row and pointer is
// 16-byte aligned and the zero-padded width rows_pad a multiple of 8 (the
// backward's operands): a thread loads an 8 x 8 block (eight 16-byte row
// segments), transposes it in registers (v_perm_b32 pairs halves of two rows:
// 32 per block), and writes its 8 columns as 16-byte LDS chunks; the output
// rows are then stored as 16-byte chunks.  The LDS tile has no padding: the
// 16-byte chunk k of tile row oc sits at chunk k ^ ((oc >> 3) & 15), so the
// 16 lanes of a ds_write_b128 or ds_read_b128 group (one 8-row block each,
// or 16 chunks of one row) reach 16 distinct bank quads.  Against the 64 x 64
// kernel's 2-byte LDS writes: 8 LDS writes per 64 values instead of 64.
constexpr int kT128 = 128;

__device__ __forceinline__ int t128_slot(int oc, int k) { return oc * (kT128 / 8) + (k ^ ((oc >> 3) & 15)); }

// Tile (bx, by) of the 128 x 128 transposes; tile: kT128 * kT128 / 8 chunks of LDS.
__device__ __forceinline__ void transpose128_body(const TransposeF16& j0, const TransposeF16& j1, int ny0, int bx,
                                                  int by, u32x4* tile) {
    const bool second = by >= ny0;
    const TransposeF16 j = second ? j1 : j0;
    const uint16_t* __restrict__ in = reinterpret_cast<const uint16_t*>(j.in);
    uint16_t* __restrict__ out = reinterpret_cast<uint16_t*>(j.out);
    const int tid = threadIdx.x;
    const int64_t c0 = (int64_t)bx * kT128, r0 = (int64_t)(second ? by - ny0 : by) * kT128;
    const int br = tid >> 4, bc = tid & 15;      // this thread's 8 x 8 block
    const int64_t r = r0 + 8 * br, c = c0 + 8 * bc;
    uint32_t w[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (r + i < j.rows && c < j.cols) v = *reinterpret_cast<const u32x4*>(in + (r + i) * j.ld_in + c);
        w[i][0] = v.x; w[i][1] = v.y; w[i][2] = v.z; w[i][3] = v.w;
    }
    // column e of the block = rows 0..7 of input column c + e: dword d pairs rows 2d, 2d + 1
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        u32x4 o;
        o.x = __builtin_amdgcn_perm(w[1][e >> 1], w[0][e >> 1], sel);
        o.y = __builtin_amdgcn_perm(w[3][e >> 1], w[2][e >> 1], sel);
        o.z = __builtin_amdgcn_perm(w[5][e >> 1], w[4][e >> 1], sel);
        o.w = __builtin_amdgcn_perm(w[7][e >> 1], w[6][e >> 1], sel);
        tile[t128_slot(8 * bc + e, br)] = o;
    }
    __syncthreads();
    // output rows c0 + oc, chunk k = output columns r0 + 8k .. r0 + 8k + 7
#pragma unroll
    for (int q = tid; q < kT128 * kT128 / 8; q += 256) {
        const int oc = q >> 4, k = q & 15;
        const int64_t orow = c0 + oc, ocol = r0 + 8 * k;
        if (orow < j.out_rows && ocol < j.rows_pad)
            *reinterpret_cast<u32x4*>(out + orow * j.ld_out + ocol) = tile[t128_slot(oc, k)];
    }
}

__global__ __launch_bounds__(256) void transpose128_f16_kernel(TransposeF16 j0, TransposeF16 j1, int ny0, int ny1,
                                                               ReduceJob red) {
    if ((int)blockIdx.y >= ny0 + ny1) {      // uniform per workgroup
        const int64_t rb = (int64_t)(blockIdx.y - ny0 - ny1) * gridDim.x + blockIdx.x;
        if (rb < red.blocks) reduce_partials_block(red.partial, red.chunks, red.cols, red.out, rb);
        return;
    }
    __shared__ __align__(16) u32x4 tile[kT128 * kT128 / 8];   // 16-byte chunks, swizzled
    transpose128_body(j0, j1, ny0, blockIdx.x, blockIdx.y, tile);
}

// The statistics tiles of dY (workgroups below nstats) and the 128 x 128
// transposes of the forward's packed operands (the gx x ny tiles after them)
// are independent: one launch for both.
template <int DT, int BS, int PASSES, bool FINAL>
__global__ __launch_bounds__(256) void stats_transpose_kernel(StatsK k, int64_t ntx, int64_t nstats, TransposeF16 j0,
                                                              TransposeF16 j1, int ny0, int gx) {
    __shared__ __align__(16) u32x4 smem[kT128 * kT128 / 8];
    __shared__ int gred[4];
    const int64_t b = blockIdx.x;
    if (b < nstats) {
        stats_tile_body<DT, BS, PASSES, FINAL>(k, ntx, b, reinterpret_cast<uint32_t*>(smem), gred);
    } else {
        const int64_t t = b - nstats;
        transpose128_body(j0, j1, ny0, (int)(t % gx), (int)(t / gx), smem);
    }
}

__global__ void init_gmax_kernel(int32_t* p) { *p = INT_MIN; }

// Launch shape of the row pack for a row of nvec 16-byte vectors: NT threads,
// NV vectors each.
struct RowsShape { int nt; int nv; };
inline RowsShape rows_shape(int64_t nvec) {
    // one wave per row, four rows per workgroup (nt 64)
    if (nvec <= 64) return {64, 1};
    if (nvec <= 128) return {64, 2};
    if (nvec <= 256) return {64, 4};
    // one row per workgroup from here.  Measured with the forward's nearest
    // pack (graph-free event timing, 2048-16384 rows): 257-512 vectors
    // 256 x 2 beats one wave of 8 vectors by 0-24% (bf16 4096 columns 14.7
    // against 19.4 us); 513-1024 256 x 4; 1025-1536 768 x 2 beats 256 x 8 by
    // 8-15% (f32 6144 and bf16 11008-12288 columns); 1537-2048 512 x 4 beats
    // it by 6-10%; 2049-3072 768 x 4 (1024 x 4 and 512 x 8 slower); beyond,
    // 512 x 8.
    if (nvec <= 512) return {256, 2};
    if (nvec <= 1024) return {256, 4};
    if (nvec <= 1536) return {768, 2};
    if (nvec <= 2048) return {512, 4};
    if (nvec <= 3072) return {768, 4};
    return {512, 8};
}
constexpr int64_t kRowsMaxVec = 4096;   // 512 threads x 8 vectors

template <int DT, int MODE, bool COLX>
void dispatch_rows_nv(const PackRowsK& k, const PackRowsK& k2, int64_t rows, RowsShape sh, hipStream_t st) {
    // one row per workgroup (the loop in the kernel runs once): independent
    // workgroups overlap better than a persistent loop (measured)
    const dim3 grid((unsigned)rows);
    if (sh.nt == 64) {
        constexpr int RPW = 4;
        const dim3 g4((unsigned)((rows + RPW - 1) / RPW));
        if (sh.nv == 1) pack_rows_kernel<DT, MODE, COLX, 1, 64, RPW><<<g4, 64 * RPW, 0, st>>>(k, k2, rows);
        else if (sh.nv == 2) pack_rows_kernel<DT, MODE, COLX, 2, 64, RPW><<<g4, 64 * RPW, 0, st>>>(k, k2, rows);
        else pack_rows_kernel<DT, MODE, COLX, 4, 64, RPW><<<g4, 64 * RPW, 0, st>>>(k, k2, rows);
    } else if (sh.nt == 768) {
        if (sh.nv == 2) pack_rows_kernel<DT, MODE, COLX, 2, 768, 1><<<grid, 768, 0, st>>>(k, k2, rows);
        else pack_rows_kernel<DT, MODE, COLX, 4, 768, 1><<<grid, 768, 0, st>>>(k, k2, rows);
    } else if (sh.nt == 512) {
        if (sh.nv == 4) pack_rows_kernel<DT, MODE, COLX, 4, 512, 1><<<grid, 512, 0, st>>>(k, k2, rows);
        else pack_rows_kernel<DT, MODE, COLX, 8, 512, 1><<<grid, 512, 0, st>>>(k, k2, rows);
    } else if (sh.nv == 2) {
        pack_rows_kernel<DT, MODE, COLX, 2, 256, 1><<<grid, 256, 0, st>>>(k, k2, rows);
    } else {
        pack_rows_kernel<DT, MODE, COLX, 4, 256, 1><<<grid, 256, 0, st>>>(k, k2, rows);
    }
}

template <int DT>
void dispatch_rows(const PackRowsK& k, const PackRowsK& k2, int64_t rows, int mode, bool colx, RowsShape sh,
                   hipStream_t st) {
    if (mode == kRaw) {
        if (colx) dispatch_rows_nv<DT, kRaw, true>(k, k2, rows, sh, st); else dispatch_rows_nv<DT, kRaw, false>(k, k2, rows, sh, st);
    } else if (mode == kNearest) {
        if (colx) dispatch_rows_nv<DT, kNearest, true>(k, k2, rows, sh, st); else dispatch_rows_nv<DT, kNearest, false>(k, k2, rows, sh, st);
    } else {
        if (colx) dispatch_rows_nv<DT, kStochastic, true>(k, k2, rows, sh, st); else dispatch_rows_nv<DT, kStochastic, false>(k, k2, rows, sh, st);
    }
}

template <int DT, int BS>
void dispatch_t_bs(const PackTK& k, int mode, int64_t ntx, int64_t ntiles, hipStream_t st) {
    // one tile per workgroup (the kernel takes tile blockIdx.x): independent
    // workgroups overlap their load, compute and store phases better than a
    // persistent loop (measured)
    const dim3 grid((unsigned)ntiles);
    // one high word for every counter of the call: the 32-bit dither path
    const bool c32 = (k.offset >> 32) == ((k.offset + (uint64_t)(k.rows * k.cols) - 1) >> 32);
    if (mode == kRaw) pack_t_kernel<DT, kRaw, BS, false><<<grid, kPackThreads, 0, st>>>(k, ntx, ntiles);
    else if (mode == kNearest) pack_t_kernel<DT, kNearest, BS, false><<<grid, kPackThreads, 0, st>>>(k, ntx, ntiles);
    else if (c32) pack_t_kernel<DT, kStochastic, BS, true><<<grid, kPackThreads, 0, st>>>(k, ntx, ntiles);
    else pack_t_kernel<DT, kStochastic, BS, false><<<grid, kPackThreads, 0, st>>>(k, ntx, ntiles);
}

template <int DT>
void dispatch_t(const PackTK& k, int mode, int64_t ntx, int64_t ntiles, hipStream_t st) {
    if (k.block == 8) dispatch_t_bs<DT, 8>(k, mode, ntx, ntiles, st);
    else if (k.block == 16) dispatch_t_bs<DT, 16>(k, mode, ntx, ntiles, st);
    else dispatch_t_bs<DT, 32>(k, mode, ntx, ntiles, st);
}

constexpr int kGlobalRowsPerChunk = kTile;

}  // namespace

int64_t pack_global_chunks(int64_t rows) { return (rows + kGlobalRowsPerChunk - 1) / kGlobalRowsPerChunk; }

namespace {

int check_pack_rows(const PackRowsArgs& a, RowsShape* sh_out) {
    const int V = a.dtype == AXS6_F32 ? 4 : 8;
    if (a.rows > INT_MAX)   // one workgroup (or a quarter of one) per row: the grid is 32-bit
        return fail(AXS6_ERR_UNSUPPORTED, "pack_rows: %lld rows exceed the launch grid", (long long)a.rows);
    // a ragged last block is fine (lanes past the row read zeros, the
    // reference's padding); rows must be whole 16-byte vectors
    if (a.cols % V != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: cols (%lld) must be a multiple of %d", (long long)a.cols, V);
    if ((uintptr_t)a.x % 16 != 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: input not 16-byte aligned");
    if (a.colx && (uintptr_t)a.colx % 16 != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: column exponents not 16-byte aligned");
    if (a.out && (a.ld_out % 8 != 0 || (uintptr_t)a.out % 16 != 0 || a.cols_pad % 8 != 0 || a.cols_pad < a.cols))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: output must be 16-byte aligned with padded width >= cols");
    if (a.out && a.ld_out < a.cols_pad)   // rows would overlap and the last row's padding run past the buffer
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_rows: ld_out (%lld) is smaller than cols_pad (%lld)",
                    (long long)a.ld_out, (long long)a.cols_pad);
    const int64_t nvec = a.cols / V;
    if (nvec > kRowsMaxVec) {
        // longer than a workgroup holds in registers: statistics pass + tiled pack
        if (a.out && a.cols_pad < pad_to(a.cols, kTile))
            return fail(AXS6_ERR_UNSUPPORTED, "pack_rows: rows of more than %lld elements need cols_pad >= "
                        "64 * ceil(cols / 64) (got cols %lld, cols_pad %lld)", (long long)(kRowsMaxVec * V),
                        (long long)a.cols, (long long)a.cols_pad);
        *sh_out = RowsShape{0, 0};
        return AXS6_OK;
    }
    *sh_out = rows_shape(nvec);
    return AXS6_OK;
}

PackRowsK to_kernel_args(const PackRowsArgs& a, const DeviceTables& t) {
    return PackRowsK{a.x, a.rows, a.cols, a.block, a.seed, a.seed_dev, a.offset, a.colx, a.out, a.ld_out, a.cols_pad,
                     a.s_out, a.rmax_out, a.rowx, a.gmax, t.lut, t.band};
}

int pack_mode(const PackRowsArgs& a) { return a.fake_quant ? (a.stochastic ? kStochastic : kNearest) : kRaw; }

// Rows past the register-resident limit: the statistics of each row from
// stats_row_kernel, then the row-major operand from pack_t_kernel with those
// shifts (same FQ values and dither counters as pack_rows_kernel).
int launch_pack_rows_long(const PackRowsArgs& a, const DeviceTables& t, hipStream_t st) {
    const PackRowsK k = to_kernel_args(a, t);
    const dim3 grid((unsigned)a.rows);
#define AXS6_STATS_ROW(DT_)                                                                         \
    do {                                                                                            \
        if (a.block == 8) stats_row_kernel<DT_, 8><<<grid, 256, 0, st>>>(k);                        \
        else if (a.block == 16) stats_row_kernel<DT_, 16><<<grid, 256, 0, st>>>(k);                 \
        else stats_row_kernel<DT_, 32><<<grid, 256, 0, st>>>(k);                                    \
    } while (0)
    if (a.dtype == AXS6_F32) AXS6_STATS_ROW(AXS6_F32);
    else if (a.dtype == AXS6_BF16) AXS6_STATS_ROW(AXS6_BF16);
    else AXS6_STATS_ROW(AXS6_F16);
#undef AXS6_STATS_ROW
    int rc = check_launch("pack_rows");
    if (rc || !a.out) return rc;
    const PackTArgs p{a.x, a.dtype, a.rows, a.cols, a.block, a.fake_quant, a.stochastic, a.seed, a.offset,
                      a.seed_dev, nullptr, nullptr, nullptr, 0, a.out, a.ld_out, a.colx, a.s_out, nullptr};
    return launch_pack_t(p, t, st);
}

}  // namespace

int launch_pack_rows(const PackRowsArgs& a, const DeviceTables& t, hipStream_t st) {
    RowsShape sh{};
    int rc = check_pack_rows(a, &sh);
    if (rc) return rc;
    if (a.rows == 0) return AXS6_OK;
    if (sh.nt == 0) return launch_pack_rows_long(a, t, st);
    const PackRowsK k = to_kernel_args(a, t);
    const bool colx = a.colx != nullptr;
    if (a.dtype == AXS6_F32) dispatch_rows<AXS6_F32>(k, k, a.rows, pack_mode(a), colx, sh, st);
    else if (a.dtype == AXS6_BF16) dispatch_rows<AXS6_BF16>(k, k, a.rows, pack_mode(a), colx, sh, st);
    else dispatch_rows<AXS6_F16>(k, k, a.rows, pack_mode(a), colx, sh, st);
    return check_launch("pack_rows");
}

int launch_pack_rows2(const PackRowsArgs& a, const PackRowsArgs& b, const DeviceTables& t, hipStream_t st) {
    RowsShape sa{}, sb{};
    int rc = check_pack_rows(a, &sa);
    if (rc) return rc;
    if ((rc = check_pack_rows(b, &sb))) return rc;
    const bool same = sa.nt != 0 && a.dtype == b.dtype && pack_mode(a) == pack_mode(b) && sa.nt == sb.nt &&
                      sa.nv == sb.nv && (a.colx != nullptr) == (b.colx != nullptr);
    if (!same || a.rows == 0 || b.rows == 0) {
        if ((rc = launch_pack_rows(a, t, st))) return rc;
        return launch_pack_rows(b, t, st);
    }
    const PackRowsK ka = to_kernel_args(a, t), kb = to_kernel_args(b, t);
    const bool colx = a.colx != nullptr;
    const int64_t rows = a.rows + b.rows;
    if (a.dtype == AXS6_F32) dispatch_rows<AXS6_F32>(ka, kb, rows, pack_mode(a), colx, sa, st);
    else if (a.dtype == AXS6_BF16) dispatch_rows<AXS6_BF16>(ka, kb, rows, pack_mode(a), colx, sa, st);
    else dispatch_rows<AXS6_F16>(ka, kb, rows, pack_mode(a), colx, sa, st);
    return check_launch("pack_rows");
}

int launch_pack_t(const PackTArgs& a, const DeviceTables& t, hipStream_t st) {
    if (a.cols % (a.dtype == AXS6_F32 ? 4 : 8) != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_t: cols must be a multiple of 4 (f32) or 8 (bf16, f16)");
    if ((uintptr_t)a.x % 16 != 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_t: input not 16-byte aligned");
    if (a.out && (a.ld_out % 8 != 0 || (uintptr_t)a.out % 16 != 0 || a.ld_out < pad_to(a.rows, kTile)))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_t: output rows must be 16-byte aligned and hold the padded rows");
    if (a.rows == 0 || a.cols == 0) return AXS6_OK;
    if (a.out_r && (a.ld_r % 8 != 0 || (uintptr_t)a.out_r % 16 != 0 || a.ld_r < pad_to(a.cols, kTile) ||
                    !a.shift_r || (a.colx_r && (uintptr_t)a.colx_r % 16 != 0)))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "pack_t: row-major output must be 16-byte aligned and hold the padded columns");
    PackTK k{a.x, a.rows, a.cols, a.block, a.seed, a.seed_dev, a.offset, a.rowx, a.gmax, a.out, a.ld_out,
             a.out_r, a.ld_r, a.colx_r, a.shift_r, a.partial, t.lut, t.band, a.gtile, a.ngtile, a.gmax_out};
    const int64_t ntx = (a.cols + kTile - 1) / kTile, ntiles = ntx * pack_global_chunks(a.rows);
    const int mode = a.fake_quant ? (a.stochastic ? kStochastic : kNearest) : kRaw;
    if (a.dtype == AXS6_F32) dispatch_t<AXS6_F32>(k, mode, ntx, ntiles, st);
    else if (a.dtype == AXS6_BF16) dispatch_t<AXS6_BF16>(k, mode, ntx, ntiles, st);
    else dispatch_t<AXS6_F16>(k, mode, ntx, ntiles, st);
    return check_launch("pack_t");
}

int64_t row_stats_col_tiles(int64_t cols) { return (cols + kStatsCols - 1) / kStatsCols; }

int64_t row_stats_final_bands(int64_t rows, int64_t cols, int dtype) {
    const int rpp = dtype == AXS6_F32 ? 16 : 32;   // rows of a one-pass tile (PASSES 1)
    return cols <= kStatsCols ? (rows + rpp - 1) / rpp : 0;
}

namespace {
bool transpose128_ok(const TransposeF16& x) {
    return x.out_rows == 0 || x.rows_pad == 0 ||
           (x.ld_in % 8 == 0 && x.ld_out % 8 == 0 && x.rows_pad % 8 == 0 && x.cols % 8 == 0 &&
            (uintptr_t)x.in % 16 == 0 && (uintptr_t)x.out % 16 == 0);
}
}  // namespace

int launch_row_stats(const RowStatsArgs& a, const DeviceTables& t, hipStream_t st, const TransposeF16* ta,
                     const TransposeF16* tb) {
    if (a.cols % (a.dtype == AXS6_F32 ? 4 : 8) != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "row_stats: cols must be a multiple of 4 (f32) or 8 (bf16, f16)");
    if ((uintptr_t)a.x % 16 != 0 || (a.colx && (uintptr_t)a.colx % 16 != 0))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "row_stats: input and column exponents must be 16-byte aligned");
    if (a.rows == 0) return ta ? launch_transpose_f16(*ta, tb, st) : AXS6_OK;
    const int64_t ntx = row_stats_col_tiles(a.cols);
    const int64_t fbands = a.gtile ? row_stats_final_bands(a.rows, a.cols, a.dtype) : 0;
    StatsK k{a.x, a.rows, a.cols, a.colx, a.scratch, a.scratch + ntx * a.rows, t.band, a.gmax,
             a.shift, a.rowx, a.gtile};
    // the transposes ride in this launch when they take 128 x 128 tiles
    // (aligned operands, as the backward's always are), else run after it
    const TransposeF16 none{nullptr, 0, 0, 0, nullptr, 0, 0, 0};
    const TransposeF16& j0 = ta ? *ta : none;
    const TransposeF16& j1 = tb ? *tb : none;
    const bool with_t = ta && transpose128_ok(j0) && transpose128_ok(j1);
    const int64_t gx0 = j0.out_rows && j0.rows_pad ? (j0.out_rows + kT128 - 1) / kT128 : 0;
    const int64_t gx1 = j1.out_rows && j1.rows_pad ? (j1.out_rows + kT128 - 1) / kT128 : 0;
    const int64_t ny0 = gx0 ? (j0.rows_pad + kT128 - 1) / kT128 : 0, ny1 = gx1 ? (j1.rows_pad + kT128 - 1) / kT128 : 0;
    const int64_t gx = gx0 > gx1 ? gx0 : gx1;
    const TransposeF16& f0 = ny0 ? j0 : j1;   // the jobs in order: j0 (when it has tiles), then j1
    const TransposeF16& f1 = ny0 ? j1 : j0;
    const int fny0 = (int)(ny0 ? ny0 : ny1);
    const int64_t tblocks = with_t ? gx * (ny0 + ny1) : 0;
    // rows per tile: 16 bytes per lane, 16 (f32) or 32 (16-bit) rows per pass;
    // with tiles of whole rows (rows of at most 256 values) one pass, else as
    // many passes as keep >= 8192 workgroups, up to 4 (measured, f32 dY:
    // 8192 x 11008 66 us with 2 passes against 70 with 4; 8192 x 4096 25.6
    // with 1 against 27.4 with 4)
    const int rpp = a.dtype == AXS6_F32 ? 16 : 32;
    auto tiles = [&](int passes) { return ntx * ((a.rows + rpp * passes - 1) / (rpp * passes)); };
    const int passes = fbands ? 1 : (tiles(4) >= 8192 ? 4 : (tiles(2) >= 8192 ? 2 : 1));
    const int64_t nstats = fbands ? fbands : tiles(passes);
    const dim3 grid((unsigned)(nstats + tblocks));
#define AXS6_STATS_K(DT_, BS_, P_, F_)                                                               \
    do {                                                                                             \
        if (with_t)                                                                                  \
            stats_transpose_kernel<DT_, BS_, P_, F_><<<grid, 256, 0, st>>>(k, ntx, nstats, f0, f1,    \
                                                                          fny0, (int)gx);            \
        else                                                                                         \
            stats_tile_kernel<DT_, BS_, P_, F_><<<grid, 256, 0, st>>>(k, ntx);                       \
    } while (0)
#define AXS6_STATS_P(DT_, BS_)                                                                       \
    do {                                                                                             \
        if (fbands) AXS6_STATS_K(DT_, BS_, 1, true);                                                 \
        else if (passes == 4) AXS6_STATS_K(DT_, BS_, 4, false);                                      \
        else if (passes == 2) AXS6_STATS_K(DT_, BS_, 2, false);                                      \
        else AXS6_STATS_K(DT_, BS_, 1, false);                                                       \
    } while (0)
#define AXS6_STATS(DT_)                                                                              \
    do {                                                                                             \
        if (a.block == 8) AXS6_STATS_P(DT_, 8);                                                      \
        else if (a.block == 16) AXS6_STATS_P(DT_, 16);                                               \
        else AXS6_STATS_P(DT_, 32);                                                                  \
    } while (0)
    if (a.dtype == AXS6_F32) AXS6_STATS(AXS6_F32);
    else if (a.dtype == AXS6_BF16) AXS6_STATS(AXS6_BF16);
    else AXS6_STATS(AXS6_F16);
#undef AXS6_STATS
#undef AXS6_STATS_P
#undef AXS6_STATS_K
    int rc = check_launch("row_stats");
    if (rc) return rc;
    if (!fbands) {
        stats_finalize_kernel<<<dim3((unsigned)((a.rows + kFinRows - 1) / kFinRows)), 256, 0, st>>>(
            a.scratch, a.scratch + ntx * a.rows, a.rows, ntx, a.shift, a.rowx, a.gmax);
        if ((rc = check_launch("row_stats"))) return rc;
    }
    if (ta && !with_t) return launch_transpose_f16(*ta, tb, st);
    return AXS6_OK;
}

int launch_reduce_partials(const float* partial, int64_t chunks, int64_t cols, float* out, hipStream_t st) {
    if (cols == 0) return AXS6_OK;
    reduce_partials_kernel<<<dim3((unsigned)((cols + kRedCols - 1) / kRedCols)), 256, 0, st>>>(partial, chunks, cols,
                                                                                               out);
    return check_launch("reduce_partials");
}

int launch_transpose_f16(const TransposeF16& a, const TransposeF16* b, hipStream_t st, const float* partial,
                         int64_t chunks, int64_t cols, float* db) {
    const TransposeF16 none{nullptr, 0, 0, 0, nullptr, 0, 0, 0};
    const TransposeF16& bb = b ? *b : none;
    const int T = transpose128_ok(a) && transpose128_ok(bb) ? kT128 : kTile;
    const int64_t gx_a = a.out_rows && a.rows_pad ? (a.out_rows + T - 1) / T : 0;
    const int64_t gx_b = bb.out_rows && bb.rows_pad ? (bb.out_rows + T - 1) / T : 0;
    const int64_t ny0 = gx_a ? (a.rows_pad + T - 1) / T : 0, ny1 = gx_b ? (bb.rows_pad + T - 1) / T : 0;
    const bool red = db && partial && cols > 0;
    if (ny0 + ny1 == 0) return red ? launch_reduce_partials(partial, chunks, cols, db, st) : AXS6_OK;
    // a tile column past one job's out_rows writes nothing for it (orow >= out_rows)
    const int64_t gx = gx_a > gx_b ? gx_a : gx_b;
    const ReduceJob rj{partial, chunks, cols, db, red ? (cols + kRedCols - 1) / kRedCols : 0};
    const int64_t nyr = (rj.blocks + gx - 1) / gx;
    const dim3 grid((unsigned)gx, (unsigned)(ny0 + ny1 + nyr));
    // the jobs in order: a (when it has tiles), then b
    if (T == kT128)
        transpose128_f16_kernel<<<grid, 256, 0, st>>>(ny0 ? a : bb, ny0 ? bb : a, (int)(ny0 ? ny0 : ny1),
                                                      (int)(ny0 ? ny1 : 0), rj);
    else
        transpose_f16_kernel<<<grid, 256, 0, st>>>(ny0 ? a : bb, ny0 ? bb : a, (int)(ny0 ? ny0 : ny1),
                                                   (int)(ny0 ? ny1 : 0), rj);
    return check_launch("transpose_f16");
}

int launch_init_gmax(int32_t* p, hipStream_t st) {
    init_gmax_kernel<<<1, 1, 0, st>>>(p);
    return check_launch("init_gmax");
}

}  // namespace axs6
