// Fused NF5 fake-quantize + contraction for small outputs (gfx950):
//   Y[M, N] = FQ(X)[M, K] . FQ(W)[N, K]^T + bias,   K a multiple of 32.
//
// The reference's single-launch fused linear (axs/unified/triton_kernels.py:
// 185-282, used by accelerated_linear for M*N <= 128K outputs,
// backend.py:567-590): each 32-wide K tile of X and W is fake-quantized as it
// is loaded (one NF5 block per row and tile), the FQ values never leave the
// registers, and the contraction runs in fp32 (the reference's tl.dot with
// input_precision "ieee").  Here:
//   * a workgroup owns a (16 WM) x (16 TN) output tile and its NW waves split
//     the K tiles into NW contiguous ranges; each wave accumulates the whole
//     output tile over its range and the NW partial tiles are added in wave
//     order at the end (deterministic).  A short, wide problem (decode: M of
//     1-32 against a 4096-wide weight) thereby runs thousands of waves;
//   * the contraction is v_mfma_f32_16x16x4_f32, which takes from lane l
//     (row l % 16, K group q = l / 16) one value per instruction.  Lane l
//     loads 8 values of its row's 32-block (kslot: two runs of 4 in f32, so
//     each 16-byte load instruction covers 64 contiguous bytes per row; the
//     run 8q .. 8q+7 in bf16/f16) and feeds its t-th value to the t-th
//     instruction: the 8 instructions together cover the block's 32 K once,
//     in a permuted order that A and B share, so no operand passes through
//     LDS;
//   * a row's block is the four lanes l % 16 = r: its amax is two cross-lane
//     maxima, then the FQ is the streaming FQ kernel's arithmetic (bit-exact
//     with fused_fake_quantize on the same values);
//   * the next K tile is loaded while the current one is quantized and
//     multiplied;
//   * with at most 16 rows of X (decode) whose FQ fits the LDS (XL), the
//     workgroup first quantizes its rows of X once into LDS -- every
//     workgroup needs all of X, and quantizing it per K tile with the 16-row
//     block of the MFMA spent as much VALU on X (mostly rows past M) as on W
//     -- and the K loop then reads FQ(X) from LDS and quantizes only W;
//   * at one or two rows of X whose FQ fits 48 KiB of LDS, the streamed
//     decode form (fused_decode_kernel) replaces it: a wave per weight row,
//     VALU products, whole-row loads;
//   * past both stagings (axs6_nf5_fused_linear_split), FQ(X) is written
//     once, in f32 and in the order the instructions read it (XA), by a
//     first launch, and the MFMA form reads it from there: one contiguous
//     KiB per load instruction, no FQ of X per workgroup.
// Unlike the packed fp16 path there is no row shift and no rounding of the
// operands: the products are those of fp32 FQ values, as in the reference's
// fused kernel.  For 16-bit inputs the FQ values stay fp32 too, as in the
// reference's fused kernel (it upcasts the operands and casts the fp32 result
// back to the input dtype).
#include "nf5_device.h"

namespace axs6 {
namespace {

typedef float f32x4f __attribute__((ext_vector_type(4)));

constexpr int kFBK = 32;             // K per tile = one NF5 block
constexpr int kFRed = 32 * 1024;     // bytes of LDS for the partial tiles
// LDS for FQ(X) in the XL form, M * (K + 4) floats: what the 160 KiB of a CU
// leaves beside the form's static 20.3 KiB (tables and 16 waves' partial
// tiles).  8 x 4096 (128.1 KiB) fits: 32.6 -> 17 us against the form that
// quantizes X in every K tile.
constexpr int kXlBytes = 139 * 1024;

struct FusedK {
    const void* x; const void* w; const float* bias; void* y;
    int M; int N; int K;
    const float* lut; const uint8_t* band;
};

// The 8 values lane (row r, group q) takes of a row's 32-block: in bf16/f16
// 8q .. 8q+7 (one 16-byte load; the four groups cover the row's 64 bytes);
// in f32 4q .. 4q+3 and 16+4q .. 16+4q+3, so each of the two 16-byte loads
// covers one contiguous 64-byte half of the block's 128 bytes per row.
template <int DT>
__device__ __forceinline__ int kslot(int q, int t) {
    return Elem<DT>::V == 4 ? (t < 4 ? 4 * q + t : 16 + 4 * q + (t - 4)) : 8 * q + t;
}

// No lane mask on the loads (the caller passes a row inside the operand): a
// load under a branch leaves the compiler's wait-count insertion paths with
// different loads outstanding, and it then waits for every load, the next
// tile's included, before the current tile is used (see the K loop).
template <int DT>
__device__ __forceinline__ void load8(const typename Elem<DT>::S* row, int kt, int q, u32x4 (&v)[2]) {
    using S = typename Elem<DT>::S;
    constexpr int V = Elem<DT>::V;
    if constexpr (V == 4) {
        const S* p = row + kt * kFBK + 4 * q;
        v[0] = *reinterpret_cast<const u32x4*>(p);
        v[1] = *reinterpret_cast<const u32x4*>(p + 16);
    } else {
        const S* p = row + kt * kFBK + 8 * q;
        v[0] = *reinterpret_cast<const u32x4*>(p);
    }
}

template <int DT>
__device__ __forceinline__ void unpack8(const u32x4 (&v)[2], float (&f)[8]) {
    using E = Elem<DT>;
    if constexpr (E::V == 4) {
        float a[4], b[4];
        E::unpack(v[0], a);
        E::unpack(v[1], b);
#pragma unroll
        for (int e = 0; e < 4; ++e) { f[e] = a[e]; f[4 + e] = b[e]; }
    } else {
        E::unpack(v[0], f);
    }
}

// FQ of a lane's 8 values; the block is the 4 lanes sharing lane % 16.
__device__ __forceinline__ void fq8(float (&f)[8], const float* lut_s, const uint8_t* band_s) {
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
        m = m > a ? m : a;
    }
    // max with lane ^ 16, then lane ^ 32: v_permlane16_swap (v, v) leaves rows
    // (0, 0, 2, 2) in its first result and (1, 1, 3, 3) in its second, so each
    // lane holds its value and its partner's across the two; permlane32_swap
    // likewise for the halves (lane layout checked on the GPU)
    const auto p16 = __builtin_amdgcn_permlane16_swap(m, m, false, false);
    m = p16[0] > p16[1] ? p16[0] : p16[1];
    const auto p32 = __builtin_amdgcn_permlane32_swap(m, m, false, false);
    m = p32[0] > p32[1] ? p32[0] : p32[1];
    const FqScale s = fq_scale(m, band_s);
    const float d[8] = {};
    fq_vector<8>(f, s, lut_s, false, d);
}

// XL prologue: FQ(X) of rows [0, M) (M <= 16) into xl (row stride K + 4
// floats: the 16 rows a ds_read_b128 group reads start 4 banks apart).  A
// thread takes 8 consecutive values, so an NF5 block is 4 neighbouring lanes
// (a DPP quad); K % 32 == 0 keeps every block's lanes together.
template <int DT, bool QX>
__device__ __forceinline__ void stage_x(const FusedK& k, float* xl, const float* lut_s, const uint8_t* band_s,
                                        int nthreads) {
    using E = Elem<DT>;
    using S = typename E::S;
    const int per_row = k.K / 8;
    const int nchunk = k.M * per_row;
    const int ld = k.K + 4;
    for (int c = threadIdx.x; c < nchunk; c += nthreads) {
        const int r = c / per_row, c8 = c - r * per_row;
        const S* p = reinterpret_cast<const S*>(k.x) + (int64_t)r * k.K + 8 * c8;
        u32x4 v[2];
        v[0] = *reinterpret_cast<const u32x4*>(p);
        if constexpr (E::V == 4) v[1] = *reinterpret_cast<const u32x4*>(p + 4);
        float f[8];
        unpack8<DT>(v, f);
        if constexpr (QX) {
            uint32_t m = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
                m = m > a ? m : a;
            }
            m = group_umax<4>(m);
            const FqScale s = fq_scale(m, band_s);
            const float d[8] = {};
            fq_vector<8>(f, s, lut_s, false, d);
        }
        float4* dst = reinterpret_cast<float4*>(xl + r * ld + 8 * c8);
        dst[0] = make_float4(f[0], f[1], f[2], f[3]);
        dst[1] = make_float4(f[4], f[5], f[6], f[7]);
    }
}

// X in the fragment order of the MFMA form (XA), written by arrange_x_kernel
// for the two-launch path: K tile kt of 16-row block b takes the 512 floats
// at (kt * nb + b) * 512 (nb = ceil(M / 16)), half h at + 256 h, and lane
// l = 16 q + r of the tile's 16x16x4 instructions finds at + 4 l its values
// for K slots kslot<DT>(q, 4 h .. 4 h + 3) of row 16 b + r.  Each of a
// wave's two 16-byte X loads per tile then reads 1 KiB contiguously instead
// of 64-byte pieces of 16 rows (32 x 4096 x 4096: 25.8 -> 19.8 us with X
// quantized beforehand either way).  f32 for every input dtype: the FQ
// values the single launch computes, not rounded to the input's type.
__host__ __device__ inline int64_t xa_floats(int64_t M, int64_t K) { return (M + 15) / 16 * 16 * K; }

// FQ (or, with QX false, a copy) of X into the XA order; the rows from M to
// the end of the last 16-row block hold zeros.  A thread takes 8 consecutive
// values of a row, so an NF5 block is a DPP quad (K % 32 == 0) and its two
// 4-value runs are two 16-byte stores.
template <int DT, bool QX>
__global__ __launch_bounds__(256) void arrange_x_kernel(FusedK k, float* xa) {
    using E = Elem<DT>;
    using S = typename E::S;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    if constexpr (QX) stage_tables(lut_s, band_w, k.lut, k.band);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);
    const int per_row = k.K / 8;
    const int nb = (k.M + 15) / 16;
    const int c = (int)blockIdx.x * 256 + (int)threadIdx.x;
    // whole quads leave together (256 and per_row are multiples of 4)
    if (c >= nb * 16 * per_row) return;
    const int r = c / per_row, c8 = c - r * per_row;
    float f[8] = {};
    if (r < k.M) {
        const S* p = reinterpret_cast<const S*>(k.x) + (int64_t)r * k.K + 8 * c8;
        u32x4 v[2];
        v[0] = *reinterpret_cast<const u32x4*>(p);
        if constexpr (E::V == 4) v[1] = *reinterpret_cast<const u32x4*>(p + 4);
        unpack8<DT>(v, f);
    }
    if constexpr (QX) {
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
            m = m > a ? m : a;
        }
        m = group_umax<4>(m);
        const FqScale s = fq_scale(m, band_s);
        const float d[8] = {};
        fq_vector<8>(f, s, lut_s, false, d);
    }
    // K offsets 8 j .. 8 j + 7 of the tile (j = c8 % 4): in f32 the slots
    // 4 q + e (h 0) and 16 + 4 q + e (h 1), so lanes q = 2 (j % 2) and + 1 of
    // half j / 2; in bf16/f16 8 q + t, so lane q = j, halves 0 and 1
    const int kt = c8 >> 2, j = c8 & 3, fr = r & 15;
    float4* tile = reinterpret_cast<float4*>(xa + ((int64_t)kt * nb + (r >> 4)) * 512);
    const float4 lo = make_float4(f[0], f[1], f[2], f[3]), hi = make_float4(f[4], f[5], f[6], f[7]);
    if constexpr (E::V == 4) {
        float4* h = tile + 64 * (j >> 1);
        const int q0 = 2 * (j & 1);
        h[16 * q0 + fr] = lo;
        h[16 * (q0 + 1) + fr] = hi;
    } else {
        tile[16 * j + fr] = lo;
        tile[64 + 16 * j + fr] = hi;
    }
}

template <int DT, int WM, int TN, int NW, bool QX, bool XL, bool XA>
__global__ __launch_bounds__(NW * 64) void fused_linear_kernel(FusedK k) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int BM = 16 * WM, BN = 16 * TN;
    static_assert(NW * BM * BN * 4 <= kFRed, "partial tiles must fit the reduction LDS");
    static_assert(!XL || WM == 1, "FQ(X) from LDS covers one 16-row block");
    static_assert(!XA || (!XL && !QX), "XA reads X as arranged, already quantized");
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ __align__(16) float red[NW * BM * BN];
    extern __shared__ __align__(16) float xl_s[];   // XL: FQ(X), M x (K + 4)
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tiles_n = (k.N + BN - 1) / BN;
    const int m0 = (int)(blockIdx.x / tiles_n) * BM;
    const int n0 = (int)(blockIdx.x % tiles_n) * BN;
    const int nkt = k.K / kFBK;
    const int kt0 = wave * nkt / NW, kt1 = (wave + 1) * nkt / NW;
    const int fr = lane & 15, q = lane >> 4;
    const S* xs = reinterpret_cast<const S*>(k.x);
    const S* ws = reinterpret_cast<const S*>(k.w);
    const S* xrow[WM];
    const S* wrow[TN];
    bool xlive[WM], wlive[TN];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int r = m0 + 16 * i + fr;
        xlive[i] = r < k.M;
        xrow[i] = xs + (int64_t)(xlive[i] ? r : 0) * k.K;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int r = n0 + 16 * j + fr;
        wlive[j] = r < k.N;
        wrow[j] = ws + (int64_t)(wlive[j] ? r : 0) * k.K;
    }
    // XA: the workgroup's 16-row blocks of X (a block wholly past M reads
    // block 0; its rows are not stored)
    const float* xa = reinterpret_cast<const float*>(k.x);
    const int nb = (k.M + 15) / 16;
    int64_t xblk[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) xblk[i] = m0 / 16 + i < nb ? m0 / 16 + i : 0;

    // The next K tile is loaded while the current one is quantized and
    // multiplied (two register buffers).  Deeper prefetch was slower: at M 1,
    // K = N = 4096, 15.0 us against 16.5 / 17.6 / 23.4 us for 2 / 3 / 7 tiles
    // ahead, and the loads alone (no FQ, no MFMA) take as long -- this read
    // pattern (64-byte pieces of 16 rows per instruction) streams the weight
    // at ~4.5 TB/s and slows with more of it in flight; whole-row reads of the
    // same bytes take 10.4-11.5 us.  Rows past M or N read row 0: an output
    // element takes only its own row of each operand, and those rows are not
    // stored.
    u32x4 xv[2][WM][2], wv[2][TN][2];
    auto load_tile = [&](int kt, u32x4 (&xd)[WM][2], u32x4 (&wd)[TN][2]) {
        if constexpr (XA) {
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const float* p = xa + ((int64_t)kt * nb + xblk[i]) * 512 + 4 * lane;
                xd[i][0] = *reinterpret_cast<const u32x4*>(p);
                xd[i][1] = *reinterpret_cast<const u32x4*>(p + 256);
            }
        } else if constexpr (!XL) {
#pragma unroll
            for (int i = 0; i < WM; ++i) load8<DT>(xrow[i], kt, q, xd[i]);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) load8<DT>(wrow[j], kt, q, wd[j]);
    };
    if (kt0 < kt1) load_tile(kt0, xv[0], wv[0]);
    stage_tables(lut_s, band_w, k.lut, k.band);
    if constexpr (XL) {
        stage_x<DT, QX>(k, xl_s, lut_s, band_s, NW * 64);
        __syncthreads();
    }
    const float* xl_row = xl_s + (xlive[0] ? fr : 0) * (k.K + 4);

    f32x4f acc[WM][TN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4f{0.0f, 0.0f, 0.0f, 0.0f};

    auto step = [&](int kt, u32x4 (&xc)[WM][2], u32x4 (&wc)[TN][2]) {
        float xf[WM][8], wf[TN][8];
        if constexpr (XL) {
            // lanes of rows past M read row 0: an output row takes only its own A row, and
            // the rows past M are not stored
            // the K slots of W's lanes (kslot): two 4-value runs in f32, one 8-value run otherwise
            const float4 a = *reinterpret_cast<const float4*>(xl_row + kt * kFBK + kslot<DT>(q, 0));
            const float4 b = *reinterpret_cast<const float4*>(xl_row + kt * kFBK + kslot<DT>(q, 4));
            xf[0][0] = a.x; xf[0][1] = a.y; xf[0][2] = a.z; xf[0][3] = a.w;
            xf[0][4] = b.x; xf[0][5] = b.y; xf[0][6] = b.z; xf[0][7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                if constexpr (XA) {
                    unpack8<AXS6_F32>(xc[i], xf[i]);
                } else {
                    unpack8<DT>(xc[i], xf[i]);
                    if constexpr (QX) fq8(xf[i], lut_s, band_s);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            unpack8<DT>(wc[j], wf[j]);
            fq8(wf[j], lut_s, band_s);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xf[i][t], wf[j][t], acc[i][j], 0, 0, 0);
    };
    // Steady state: two tiles per iteration, both prefetches inside the
    // wave's range; the last one or two tiles after the loop.  No load sits
    // under a branch inside the loop: the compiler's wait-count insertion would
    // see loop paths with different loads outstanding and wait for every
    // load, the next tile's included, before each tile (a full memory round
    // trip per K step; 16.3 -> 15.0 us at M 1 once removed), and loading
    // tiles past the range unconditionally instead costs a wave of one or two
    // tiles its time (256 x 512 x 512: 7.7 -> 10.0 us).
    int kt = kt0;
    for (; kt + 2 < kt1; kt += 2) {
        load_tile(kt + 1, xv[1], wv[1]);
        step(kt, xv[0], wv[0]);
        load_tile(kt + 2, xv[0], wv[0]);
        step(kt + 1, xv[1], wv[1]);
    }
    if (kt + 1 < kt1) {
        load_tile(kt + 1, xv[1], wv[1]);
        step(kt, xv[0], wv[0]);
        step(kt + 1, xv[1], wv[1]);
    } else if (kt < kt1) {
        step(kt, xv[0], wv[0]);
    }

    // the NW partial tiles, added in wave order: accumulator r of block
    // (i, j) is row 16 i + 4 (lane / 16) + r, column 16 j + lane % 16
    float* mine = red + wave * (BM * BN);
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) mine[(16 * i + 4 * q + r) * BN + 16 * j + fr] = acc[i][j][r];
    __syncthreads();
    for (int o = tid; o < BM * BN; o += NW * 64) {
        const int m = m0 + o / BN, n = n0 + o % BN;
        if (m >= k.M || n >= k.N) continue;
        float v = red[o];
#pragma unroll
        for (int w = 1; w < NW; ++w) v += red[w * (BM * BN) + o];
        if (k.bias) v += k.bias[n];
        reinterpret_cast<S*>(k.y)[(int64_t)m * k.N + n] = E::from_f(v);
    }
}

// ---- streamed decode form (M <= 2) ----------------------------------------
//
// One weight row per wave (K split over KS waves when the weight is short or
// very tall), streamed in steps of 512 values with two steps prefetched in a
// register ring; FQ(X) once per workgroup in LDS.  Lane l takes the 8
// consecutive values 8l .. 8l+7 of a step, so an NF5 block is a DPP quad and
// a wave's loads cover 2 KiB (f32) of one row: the whole-row read pattern the
// MFMA form's 16-row fragments cannot have (it streams the weight ~25% slower).
// The contraction is VALU FMAs against FQ(X) from LDS: at M <= 2 a 16-row
// MFMA block would be 7/8 or more padding, and the FQ, not the products, is
// the VALU work.  Per block the quantized magnitudes are taken unscaled
// (+-lut, exact zeros masked) and the block's 2^e1 is applied once to the
// lane's partial sum: (lut 2^e1) x = (lut x) 2^e1 exactly for the normal
// blocks this covers; other blocks (NaN, inf, tiny, overflowing scale) take
// the full FQ values with e1 = 0.
constexpr int kDecStep = 512;               // values of a row per wave step (8 per lane)
constexpr int kDecWaves = 8;                // waves per workgroup
constexpr int kDecPf = 2;                   // steps prefetched ahead
constexpr int kDecXBytes = 48 * 1024;       // LDS for FQ(X): three workgroups per CU

template <int DT> constexpr int dec_loads() { return Elem<DT>::V == 4 ? 2 : 1; }

// The 8 values of one lane at p (16-byte aligned).
template <int DT>
__device__ __forceinline__ void dec_load(const typename Elem<DT>::S* p, u32x4 (&v)[dec_loads<DT>()]) {
    v[0] = *reinterpret_cast<const u32x4*>(p);
    if constexpr (dec_loads<DT>() == 2) v[1] = *reinterpret_cast<const u32x4*>(p + 4);
}

// The same from a weight row through a buffer resource of `bytes` bytes from
// `base`: lanes past the row's end read zeros (the buffer's range check), so
// a step past K needs neither a clamp nor a mask.
template <int DT>
__device__ __forceinline__ void dec_load_row(const char* base, int bytes, int voff, u32x4 (&v)[dec_loads<DT>()]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, bytes, 0x00020000);
    v[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
    if constexpr (dec_loads<DT>() == 2)
        v[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, 0, 0));
}

template <int DT>
__device__ __forceinline__ void dec_unpack(const u32x4 (&v)[dec_loads<DT>()], float (&f)[8]) {
    using E = Elem<DT>;
    if constexpr (E::V == 4) {
        float a[4], b[4];
        E::unpack(v[0], a);
        E::unpack(v[1], b);
#pragma unroll
        for (int e = 0; e < 4; ++e) { f[e] = a[e]; f[4 + e] = b[e]; }
    } else {
        E::unpack(v[0], f);
    }
}

__device__ __forceinline__ float dec_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int DT, int MR, int KS, bool QX>
__global__ __launch_bounds__(kDecWaves * 64) void fused_decode_kernel(FusedK k) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int L = dec_loads<DT>();
    constexpr int NB = kDecPf + 1;
    constexpr int ES = sizeof(S);
    static_assert(kDecWaves % KS == 0, "waves per row");
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ float part_s[kDecWaves * MR];
    extern __shared__ __align__(16) float xq_s[];   // FQ(X) in the lanes' read order
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int SP = (k.K + kDecStep - 1) / kDecStep;       // steps per row
    const int ks = wave % KS;
    const int j0 = ks * SP / KS;
    const int SW = (ks + 1) * SP / KS - j0;               // this wave's steps (>= 1: SP >= KS)
    const int nw = (int)blockIdx.x * (kDecWaves / KS) + wave / KS;
    const bool live = nw < k.N;
    const int n = live ? nw : k.N - 1;                    // rows past N stream row N-1, unstored
    const char* wrow = reinterpret_cast<const char*>(k.w) + (int64_t)n * k.K * ES;
    const int voff = lane * 8 * ES;

    // The tables and this thread's first chunk of X are loaded first, then
    // the weight prefetch, and only then is FQ(X) computed: loads queued
    // behind the weight's would delay the prologue by their latency.
    float4 lutv = make_float4(0.f, 0.f, 0.f, 0.f);
    uint32_t bandv = 0;
    if (tid < kLutSize / 4) lutv = reinterpret_cast<const float4*>(k.lut)[tid];
    if (tid < kBandSize / 4) bandv = reinterpret_cast<const uint32_t*>(k.band)[tid];
    // X chunk c: row m, step j, lane slot l -> x[m, 512 j + 8 l .. + 7],
    // stored as float4 ((m SP + j) 2 + h) 64 + l (h: first / second four)
    const S* xs = reinterpret_cast<const S*>(k.x);
    const int nchunk = MR * SP * 64;
    auto x_load = [&](int c, u32x4 (&v)[L], bool& valid) {
        const int m = c / (SP * 64), j = (c / 64) % SP, l = c % 64;
        const int o = j * kDecStep + 8 * l;
        valid = c < nchunk && m < k.M && o < k.K;
        dec_load<DT>(xs + (valid ? (int64_t)m * k.K + o : 0), v);
    };
    u32x4 xv[L];
    bool xvalid;
    x_load(tid, xv, xvalid);

    u32x4 buf[NB][L];
    int pf = 0;                                           // steps prefetched so far
    auto prefetch = [&](u32x4 (&b)[L]) {
        const int j = j0 + (pf < SW ? pf : SW - 1);       // past the range: reload the last step
        const int done = j * kDecStep;
        dec_load_row<DT>(wrow + (int64_t)done * ES, (k.K - done) * ES, voff, b);
        ++pf;
    };
#pragma unroll
    for (int u = 0; u < kDecPf; ++u) prefetch(buf[u]);

    if (tid < kLutSize / 4) reinterpret_cast<float4*>(lut_s)[tid] = lutv;
    if (tid < kBandSize / 4) band_w[tid] = bandv;
    __syncthreads();
    auto x_stage = [&](int c, const u32x4 (&v)[L], bool valid) {
        float f[8];
        dec_unpack<DT>(v, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = valid ? f[e] : 0.0f;
        if constexpr (QX) {
            uint32_t mx = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
                mx = mx > a ? mx : a;
            }
            mx = group_umax<4>(mx);
            const FqScale s = fq_scale(mx, band_s);
            const float d[8] = {};
            fq_vector<8>(f, s, lut_s, false, d);
        }
        if (c < nchunk) {
            const int m = c / (SP * 64), j = (c / 64) % SP, l = c % 64;
            float4* dst = reinterpret_cast<float4*>(xq_s) + ((m * SP + j) * 2) * 64 + l;
            dst[0] = make_float4(f[0], f[1], f[2], f[3]);
            dst[64] = make_float4(f[4], f[5], f[6], f[7]);
        }
    };
    x_stage(tid, xv, xvalid);
    for (int c = tid + kDecWaves * 64; c < nchunk; c += kDecWaves * 64) {
        x_load(c, xv, xvalid);
        x_stage(c, xv, xvalid);
    }
    __syncthreads();

    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.0f;
    auto step = [&](const u32x4 (&wv)[L], int j) {
        float f[8];
        dec_unpack<DT>(wv, f);
        // block maximum and minimum of |w| (v_maximum3 / v_minimum3 with |.|
        // modifiers; the maximum propagates NaN, whose bits exceed inf's)
        float amx = __builtin_elementwise_maximum(__builtin_fabsf(f[0]), __builtin_fabsf(f[1]));
        float amn = __builtin_elementwise_minimum(__builtin_fabsf(f[0]), __builtin_fabsf(f[1]));
#pragma unroll
        for (int e = 2; e < 8; ++e) {
            amx = __builtin_elementwise_maximum(amx, __builtin_fabsf(f[e]));
            amn = __builtin_elementwise_minimum(amn, __builtin_fabsf(f[e]));
        }
        const uint32_t mx = group_umax<4>(__float_as_uint(amx));
        // fq_scale's short form, its general form when any lane needs it
        const int fexp = (int)(mx >> 23) - kExpBias;
        const uint32_t kb = (mx & 0x7f800000u) + 0x00800000u;
        int e1 = (kb - mx <= (uint32_t)band_s[fexp + 150]) ? fexp + 2 : fexp + 1;
        const bool wide = mx != 0u && (mx < kFastMinAmaxBits || e1 >= 128);
        if (__builtin_amdgcn_ballot_w64(wide) != 0) {
            const FqScale s = fq_scale_general(mx, band_s);
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = fq_value(f[e], s, lut_s, false, 0.0f);
            e1 = 0;
        } else {
            // fq_vector's short sequence without the final 2^e1 (lut_pos: the
            // index of |w| 1023 2^-e1)
            e1 = mx == 0u ? 0 : e1;
            const float c = __builtin_amdgcn_ldexpf(1023.0f, -e1);
            float g[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float mag = lut_s[(int)(__builtin_fabsf(f[e]) * c)];
                g[e] = __uint_as_float(__float_as_uint(mag) ^ (__float_as_uint(f[e]) & 0x80000000u));
            }
            // FQ(+-0) = +0 (lut[0] is not 0): masked only where a zero occurs
            if (__builtin_amdgcn_ballot_w64(__float_as_uint(amn) == 0u) != 0) {
#pragma unroll
                for (int e = 0; e < 8; ++e) g[e] = f[e] != 0.0f ? g[e] : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = g[e];
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float4* xp = reinterpret_cast<const float4*>(xq_s) + ((m * SP + j) * 2) * 64 + lane;
            const float4 xa = xp[0], xb = xp[64];
            float p0 = f[0] * xa.x, p1 = f[1] * xa.y;
            p0 = __builtin_fmaf(f[2], xa.z, p0);
            p1 = __builtin_fmaf(f[3], xa.w, p1);
            p0 = __builtin_fmaf(f[4], xb.x, p0);
            p1 = __builtin_fmaf(f[5], xb.y, p1);
            p0 = __builtin_fmaf(f[6], xb.z, p0);
            p1 = __builtin_fmaf(f[7], xb.w, p1);
            acc[m] += __builtin_amdgcn_ldexpf(p0 + p1, e1);
        }
    };
    // NB steps per iteration so the ring's slots are compile-time; every
    // prefetch is unconditional (a load under a branch would make the
    // compiler wait for all outstanding loads, the ring's included).
    for (int s0 = 0; s0 < SW; s0 += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            prefetch(buf[(u + kDecPf) % NB]);
            if (s0 + u < SW) step(buf[u], j0 + s0 + u);
        }
    }

    float t[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) t[m] = dec_wave_sum(acc[m]);
    if constexpr (KS > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m) part_s[wave * MR + m] = t[m];
        }
        __syncthreads();
        if (ks == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float v = part_s[wave * MR + m];
#pragma unroll
                for (int q = 1; q < KS; ++q) v += part_s[(wave + q) * MR + m];   // fixed order
                t[m] = v;
            }
        }
    }
    if (ks == 0 && lane == 0 && live) {
        const float bn = k.bias ? k.bias[n] : 0.0f;
#pragma unroll
        for (int m = 0; m < MR; ++m)
            if (m < k.M) reinterpret_cast<S*>(k.y)[(int64_t)m * k.N + n] = E::from_f(t[m] + bn);
    }
}

// The streamed decode form applies for M <= 2 when FQ(X) fits kDecXBytes.
bool decode_form_fits(const FusedK& k) {
    const int64_t sp = (k.K + kDecStep - 1) / kDecStep;
    return k.M <= 2 && (int64_t)k.M * sp * kDecStep * (int64_t)sizeof(float) <= kDecXBytes;
}

template <int DT, int MR, int KS>
void launch_decode_ks(const FusedK& k, bool qx, hipStream_t st) {
    const int sp = (k.K + kDecStep - 1) / kDecStep;
    const size_t xl = (size_t)MR * sp * kDecStep * sizeof(float);
    const unsigned grid = (unsigned)((k.N + kDecWaves / KS - 1) / (kDecWaves / KS));
    if (qx) fused_decode_kernel<DT, MR, KS, true><<<grid, kDecWaves * 64, xl, st>>>(k);
    else fused_decode_kernel<DT, MR, KS, false><<<grid, kDecWaves * 64, xl, st>>>(k);
}

// Two waves per row (each half of the steps) when the rows alone would give
// too few waves (N < 2048, at least 8 steps a row) or the row is long (16
// steps or more); measured at M = 1 (K x N): 4096 x 1024 6.8 -> 5.4 us,
// 8192 x 8192 47.4 -> 41.2 us, 8192 x 16000 97.3 -> 87.1 us; one wave per
// row at 4096 x 4096 12.6 against 13.9 us, 4096 x 32000 89.8 against
// 106.3 us, 4096 x 128000 324 against 362 us.
template <int DT, int MR>
void launch_decode(const FusedK& k, bool qx, hipStream_t st) {
    const int sp = (k.K + kDecStep - 1) / kDecStep;
    if ((sp >= 8 && k.N < 2048) || sp >= 16) launch_decode_ks<DT, MR, 2>(k, qx, st);
    else launch_decode_ks<DT, MR, 1>(k, qx, st);
}

template <int DT, int WM, int TN, int NW, bool XL = false, bool XA = false>
void launch_cfg(const FusedK& k, bool qx, hipStream_t st) {
    const int tiles = ((k.M + 16 * WM - 1) / (16 * WM)) * ((k.N + 16 * TN - 1) / (16 * TN));
    const size_t xl_bytes = XL ? (size_t)k.M * (k.K + 4) * sizeof(float) : 0;
    if constexpr (XL) {
        // up to kXlBytes of dynamic LDS beside ~20 KiB static (159.3 KiB of
        // the CU's 160 KiB): raise the per-kernel limit once
        static bool attr_set = false;
        if (!attr_set) {
            (void)hipFuncSetAttribute((const void*)fused_linear_kernel<DT, WM, TN, NW, true, XL, false>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kXlBytes);
            (void)hipFuncSetAttribute((const void*)fused_linear_kernel<DT, WM, TN, NW, false, XL, false>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kXlBytes);
            attr_set = true;
        }
    }
    const dim3 grid((unsigned)tiles);
    if constexpr (XA) fused_linear_kernel<DT, WM, TN, NW, false, false, true><<<grid, NW * 64, 0, st>>>(k);
    else if (qx) fused_linear_kernel<DT, WM, TN, NW, true, XL, false><<<grid, NW * 64, xl_bytes, st>>>(k);
    else fused_linear_kernel<DT, WM, TN, NW, false, XL, false><<<grid, NW * 64, xl_bytes, st>>>(k);
}

// The MFMA form's tile and K split by shape: one 16-row block for M <= 16
// (decode), else two; the widest column tile (64, 32, 16) that still gives
// >= 256 workgroups; as many K-splitting waves (up to 16, within the
// reduction LDS) as there are K tiles, but 8 for two 16-row blocks of 16
// columns (graph replays, 16 -> 8 waves: 48 x 768 x 2048 10.4 -> 9.2 us,
// 256 x 512 x 512 7.7 -> 7.3; arranged X: 362 x 4096 x 362 34.4 -> 32.3,
// 32 x 4096 x 4096 19.7 -> 19.3; others within 1%).  XA: X arranged by
// arrange_x_kernel.
template <int DT, bool XA>
void launch_mfma(const FusedK& k, bool qx, hipStream_t st) {
    const int64_t nkt = k.K / kFBK;
    auto tiles = [&](int bm, int bn) { return ((k.M + bm - 1) / bm) * (int64_t)((k.N + bn - 1) / bn); };
    if (k.M <= 16) {
        const bool xl = !XA && (int64_t)k.M * (k.K + 4) * (int64_t)sizeof(float) <= kXlBytes;
        if (nkt >= 16) {
            if (xl) launch_cfg<DT, 1, 1, 16, true>(k, qx, st);
            else launch_cfg<DT, 1, 1, 16, false, XA>(k, qx, st);
        } else {
            if (xl) launch_cfg<DT, 1, 1, 4, true>(k, qx, st);
            else launch_cfg<DT, 1, 1, 4, false, XA>(k, qx, st);
        }
        return;
    }
    if (tiles(32, 64) >= 256) {
        if (nkt >= 4) launch_cfg<DT, 2, 4, 4, false, XA>(k, qx, st);
        else launch_cfg<DT, 2, 4, 1, false, XA>(k, qx, st);
    } else if (tiles(32, 32) >= 256) {
        if (nkt >= 8) launch_cfg<DT, 2, 2, 8, false, XA>(k, qx, st);
        else launch_cfg<DT, 2, 2, 2, false, XA>(k, qx, st);
    } else {
        if (nkt >= 16) launch_cfg<DT, 2, 1, 8, false, XA>(k, qx, st);
        else launch_cfg<DT, 2, 1, 4, false, XA>(k, qx, st);
    }
}

template <int DT>
void launch_dt(const FusedK& k, bool qx, hipStream_t st) {
    if (decode_form_fits(k)) {
        if (k.M == 1) launch_decode<DT, 1>(k, qx, st);
        else launch_decode<DT, 2>(k, qx, st);
        return;
    }
    launch_mfma<DT, false>(k, qx, st);
}

// The two-launch path: X (quantized with qx) into the XA order, then the
// MFMA form on it.
template <int DT>
void launch_split(const FusedK& k, float* xa, bool qx, hipStream_t st) {
    const unsigned blocks = (unsigned)((xa_floats(k.M, k.K) / 8 + 255) / 256);
    if (qx) arrange_x_kernel<DT, true><<<blocks, 256, 0, st>>>(k, xa);
    else arrange_x_kernel<DT, false><<<blocks, 256, 0, st>>>(k, xa);
    FusedK ka = k;
    ka.x = xa;
    launch_mfma<DT, true>(ka, false, st);
}

}  // namespace
}  // namespace axs6

using namespace axs6;

// Whether a caller does better with the two-launch path
// (axs6_nf5_fused_linear_split): the shapes whose X neither the decode form
// nor the MFMA form's LDS staging holds, so every workgroup of the single
// launch reads (and quantizes) all of X again in its K tiles as 64-byte
// pieces of 16 rows, with contractions long enough (K >= 1024) for that to
// outweigh a second launch.  Measured (graph replays, f32, us, two launches
// against one): 32 x 4096 x 4096 24.0 / 31.0, 16 x 4096 x 4096 18.5 / 32.4,
// 16 x 8192 x 512 25.4 / 52.3, 362 x 4096 x 362 41.7 / 56.3, 32 x 1024 x
// 4096 10.4 / 11.2, 256 x 1024 x 512 11.3 / 11.1; K 512: 32 x 512 x 4096
// 7.7 / 7.4; X within the staging: 8 x 4096 x 4096 18.9 / 17.7.
extern "C" int32_t axs6_nf5_fused_linear_split_x(int64_t M, int64_t N, int64_t K, int32_t dtype) {
    if (!valid_dtype(dtype) || M <= 0 || N <= 0 || K < 1024 || K % 32 != 0 || K > (1 << 30) || M > (1 << 30))
        return 0;
    const FusedK k{nullptr, nullptr, nullptr, nullptr, (int)M, (int)N, (int)K, nullptr, nullptr};
    if (decode_form_fits(k)) return 0;
    const bool xl = M <= 16 && M * (K + 4) * (int64_t)sizeof(float) <= kXlBytes;
    return xl ? 0 : 1;
}

namespace {

// Arguments of both fused entry points; *empty set when there is nothing to
// compute (M or N zero).
int fused_args(const char* fn, const void* x, const void* w, const void* y, int32_t dtype, int64_t M, int64_t N,
               int64_t K, int32_t block_size, bool* empty) {
    *empty = false;
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    if (block_size != 32)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: the fused linear requires block_size=32 (got %d)", fn, block_size);
    if (M < 0 || N < 0 || K < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative dimension", fn);
    if (K % 32 != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: K (%lld) must be a multiple of 32 (pad it with zeros first)", fn,
                    (long long)K);
    if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30) || M * ((N + 15) / 16) > (int64_t)INT32_MAX)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: dimension too large", fn);
    if (M == 0 || N == 0) {
        *empty = true;
        return AXS6_OK;
    }
    if (K == 0) return fail(AXS6_ERR_UNSUPPORTED, "%s: empty contraction (K = 0)", fn);
    if (!x || !w || !y) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: x and w must be 16-byte aligned", fn);
    return AXS6_OK;
}

}  // namespace

extern "C" int axs6_nf5_fused_linear(const void* x, const void* w, const float* bias, void* y, int32_t dtype,
                                     int64_t M, int64_t N, int64_t K, int32_t block_size, int32_t quantize_input,
                                     void* stream) {
    const char* fn = "axs6_nf5_fused_linear";
    bool empty;
    int rc = fused_args(fn, x, w, y, dtype, M, N, K, block_size, &empty);
    if (rc || empty) return rc;
    DeviceTables t;
    rc = device_tables(&t);
    if (rc) return rc;
    const FusedK k{x, w, bias, y, (int)M, (int)N, (int)K, t.lut, t.band};
    hipStream_t st = (hipStream_t)stream;
    const bool qx = quantize_input != 0;
    if (dtype == AXS6_F32) launch_dt<AXS6_F32>(k, qx, st);
    else if (dtype == AXS6_BF16) launch_dt<AXS6_BF16>(k, qx, st);
    else launch_dt<AXS6_F16>(k, qx, st);
    return check_launch(fn);
}

extern "C" int64_t axs6_nf5_fused_linear_split_workspace(int64_t M, int64_t K) {
    return M > 0 && K > 0 && M <= (1 << 30) && K <= (1 << 30) ? xa_floats(M, K) * (int64_t)sizeof(float) : 0;
}

extern "C" int axs6_nf5_fused_linear_split(const void* x, const void* w, const float* bias, void* y,
                                           float* x_arranged, int32_t dtype, int64_t M, int64_t N, int64_t K,
                                           int32_t block_size, int32_t quantize_input, void* stream) {
    const char* fn = "axs6_nf5_fused_linear_split";
    bool empty;
    int rc = fused_args(fn, x, w, y, dtype, M, N, K, block_size, &empty);
    if (rc || empty) return rc;
    if (xa_floats(M, K) > (int64_t)INT32_MAX)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: x too large for the arranged workspace", fn);
    if (!x_arranged || (uintptr_t)x_arranged % 16)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: x_arranged must be a 16-byte aligned device buffer", fn);
    DeviceTables t;
    rc = device_tables(&t);
    if (rc) return rc;
    const FusedK k{x, w, bias, y, (int)M, (int)N, (int)K, t.lut, t.band};
    hipStream_t st = (hipStream_t)stream;
    const bool qx = quantize_input != 0;
    if (dtype == AXS6_F32) launch_split<AXS6_F32>(k, x_arranged, qx, st);
    else if (dtype == AXS6_BF16) launch_split<AXS6_BF16>(k, x_arranged, qx, st);
    else launch_split<AXS6_F16>(k, x_arranged, qx, st);
    return check_launch(fn);
}
