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
//     -- and the K loop then reads FQ(X) from LDS and quantizes only W.
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
constexpr int kXlBytes = 128 * 1024; // LDS for FQ(X) in the XL form: M * (K + 4) floats

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

template <int DT, int WM, int TN, int NW, bool QX, bool XL>
__global__ __launch_bounds__(NW * 64) void fused_linear_kernel(FusedK k) {
    using E = Elem<DT>;
    using S = typename E::S;
    constexpr int BM = 16 * WM, BN = 16 * TN;
    static_assert(NW * BM * BN * 4 <= kFRed, "partial tiles must fit the reduction LDS");
    static_assert(!XL || WM == 1, "FQ(X) from LDS covers one 16-row block");
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
        if constexpr (!XL) {
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
                unpack8<DT>(xc[i], xf[i]);
                if constexpr (QX) fq8(xf[i], lut_s, band_s);
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

template <int DT, int WM, int TN, int NW, bool XL = false>
void launch_cfg(const FusedK& k, bool qx, hipStream_t st) {
    const int tiles = ((k.M + 16 * WM - 1) / (16 * WM)) * ((k.N + 16 * TN - 1) / (16 * TN));
    const size_t xl_bytes = XL ? (size_t)k.M * (k.K + 4) * sizeof(float) : 0;
    if constexpr (XL) {
        // up to kXlBytes of dynamic LDS beside ~20 KiB static (148 KiB of the
        // CU's 160 KiB): raise the per-kernel limit once
        static bool attr_set = false;
        if (!attr_set) {
            (void)hipFuncSetAttribute((const void*)fused_linear_kernel<DT, WM, TN, NW, true, XL>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kXlBytes);
            (void)hipFuncSetAttribute((const void*)fused_linear_kernel<DT, WM, TN, NW, false, XL>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kXlBytes);
            attr_set = true;
        }
    }
    if (qx) fused_linear_kernel<DT, WM, TN, NW, true, XL><<<dim3((unsigned)tiles), NW * 64, xl_bytes, st>>>(k);
    else fused_linear_kernel<DT, WM, TN, NW, false, XL><<<dim3((unsigned)tiles), NW * 64, xl_bytes, st>>>(k);
}

// Tile and K split by shape: one 16-row block for M <= 16 (decode), else
// two; the widest column tile (64, 32, 16) that still gives >= 256
// workgroups; as many K-splitting waves (up to 16, within the reduction LDS)
// as there are K tiles.
template <int DT>
void launch_dt(const FusedK& k, bool qx, hipStream_t st) {
    const int64_t nkt = k.K / kFBK;
    auto tiles = [&](int bm, int bn) { return ((k.M + bm - 1) / bm) * (int64_t)((k.N + bn - 1) / bn); };
    if (k.M <= 16) {
        const bool xl = (int64_t)k.M * (k.K + 4) * (int64_t)sizeof(float) <= kXlBytes;
        if (nkt >= 16) {
            if (xl) launch_cfg<DT, 1, 1, 16, true>(k, qx, st);
            else launch_cfg<DT, 1, 1, 16>(k, qx, st);
        } else {
            if (xl) launch_cfg<DT, 1, 1, 4, true>(k, qx, st);
            else launch_cfg<DT, 1, 1, 4>(k, qx, st);
        }
        return;
    }
    if (tiles(32, 64) >= 256) {
        if (nkt >= 4) launch_cfg<DT, 2, 4, 4>(k, qx, st);
        else launch_cfg<DT, 2, 4, 1>(k, qx, st);
    } else if (tiles(32, 32) >= 256) {
        if (nkt >= 8) launch_cfg<DT, 2, 2, 8>(k, qx, st);
        else launch_cfg<DT, 2, 2, 2>(k, qx, st);
    } else {
        if (nkt >= 16) launch_cfg<DT, 2, 1, 16>(k, qx, st);
        else launch_cfg<DT, 2, 1, 4>(k, qx, st);
    }
}

}  // namespace
}  // namespace axs6

using namespace axs6;

extern "C" int axs6_nf5_fused_linear(const void* x, const void* w, const float* bias, void* y, int32_t dtype,
                                     int64_t M, int64_t N, int64_t K, int32_t block_size, int32_t quantize_input,
                                     void* stream) {
    const char* fn = "axs6_nf5_fused_linear";
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    if (block_size != 32)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: the fused linear requires block_size=32 (got %d)", fn, block_size);
    if (M < 0 || N < 0 || K < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative dimension", fn);
    if (K % 32 != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: K (%lld) must be a multiple of 32 (pad it with zeros first)", fn,
                    (long long)K);
    if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30) || M * ((N + 15) / 16) > (int64_t)INT32_MAX)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: dimension too large", fn);
    if (M == 0 || N == 0) return AXS6_OK;
    if (K == 0) return fail(AXS6_ERR_UNSUPPORTED, "%s: empty contraction (K = 0)", fn);
    if (!x || !w || !y) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: x and w must be 16-byte aligned", fn);
    DeviceTables t;
    int rc = device_tables(&t);
    if (rc) return rc;
    const FusedK k{x, w, bias, y, (int)M, (int)N, (int)K, t.lut, t.band};
    hipStream_t st = (hipStream_t)stream;
    const bool qx = quantize_input != 0;
    if (dtype == AXS6_F32) launch_dt<AXS6_F32>(k, qx, st);
    else if (dtype == AXS6_BF16) launch_dt<AXS6_BF16>(k, qx, st);
    else launch_dt<AXS6_F16>(k, qx, st);
    return check_launch(fn);
}
