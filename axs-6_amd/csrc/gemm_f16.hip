// fp16 MFMA GEMM for the quantized linear (gfx950):
//   C[M, N] = epilogue( A[M, Kp] . B[N, Kp]^T ),  fp32 accumulation,
// both operands contraction-contiguous ("NT"), Kp a multiple of 64 with
// zero padding (the packing kernels write it).
//
// Tiling.  A workgroup of 4 waves owns a BM x BN tile of C; the waves form a
// 2 x 2 grid, each wave a (BM/2) x (BN/2) sub-tile built from 32x32 MFMA
// blocks (v_mfma_f32_32x32x16_f16: 32x32 fp32 accumulators, K = 16 per
// instruction, 16 accumulator registers per lane).  Per K-step of 64 the A
// and B tiles are staged through LDS (row pitch 64 + 8 halves, so the
// 16-byte fragment reads of 8 consecutive rows hit distinct bank groups);
// the next K-step's tiles are loaded into registers while the current one
// is multiplied (two LDS buffers, one barrier per step).
//
// Schedule.  Workgroup ids are dispatched round-robin over the 8 XCDs; the
// id is remapped so that each XCD receives a contiguous range of the grouped
// (GROUP_M rows of tiles) order, keeping the A rows and B columns an XCD
// touches inside its own L2.
//
// Epilogue.  v = ldexp(acc, row_exp[m] + col_exp[n] + glob) + bias[n], written
// as fp32, bf16 or fp16; the exponents undo the packing kernels' power-of-two
// row scales exactly.
#include <limits.h>

#include "linear_internal.h"

namespace axs6 {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;
constexpr int kLDK = kBK + 8;       // LDS row pitch in halves
constexpr int kGemmThreads = 256;
constexpr int kGroupM = 8;

struct GemmK {
    const _Float16* A; int64_t lda; const _Float16* B; int64_t ldb;
    int M; int N; int Kp;
    const int32_t* row_exp; const int32_t* col_exp; const int32_t* glob_exp; int glob_add;
    const float* bias; void* out; int64_t ldo; int out_dtype;
};

__device__ __forceinline__ uint16_t to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <int BM, int BN>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_f16_nt_kernel(GemmK g) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int A_LOADS = BM * (kBK / 8) / kGemmThreads;   // 16-byte chunks per thread
    constexpr int B_LOADS = BN * (kBK / 8) / kGemmThreads;
    static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small");
    extern __shared__ __align__(16) _Float16 smem[];
    _Float16* As = smem;                          // [2][BM * kLDK]
    _Float16* Bs = smem + 2 * BM * kLDK;          // [2][BN * kLDK]

    // ---- tile schedule -----------------------------------------------------
    const int tiles_m = (g.M + BM - 1) / BM;
    const int tiles_n = (g.N + BN - 1) / BN;
    const int total = tiles_m * tiles_n;
    int bid = blockIdx.x;
    if (total % 8 == 0) bid = (bid % 8) * (total / 8) + bid / 8;
    const int per_group = kGroupM * tiles_n;
    const int group = bid / per_group;
    const int first_m = group * kGroupM;
    const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int in_group = bid - group * per_group;
    const int tm0 = first_m + in_group % gsize;
    const int tn0 = in_group / gsize;
    const int m0 = tm0 * BM, n0 = tn0 * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // ---- global -> register staging ------------------------------------------
    u32x4g ra[A_LOADS], rb[B_LOADS];
    auto gload = [&](int kt) {
        const int64_t k0 = (int64_t)kt * kBK;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 3, c8 = q & 7;
            const int gr = m0 + row;
            ra[i] = gr < g.M ? *reinterpret_cast<const u32x4g*>(g.A + (int64_t)gr * g.lda + k0 + c8 * 8)
                             : u32x4g{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int q = tid + kGemmThreads * i;
            const int row = q >> 3, c8 = q & 7;
            const int gr = n0 + row;
            rb[i] = gr < g.N ? *reinterpret_cast<const u32x4g*>(g.B + (int64_t)gr * g.ldb + k0 + c8 * 8)
                             : u32x4g{0u, 0u, 0u, 0u};
        }
    };
    auto sstore = [&](int buf) {
        _Float16* as = As + buf * BM * kLDK;
        _Float16* bs = Bs + buf * BN * kLDK;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int q = tid + kGemmThreads * i;
            *reinterpret_cast<u32x4g*>(as + (q >> 3) * kLDK + (q & 7) * 8) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int q = tid + kGemmThreads * i;
            *reinterpret_cast<u32x4g*>(bs + (q >> 3) * kLDK + (q & 7) * 8) = rb[i];
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int KT = g.Kp / kBK;
    gload(0);
    sstore(0);
    __syncthreads();
    const int frow = lane & 31;          // fragment row within a 32-block
    const int fk = (lane >> 5) * 8;      // fragment K offset within a K=16 slice
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
        const _Float16* as = As + cur * BM * kLDK + (wm * WM + frow) * kLDK + fk;
        const _Float16* bs = Bs + cur * BN * kLDK + (wn * WN + frow) * kLDK + fk;
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            f16x8 af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const f16x8*>(as + i * 32 * kLDK + kk * 16);
#pragma unroll
            for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const f16x8*>(bs + j * 32 * kLDK + kk * 16);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue -------------------------------------------------------------
    const int gexp = g.glob_exp ? (*g.glob_exp == INT_MIN ? 0 : *g.glob_exp + g.glob_add) : 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WN + j * 32 + (lane & 31);
            if (col >= g.N) continue;
            const int cexp = (g.col_exp ? g.col_exp[col] : 0) + gexp;
            const float bias = g.bias ? g.bias[col] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (row >= g.M) continue;
                const int e = cexp + (g.row_exp ? g.row_exp[row] : 0);
                const float v = __builtin_amdgcn_ldexpf(acc[i][j][r], e) + bias;
                const int64_t o = (int64_t)row * g.ldo + col;
                if (g.out_dtype == AXS6_F32) reinterpret_cast<float*>(g.out)[o] = v;
                else if (g.out_dtype == AXS6_BF16) reinterpret_cast<uint16_t*>(g.out)[o] = to_bf16(v);
                else reinterpret_cast<_Float16*>(g.out)[o] = (_Float16)v;
            }
        }
    }
}

template <int BM, int BN>
int run_gemm(const GemmK& k, hipStream_t st) {
    const int tiles = ((k.M + BM - 1) / BM) * ((k.N + BN - 1) / BN);
    const size_t lds = (size_t)2 * (BM + BN) * kLDK * sizeof(_Float16);
    static bool attr_set = false;
    if (!attr_set) {
        hipFuncSetAttribute((const void*)gemm_f16_nt_kernel<BM, BN>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        attr_set = true;
    }
    gemm_f16_nt_kernel<BM, BN><<<dim3((unsigned)tiles), kGemmThreads, lds, st>>>(k);
    return check_launch("gemm_f16");
}

}  // namespace

int launch_gemm_f16(const GemmArgs& a, hipStream_t st) {
    if (a.M == 0 || a.N == 0) return AXS6_OK;
    if (a.Kp % kBK != 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: Kp (%lld) must be a multiple of %d", (long long)a.Kp, kBK);
    if (a.lda % 8 || a.ldb % 8 || (uintptr_t)a.A % 16 || (uintptr_t)a.B % 16)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: operands must be 16-byte aligned with ld a multiple of 8");
    if (a.M > INT_MAX || a.N > INT_MAX || a.Kp > INT_MAX)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: dimension exceeds int32");
    GemmK k{a.A, a.lda, a.B, a.ldb, (int)a.M, (int)a.N, (int)a.Kp, a.row_exp, a.col_exp, a.glob_exp,
            a.glob_add, a.bias, a.out, a.ldo, a.out_dtype};
#if defined(AXS6_GEMM_BM) && defined(AXS6_GEMM_BN)
    return run_gemm<AXS6_GEMM_BM, AXS6_GEMM_BN>(k, st);
#else
    return run_gemm<128, 128>(k, st);
#endif
}

}  // namespace axs6
