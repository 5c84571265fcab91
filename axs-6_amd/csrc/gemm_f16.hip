// fp16 MFMA GEMM for the quantized linear (gfx950):
//   C[M, N] = epilogue( A[M, Kp] . B[N, Kp]^T ),  fp32 accumulation,
// both operands contraction-contiguous ("NT"), Kp a multiple of 64 with
// zero padding (the packing kernels write it).
//
// Tiling.  A workgroup of WGM x WGN waves owns a BM x BN tile of C; each wave
// a (BM/WGM) x (BN/WGN) sub-tile of 16x16 MFMA blocks
// (v_mfma_f32_16x16x32_f16: K = 32 per instruction, 4 fp32 accumulators per
// lane).  Per K-step of 64 halves the A and B tiles go from HBM straight into
// LDS (buffer_load ... lds; rows past M/N read as zero through the buffer's
// range check) while the previous slab is multiplied; two LDS slabs, one
// barrier per step.  Each 64-half row is 8 slots of 16 bytes, XOR-swizzled
// (swz_key) so the 16-byte fragment reads are bank-conflict free.
//
// Schedule.  Workgroup ids are dispatched round-robin over the 8 XCDs; the
// id is remapped so that each XCD receives a contiguous range of the grouped
// (GROUP_M rows of tiles) order, keeping the A rows and B columns an XCD
// touches inside its own L2.
//
// Epilogue.  v = ldexp(acc, row_exp[m] + col_exp[n] + glob) + bias[n], written
// as fp32, bf16 or fp16; the exponents undo the packing kernels' power-of-two
// row scales exactly.  The accumulators leave through LDS: each wave stages
// one 32-row block row of its sub-tile at a time and writes whole row
// segments with 16 bytes per lane (f32) or 8 bytes (16-bit outputs), so a
// store instruction covers full 128-byte lines.  With one tile per CU every
// tile finishes at once; the scattered per-lane stores of the MFMA layout
// (two 128-byte rows per instruction) cost ~8% of the 4096^3 GEMM, the staged
// stores ~1%.
#include <limits.h>

#include "gemm_tile.h"
#include "partials.h"

namespace axs6 {
namespace {

struct GemmK {
    const _Float16* A; int64_t lda; const _Float16* B; int64_t ldb;
    int M; int N; int Kp;
    const int32_t* row_exp; const int32_t* col_exp; const int32_t* glob_exp; int glob_add;
    const float* bias; void* out; int64_t ldo; int out_dtype;
    int k_iters;            // 64-half K-steps per blockIdx.y (all of them without split-K)
    int64_t split_stride;   // elements between the split outputs (0 without split-K)
    int nt;                 // final output with nontemporal stores (gemm_streams_output)
};

template <int BM, int BN>
__device__ __forceinline__ void tile_origin(const GemmK& g, int bx, int& m0, int& n0) {
    tile_origin_mn<BM, BN>(g.M, g.N, bx, m0, n0);
}

// The epilogue through LDS, after the K loop.  Each wave stages its 32-row
// block row i (32 x WN floats, row stride WN+4 to spread banks;
// stage_block_row) in its own LDS region, then reads it back as 4
// consecutive columns per lane.  The slabs are dead once every wave has left
// the K loop (barrier); after that a wave touches only its own region, and
// LDS operations of one wave complete in order, so no further barrier is
// needed.
template <int WM, int WN>
__device__ __forceinline__ void gemm_epilogue(const GemmK& g, const WaveAcc<WM, WN>& acc, char* smem, int m0,
                                              int n0, int wm, int wn, int wave, int lane, int by) {
    constexpr int LDW = WN + 4;
    constexpr int LANES_PER_ROW = WN / 4;
    static_assert(64 % LANES_PER_ROW == 0 && 32 % (64 / LANES_PER_ROW) == 0, "wave tile width");
    wait_vmcnt<0>();
    __syncthreads();
    float* ws = reinterpret_cast<float*>(smem) + wave * (32 * LDW);
    const int gexp = g.glob_exp ? (*g.glob_exp == INT_MIN ? 0 : *g.glob_exp + g.glob_add) : 0;
    const int gcol = n0 + wn * WN + (lane % LANES_PER_ROW) * 4;
    int cexp[4];
    float cbias[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const bool in = gcol + t < g.N;
        cexp[t] = gexp + ((g.col_exp && in) ? g.col_exp[gcol + t] : 0);
        cbias[t] = (g.bias && in) ? g.bias[gcol + t] : 0.0f;
    }
    // Row exponents of the wave's WM rows, WM/64 per lane, loaded once: a load
    // per store pass would sit behind the previous pass's stores (the output
    // may alias row_exp as far as the compiler knows) and pay a full memory
    // latency each time -- ~15 us per launch, all of a small GEMM's runtime.
    constexpr int RPL = WM / 64;                      // row exponents held per lane
    static_assert(WM % 64 == 0, "wave tile height");
    int rexp_l[RPL];
#pragma unroll
    for (int q = 0; q < RPL; ++q) {
        const int grow = m0 + wm * WM + q * 64 + lane;
        rexp_l[q] = (g.row_exp && grow < g.M) ? g.row_exp[grow] : 0;
    }
    const int esize = g.out_dtype == AXS6_F32 ? 4 : 2;
    void* const out = reinterpret_cast<char*>(g.out) + (int64_t)by * g.split_stride * esize;
    const bool vec = (g.ldo % 4 == 0) && ((uintptr_t)out % (4 * esize) == 0);
    const int row0 = m0 + wm * WM;
    // the hint is a template argument (a run-time flag inside the store would
    // let the compiler merge the two stores and drop it); g.nt is uniform
    if (g.out_dtype == AXS6_F32) {
        if (g.nt)
            epilogue_store<AXS6_F32, true, WM, WN, LDW>(acc, ws, rexp_l, cexp, cbias, out, g.ldo, g.M, g.N, row0,
                                                        gcol, vec, lane);
        else
            epilogue_store<AXS6_F32, false, WM, WN, LDW>(acc, ws, rexp_l, cexp, cbias, out, g.ldo, g.M, g.N, row0,
                                                         gcol, vec, lane);
    } else if (g.out_dtype == AXS6_BF16) {
        if (g.nt)
            epilogue_store<AXS6_BF16, true, WM, WN, LDW>(acc, ws, rexp_l, cexp, cbias, out, g.ldo, g.M, g.N, row0,
                                                         gcol, vec, lane);
        else
            epilogue_store<AXS6_BF16, false, WM, WN, LDW>(acc, ws, rexp_l, cexp, cbias, out, g.ldo, g.M, g.N,
                                                          row0, gcol, vec, lane);
    } else {
        if (g.nt)
            epilogue_store<AXS6_F16, true, WM, WN, LDW>(acc, ws, rexp_l, cexp, cbias, out, g.ldo, g.M, g.N, row0,
                                                        gcol, vec, lane);
        else
            epilogue_store<AXS6_F16, false, WM, WN, LDW>(acc, ws, rexp_l, cexp, cbias, out, g.ldo, g.M, g.N, row0,
                                                         gcol, vec, lane);
    }
}

// Multi-stage variant: operand tiles go from HBM straight into LDS
// (buffer_load_dwordx4 ... lds, 16 bytes per lane, a wave instruction fills
// 1 KiB = 8 rows of a 64-half K-slab) with STAGES slabs in flight, so a
// slab's load latency is covered by STAGES-1 K-steps of MFMA work and no
// registers are spent on staging.  Lane l of a load instruction lands at
// byte 16*l of its 1 KiB, i.e. row l/8, slot l%8, and therefore fetches
// logical chunk (l%8) ^ key(row) -- the same XOR layout the fragment reads use.
// Output tile bx (before the XCD remap) and K split by of g.
template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int LW>
__device__ __forceinline__ void gemm_lds_body(const GemmK& g, int bx, int by) {
#if defined(__HIP_DEVICE_COMPILE__)  // LDS-DMA builtins exist only in the device pass
    constexpr int NW = WGM * WGN;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int RB = BK * 2;                                 // bytes per slab row
    constexpr int SPR = BK / 8;                                // 16-byte slots per row
    constexpr int ROWS_PER_INST = 1024 / RB;                   // rows one wave load fills
    static_assert(LW >= 1 && LW <= NW && NW % LW == 0, "loading waves");
    constexpr int A_INST = BM / ROWS_PER_INST / LW;            // load instructions per loading wave per slab
    constexpr int B_INST = BN / ROWS_PER_INST / LW;
    constexpr int IPW = A_INST + B_INST;
    constexpr int SLAB = (BM + BN) * RB;
    static_assert(A_INST >= 1 && B_INST >= 1 && STAGES >= 2, "tile shape");
    extern __shared__ __align__(16) char smem[];

    int m0, n0;
    tile_origin<BM, BN>(g, bx, m0, n0);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    // waves 0 .. LW-1 issue the slab loads (wave-uniform branch)
    const bool loader = wave < LW;

    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)g.A, 0, (int)((int64_t)g.M * g.lda * 2), kBufferConfig);
    const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)g.B, 0, (int)((int64_t)g.N * g.ldb * 2), kBufferConfig);
    // per-lane global byte offsets and per-wave LDS offsets of this wave's loads
    const int lrow = lane / SPR;                      // row inside the load's row group
    const int lslot = lane % SPR;                     // LDS slot this lane fills
    int a_goff[A_INST], a_loff[A_INST], b_goff[B_INST], b_loff[B_INST];
#pragma unroll
    for (int i = 0; i < A_INST; ++i) {
        const int row = (wave % LW + LW * i) * ROWS_PER_INST + lrow;     // row of the A slab
        a_goff[i] = (int)((int64_t)(m0 + row) * g.lda * 2) + ((lslot ^ swz_key<BK>(row)) << 4);
        a_loff[i] = (wave % LW + LW * i) * 1024;
    }
#pragma unroll
    for (int i = 0; i < B_INST; ++i) {
        const int row = (wave % LW + LW * i) * ROWS_PER_INST + lrow;
        b_goff[i] = (int)((int64_t)(n0 + row) * g.ldb * 2) + ((lslot ^ swz_key<BK>(row)) << 4);
        b_loff[i] = BM * RB + (wave % LW + LW * i) * 1024;
    }
    // split-K: this workgroup's range of K-steps (k_iters counts 64-half steps)
    static_assert(kGemmK % BK == 0, "K-slab must divide the padding unit");
    const int per = g.k_iters * (kGemmK / BK);
    const int kbeg = by * per;
    const int KT = min(per, g.Kp / BK - kbeg);
#pragma unroll
    for (int i = 0; i < A_INST; ++i) a_goff[i] += kbeg * RB;
#pragma unroll
    for (int i = 0; i < B_INST; ++i) b_goff[i] += kbeg * RB;
    auto lds_ptr = [](char* p) { return (__attribute__((address_space(3))) void*)p; };

    using Acc = WaveAcc<WM, WN>;
    Acc acc;
#pragma unroll
    for (int i = 0; i < Acc::TM; ++i)
#pragma unroll
        for (int j = 0; j < Acc::TN; ++j)
#pragma unroll
            for (int r = 0; r < Acc::R; ++r) acc.v[i][j][r] = 0.0f;

    // prologue: slabs 0 .. STAGES-2
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
        if (s < KT && loader) {
            char* slab = smem + s * SLAB;
#pragma unroll
            for (int i = 0; i < A_INST; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, lds_ptr(slab + a_loff[i]), 16, a_goff[i] + s * RB, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < B_INST; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, lds_ptr(slab + b_loff[i]), 16, b_goff[i] + s * RB, 0, 0, 0);
        }
    }

    // fragment row and K-group of this lane
    const int fr = lane % 16;
    const int fg = lane / 16;
    const int a_row0 = wm * WM + fr;
    const int b_row0 = wn * WN + fr;
    for (int kt = 0; kt < KT; ++kt) {
        // slab kt has landed once at most (slabs issued after it) * IPW loads are outstanding
        const int ahead = (KT - 1 - kt) < (STAGES - 2) ? (KT - 1 - kt) : (STAGES - 2);
        wait_slabs<STAGES - 2, IPW>(ahead);
        // a bare s_barrier: __syncthreads() would also drain every outstanding
        // load (vmcnt(0)) and serialise the pipeline; the explicit vmcnt wait
        // above already orders this wave's LDS fills before the barrier.
        __builtin_amdgcn_s_barrier();
        const int nk = kt + STAGES - 1;
        if (nk < KT && loader) {
            char* slab = smem + (nk % STAGES) * SLAB;
#pragma unroll
            for (int i = 0; i < A_INST; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, lds_ptr(slab + a_loff[i]), 16, a_goff[i] + nk * RB, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < B_INST; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, lds_ptr(slab + b_loff[i]), 16, b_goff[i] + nk * RB, 0, 0, 0);
        }
        const char* slab = smem + (kt % STAGES) * SLAB;
        mma_step16<BK, WM, WN>(acc, slab, slab + BM * RB, a_row0, b_row0, fg);
    }

    static_assert(NW * 32 * (WN + 4) * 4 <= STAGES * SLAB, "epilogue staging must fit in the slab LDS");
    gemm_epilogue<WM, WN>(g, acc, smem, m0, n0, wm, wn, wave, lane, by);
#endif
}

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int LW>
__global__ __launch_bounds__(WGM * WGN * 64, 1) void gemm_f16_nt_lds_kernel(GemmK g) {
    gemm_lds_body<BM, BN, BK, STAGES, WGM, WGN, LW>(g, (int)blockIdx.x, (int)blockIdx.y);
}

// Two independent GEMMs of one configuration in one launch (the backward's dX
// and dW): workgroups below n0 take g0's tiles x splits (tile-fastest, as
// the grid of a launch of its own orders them), the rest g1's.  n0 is g0's
// count rounded up to a multiple of 8, so both keep their own workgroup-to-XCD
// placement; the workgroups in between exit at once.
// A fixed-order column sum (reduce_partials_block, 256 threads) riding in a
// GEMM launch: `blocks` workgroups after the GEMM tiles.
struct GemmRedJob { const float* partial; int64_t chunks; int64_t cols; float* out; int blocks; };

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int LW>
__global__ __launch_bounds__(WGM * WGN * 64, 1) void gemm_f16_nt_lds_pair_kernel(GemmK g0, GemmK g1, int n0,
                                                                                 int t0, int s0, int t1, int s1,
                                                                                 GemmRedJob red) {
    const int b = (int)blockIdx.x;
    if (b < n0) {
        if (b < t0 * s0) gemm_lds_body<BM, BN, BK, STAGES, WGM, WGN, LW>(g0, b % t0, b / t0);
    } else if (b < n0 + t1 * s1) {
        const int c = b - n0;
        gemm_lds_body<BM, BN, BK, STAGES, WGM, WGN, LW>(g1, c % t1, c / t1);
    } else if constexpr (WGM * WGN * 64 == 256) {
        reduce_partials_block(red.partial, red.chunks, red.cols, red.out, b - n0 - t1 * s1);
    }
}

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int LW = WGM * WGN>
int run_gemm_lds(const GemmK& k, int splits, hipStream_t st) {
    const int tiles = ((k.M + BM - 1) / BM) * ((k.N + BN - 1) / BN);
    const size_t lds = (size_t)STAGES * (BM + BN) * BK * 2;
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)gemm_f16_nt_lds_kernel<BM, BN, BK, STAGES, WGM, WGN, LW>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        attr_set = true;
    }
    gemm_f16_nt_lds_kernel<BM, BN, BK, STAGES, WGM, WGN, LW>
        <<<dim3((unsigned)tiles, (unsigned)splits), WGM * WGN * 64, lds, st>>>(k);
    return check_launch("gemm_f16_lds");
}

template <int BM, int BN, int BK, int STAGES, int WGM, int WGN, int LW = WGM * WGN>
int run_gemm_lds_pair(const GemmK& k0, int s0, const GemmK& k1, int s1, const GemmRedJob& red, hipStream_t st) {
    const int t0 = ((k0.M + BM - 1) / BM) * ((k0.N + BN - 1) / BN);
    const int t1 = ((k1.M + BM - 1) / BM) * ((k1.N + BN - 1) / BN);
    const int n0 = (t0 * s0 + 7) / 8 * 8;
    const size_t lds = (size_t)STAGES * (BM + BN) * BK * 2;
    static bool attr_set = false;
    if (!attr_set) {
        (void)hipFuncSetAttribute((const void*)gemm_f16_nt_lds_pair_kernel<BM, BN, BK, STAGES, WGM, WGN, LW>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        attr_set = true;
    }
    gemm_f16_nt_lds_pair_kernel<BM, BN, BK, STAGES, WGM, WGN, LW>
        <<<dim3((unsigned)(n0 + t1 * s1 + red.blocks)), WGM * WGN * 64, lds, st>>>(k0, k1, n0, t0, s0, t1, s1, red);
    return check_launch("gemm_f16_lds_pair");
}

// Split-K finish: out[m, n] = ldexp(sum_z partial[z, m, n], row_exp[m] +
// col_exp[n] + glob) + bias[n], the splits summed in a fixed order (the
// result depends on the split count, never on scheduling); partial rows are
// N floats long.
struct SplitReduceK {
    const float* partial; int splits; int64_t stride; int M; int N;
    const int32_t* row_exp; const int32_t* col_exp; const int32_t* glob_exp; int glob_add;
    const float* bias; void* out; int64_t ldo; int out_dtype;
    // an independent fixed-order column sum riding in the same launch: the
    // workgroups past the split reduction's (GemmArgs::red_*)
    int64_t split_blocks; const float* red_partial; int64_t red_chunks; int64_t red_cols; float* red_out;
};

// A workgroup takes 64 groups of four output columns; its four waves sum four
// consecutive ranges of splits (eight loads in flight each), then the ranges
// are added in order.
constexpr int kSplitGroups = 64, kSplitRanges = 4;

__global__ __launch_bounds__(256) void splitk_reduce_kernel(SplitReduceK k) {
    if ((int64_t)blockIdx.x >= k.split_blocks) {   // uniform per workgroup
        reduce_partials_block(k.red_partial, k.red_chunks, k.red_cols, k.red_out, blockIdx.x - k.split_blocks);
        return;
    }
    __shared__ float4 part[kSplitRanges][kSplitGroups];
    const int n4 = (k.N + 3) / 4;
    const int lg = threadIdx.x % kSplitGroups, q = threadIdx.x / kSplitGroups;
    const int64_t idx = (int64_t)blockIdx.x * kSplitGroups + lg;
    const bool live = idx < (int64_t)k.M * n4;
    const int row = live ? (int)(idx / n4) : 0;
    const int col = live ? (int)(idx - (int64_t)row * n4) * 4 : 0;
    const bool full = col + 3 < k.N && k.N % 4 == 0;
    const int64_t o = (int64_t)row * k.N + col;
    const int per = (k.splits + kSplitRanges - 1) / kSplitRanges;
    const int z0 = q * per, z1 = (z0 + per) < k.splits ? z0 + per : k.splits;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (live && full) {
        int z = z0;
        for (; z + 8 <= z1; z += 8) {
            float4 w[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const float4*>(k.partial + (z + u) * k.stride + o);
#pragma unroll
            for (int u = 0; u < 8; ++u) { v[0] += w[u].x; v[1] += w[u].y; v[2] += w[u].z; v[3] += w[u].w; }
        }
        for (; z < z1; ++z) {
            const float4 w = *reinterpret_cast<const float4*>(k.partial + z * k.stride + o);
            v[0] += w.x; v[1] += w.y; v[2] += w.z; v[3] += w.w;
        }
    } else if (live) {
        for (int z = z0; z < z1; ++z)
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (col + t < k.N) v[t] += k.partial[z * k.stride + o + t];
    }
    part[q][lg] = make_float4(v[0], v[1], v[2], v[3]);
    __syncthreads();
    if (q != 0 || !live) return;
#pragma unroll
    for (int r = 1; r < kSplitRanges; ++r) {
        const float4 w = part[r][lg];
        v[0] += w.x; v[1] += w.y; v[2] += w.z; v[3] += w.w;
    }
    const int gexp = k.glob_exp ? (*k.glob_exp == INT_MIN ? 0 : *k.glob_exp + k.glob_add) : 0;
    const int rexp = gexp + (k.row_exp ? k.row_exp[row] : 0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (col + t >= k.N) break;
        v[t] = __builtin_amdgcn_ldexpf(v[t], rexp + (k.col_exp ? k.col_exp[col + t] : 0)) +
               (k.bias ? k.bias[col + t] : 0.0f);
    }
    const int esize = k.out_dtype == AXS6_F32 ? 4 : 2;
    const bool vec = (k.ldo % 4 == 0) && ((uintptr_t)k.out % (4 * esize) == 0);
    store4(k.out, k.ldo, k.N, k.out_dtype, row, col, v, vec);
}

// Launch configurations (BMxBN tile / 64-half K-slab / LDS stages / waves),
// all on 16x16x32 MFMAs:
//   big:    256x256 / 2 stages / 8 waves (2x4), waves 0-3 issue the slab loads
//   small:  128x128 / 2 stages / 4 waves (2x2)
//   narrow: 128x64 / 2 stages (3 on contractions of 32+ K-steps) / 4 waves
// Big by default; small when the 256x256 tiles do not cover the 256 CUs
// once; narrow when the 128x128 ones do not either (8192 x 256 outputs: 128
// -> 256 workgroups, 9.7 -> 7.5 us at K 256, 15.1 -> 11.0 us at K 1024;
// 2048 x 768 at K 3072 34.5 -> 29.3 us; where 128x128 tiles already fill the
// CUs, 128x64 ones are up to 11% slower).
// Loads from waves 0-3 only (against every wave loading): 6-12% shorter on
// the large shapes.  Waves are placed on the CU's four SIMDs round-robin, so
// each SIMD holds one loading and one compute-only wave.  When all eight
// waves leave the barrier and issue their loads together, the address unit
// (~64 bytes per clock) backs up and both waves of a SIMD stall in the
// issue, leaving its MFMA pipe idle; with one loader per SIMD the other wave
// runs its MFMAs meanwhile (the loads still land well inside the K-step).
// Measured: the stalled-issue counters SQ_VMEM_TA_ADDR_FIFO_FULL /
// _CMD_FIFO_FULL were 50x those of hipBLASLt's fp16 kernel with every wave
// loading.
// The epilogue of a tile (LDS staging, exponent scaling, stores) costs a
// fixed ~7 us per 256x256 f32 tile and CU, all of a short-K GEMM's runtime
// when 32 CUs carry it; 128x128 tiles spread it over 4x the CUs, two
// workgroups sharing a CU.
enum GemmCfg { kCfgBig = 0, kCfgSmall = 1, kCfgNarrow = 2 };
constexpr int kNarrowDeepSteps = 32;   // 64-deep K-steps per workgroup from which narrow runs three slabs

int64_t tiles_of(int64_t M, int64_t N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

int pick_cfg(int64_t M, int64_t N) {
    if (tiles_of(M, N, 256, 256) >= 256) return kCfgBig;
    return tiles_of(M, N, 128, 128) >= 256 ? kCfgSmall : kCfgNarrow;
}

// output tile of a configuration
void cfg_tile(int cfg, int* bm, int* bn) {
    *bm = 256; *bn = 256;
    if (cfg == kCfgSmall) *bm = *bn = 128;
    if (cfg == kCfgNarrow) { *bm = 128; *bn = 64; }
}

}  // namespace

int gemm_split_count(int64_t M, int64_t N, int64_t Kp) {
    if (M <= 0 || N <= 0) return 1;   // nothing to split (and no division by a zero tile count)
    int bm, bn;
    cfg_tile(pick_cfg(M, N), &bm, &bn);
    const int64_t tiles = tiles_of(M, N, bm, bn);
    const int64_t iters = Kp / kGemmK;
    if (tiles >= 64 || iters < 8) return 1;
    int64_t s = iters / 4;                                   // at least 4 K-steps per split
    s = s < 256 / tiles ? s : 256 / tiles;                   // about one workgroup per CU
    const int64_t cap = ((int64_t)4 << 20) / (M * N);       // partials <= 16 MiB
    s = s < cap ? s : cap;
    if (s < 2) return 1;
    const int64_t per = (iters + s - 1) / s;       // no empty split
    return (int)((iters + per - 1) / per);
}

size_t gemm_split_bytes(int64_t M, int64_t N, int64_t Kp) {
    const int s = gemm_split_count(M, N, Kp);
    return s > 1 ? (size_t)s * (size_t)M * (size_t)N * sizeof(float) : 0;
}

namespace {

// The last round of 256x256 tiles.  With 256 CUs and one tile per CU, an
// output of R full rounds plus r < 128 tiles takes R + 1 rounds while the
// r tiles leave most CUs idle.  Such a launch is cut along whichever
// dimension leaves a multiple of 256 tiles in the first part: that part
// runs as before, the remainder as a separate launch with its own
// configuration (128x128 tiles).  8192 x 11008 (K 4096): 1376 tiles =
// 5 rounds + 96 -> 1280 tiles + an 8192 x 768 remainder, 617 -> 607 us on
// packed operands (the remainder's 384 small tiles, 1.5 per CU, take ~85 us
// against the ~20 us their FLOPs would take at the large tiles' rate).
// Returns the cut (rows or columns, 0 for none).
struct TailCut { int64_t rows = 0, cols = 0; };

TailCut tail_cut(int64_t M, int64_t N) {
    TailCut c;
    const int64_t tm = (M + 255) / 256, tn = (N + 255) / 256, tiles = tm * tn;
    if (tiles < 256 || tiles % 256 == 0 || tiles % 256 > 128) return c;
    int64_t best = 0;
    for (int64_t n1 = tn - 1; n1 >= 1; --n1)
        if ((tm * n1) % 256 == 0) { best = tm * n1; c.cols = n1 * 256; break; }
    for (int64_t m1 = tm - 1; m1 >= 1; --m1)
        if ((m1 * tn) % 256 == 0) {
            if (m1 * tn > best) { c.cols = 0; c.rows = m1 * 256; }
            break;
        }
    return c;
}

}  // namespace

static int launch_gemm_one(const GemmArgs& a, hipStream_t st, bool cut);
static int launch_split_reduce(const GemmArgs& a, int splits, hipStream_t st);

namespace {

// Kernel variant, split count and kernel arguments of a GEMM that is not cut.
enum GemmVariant { kVarBig = 0, kVarSmall = 1, kVarNarrow = 2, kVarNarrow3 = 3 };
struct GemmPlan { int variant; int splits; GemmK k; };

// Whether a GEMM's final output goes out with nontemporal stores (the `nt`
// bit) instead of plain ones.  A plain store leaves the line dirty in the
// 256 MiB last-level cache, and its write-back to HBM then lands in
// whichever later kernel evicts it (the backward's first dY pass read 361 MB
// in 100.7 us after the forward's 361 MB plain output, against 67-71 us
// alone); nt stores write through while the GEMM, not HBM, is busy, and keep
// the output out of the L2 the operand tiles use.  Measured forward +
// backward, in one process against plain stores: [8192, 4096, 11008]
// 2186-2221 -> 2097-2109 us, [8192, 11008, 4096] 2087-2116 -> 2057-2067 us,
// [2048, 768, 3072] 83.4-84.7 -> 81.1-82.7 us.  The exception: one round of
// 256 x 256 tiles (at most one per CU) writes its whole output after the
// last K-step with nothing to overlap, and there the write-through is
// exposed (4096^3 forward 140.3-141.5 us plain against 143.2-144.1 us); and
// outputs under 4 MiB, which neither cache pressure nor write-back makes
// costly (64 x 1000 x 1000: 37.0 us plain against 37.7 us).  Split-K
// partials, read back at once by the reduction, stay plain.
bool gemm_streams_output(const GemmArgs& a, bool split) {
    if (split) return false;
    if ((int64_t)a.M * a.N * (a.out_dtype == AXS6_F32 ? 4 : 2) < ((int64_t)4 << 20)) return false;
    int bm, bn;
    cfg_tile(pick_cfg(a.M, a.N), &bm, &bn);
    return !(bm == 256 && tiles_of(a.M, a.N, bm, bn) <= 256);
}

int gemm_plan(const GemmArgs& a, GemmPlan* p) {
    const int iters = (int)(a.Kp / kGemmK);
    int splits = 1, per = iters;
    if (a.split_partial) {
        splits = gemm_split_count(a.M, a.N, a.Kp);
        per = (iters + splits - 1) / splits;
        if (a.split_bytes < gemm_split_bytes(a.M, a.N, a.Kp))
            return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: split-K buffer of %zu bytes, need %zu", a.split_bytes,
                        gemm_split_bytes(a.M, a.N, a.Kp));
    }
    const bool split = splits > 1;
    p->k = GemmK{a.A, a.lda, a.B, a.ldb, (int)a.M, (int)a.N, (int)a.Kp,
                 split ? nullptr : a.row_exp, split ? nullptr : a.col_exp, split ? nullptr : a.glob_exp, a.glob_add,
                 split ? nullptr : a.bias, split ? (void*)a.split_partial : a.out, split ? a.N : a.ldo,
                 split ? (int)AXS6_F32 : a.out_dtype, per, split ? a.M * a.N : 0,
                 gemm_streams_output(a, split) ? 1 : 0};
    p->splits = splits;
    const int cfg = pick_cfg(a.M, a.N);
    // a long contraction on the narrow tiles: a third slab in flight
    // (2048 x 768, K 3072: 28.5 -> 21.3 us; at K <= 1024 it costs 3-5%)
    p->variant = cfg == kCfgSmall ? kVarSmall
                 : cfg == kCfgNarrow ? (per >= kNarrowDeepSteps ? kVarNarrow3 : kVarNarrow) : kVarBig;
    return AXS6_OK;
}

int check_gemm_args(const GemmArgs& a) {
    if (a.Kp % 64 != 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: Kp (%lld) must be a multiple of 64", (long long)a.Kp);
    if (a.lda % 8 || a.ldb % 8 || (uintptr_t)a.A % 16 || (uintptr_t)a.B % 16)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: operands must be 16-byte aligned with ld a multiple of 8");
    if (a.Kp > a.lda || a.Kp > a.ldb) return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: Kp exceeds the leading dimension");
    if (a.ldo < a.N) return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: ldo (%lld) is smaller than N (%lld)",
                                 (long long)a.ldo, (long long)a.N);
    // buffer offsets are 32-bit: every operand byte (plus one tile of rows) must be addressable
    if ((a.M + 256) * a.lda * 2 >= ((int64_t)1 << 31) || (a.N + 256) * a.ldb * 2 >= ((int64_t)1 << 31))
        return fail(AXS6_ERR_UNSUPPORTED, "gemm: operand larger than 2 GiB");
    if (a.M > INT_MAX || a.N > INT_MAX || a.Kp > INT_MAX)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "gemm: dimension exceeds int32");
    return AXS6_OK;
}

}  // namespace

namespace {
// Whether a and b run as one pair launch (plans filled when they do).
bool pair_plans(const GemmArgs& a, const GemmArgs& b, GemmPlan* pa, GemmPlan* pb) {
    const TailCut ca = tail_cut(a.M, a.N), cb = tail_cut(b.M, b.N);
    const bool empty = a.M == 0 || a.N == 0 || b.M == 0 || b.N == 0;
    return !(empty || ca.rows || ca.cols || cb.rows || cb.cols || check_gemm_args(a) || check_gemm_args(b) ||
             gemm_plan(a, pa) || gemm_plan(b, pb) || pa->variant != pb->variant || pa->variant == kVarBig ||
             (pa->splits > 1 && pb->splits > 1));
}
}  // namespace

bool gemm_pairs(const GemmArgs& a, const GemmArgs& b) {
    GemmPlan pa, pb;
    return pair_plans(a, b, &pa, &pb);
}

int launch_gemm_pair(const GemmArgs& a, const GemmArgs& b, hipStream_t st) {
    GemmPlan pa, pb;
    int rc;
    if (!pair_plans(a, b, &pa, &pb)) {
        // one launch each: shapes the pair cannot share, the split buffer both
        // need, or the 256 x 256 tiles -- those launches run whole rounds of
        // tiles, and mixing two problems' tiles in one grid measured 1% slower
        // (8192 x 4096 x 11008 forward + backward 2.24 -> 2.26 ms)
        if ((rc = launch_gemm_f16(a, st))) return rc;
        return launch_gemm_f16(b, st);
    }
    // b's reduction job rides in its split reduction when b splits, else here
    const bool red_here = pb.splits == 1 && b.red_out && b.red_cols > 0;
    const GemmRedJob red{b.red_partial, b.red_chunks, b.red_cols, b.red_out,
                         red_here ? (int)((b.red_cols + kRedCols - 1) / kRedCols) : 0};
    switch (pa.variant) {   // the small-tile variants: 256 threads, as the reduction takes
        case kVarSmall: rc = run_gemm_lds_pair<128, 128, 64, 2, 2, 2>(pa.k, pa.splits, pb.k, pb.splits, red, st); break;
        case kVarNarrow3: rc = run_gemm_lds_pair<128, 64, 64, 3, 2, 2>(pa.k, pa.splits, pb.k, pb.splits, red, st); break;
        default: rc = run_gemm_lds_pair<128, 64, 64, 2, 2, 2>(pa.k, pa.splits, pb.k, pb.splits, red, st); break;
    }
    if (rc) return rc;
    if (pa.splits > 1 && (rc = launch_split_reduce(a, pa.splits, st))) return rc;
    if (pb.splits > 1 && (rc = launch_split_reduce(b, pb.splits, st))) return rc;
    return AXS6_OK;
}

bool gemm_splits(const GemmArgs& a) {
    if (!a.split_partial || a.M == 0 || a.N == 0) return false;
    const TailCut c = tail_cut(a.M, a.N);
    return !(c.rows || c.cols) && gemm_split_count(a.M, a.N, a.Kp) > 1 &&
           a.split_bytes >= gemm_split_bytes(a.M, a.N, a.Kp);
}

int launch_gemm_f16(const GemmArgs& a, hipStream_t st) { return launch_gemm_one(a, st, true); }

static int launch_gemm_one(const GemmArgs& a, hipStream_t st, bool cut) {
    if (a.M == 0 || a.N == 0) return AXS6_OK;
    int rc0 = check_gemm_args(a);
    if (rc0) return rc0;
    if (cut) {
        const TailCut c = tail_cut(a.M, a.N);
        if (c.rows || c.cols) {
            const int esize = a.out_dtype == AXS6_F32 ? 4 : 2;
            GemmArgs head = a, tail = a;
            // both parts have enough tiles for one workgroup per CU: no split-K
            head.split_partial = tail.split_partial = nullptr;
            head.split_bytes = tail.split_bytes = 0;
            if (c.cols) {
                head.N = c.cols;
                tail.N = a.N - c.cols;
                tail.B = a.B + c.cols * a.ldb;
                if (a.col_exp) tail.col_exp = a.col_exp + c.cols;
                if (a.bias) tail.bias = a.bias + c.cols;
                tail.out = (char*)a.out + c.cols * esize;
            } else {
                head.M = c.rows;
                tail.M = a.M - c.rows;
                tail.A = a.A + c.rows * a.lda;
                if (a.row_exp) tail.row_exp = a.row_exp + c.rows;
                tail.out = (char*)a.out + c.rows * a.ldo * esize;
            }
            const int rc = launch_gemm_one(head, st, false);
            return rc ? rc : launch_gemm_one(tail, st, false);
        }
    }
    GemmPlan p;
    int rc = gemm_plan(a, &p);
    if (rc) return rc;
    switch (p.variant) {
        case kVarSmall: rc = run_gemm_lds<128, 128, 64, 2, 2, 2>(p.k, p.splits, st); break;
        case kVarNarrow3: rc = run_gemm_lds<128, 64, 64, 3, 2, 2>(p.k, p.splits, st); break;
        case kVarNarrow: rc = run_gemm_lds<128, 64, 64, 2, 2, 2>(p.k, p.splits, st); break;
        default: rc = run_gemm_lds<256, 256, 64, 2, 2, 4, 4>(p.k, p.splits, st); break;   // kVarBig
    }
    if (rc || p.splits == 1) return rc;
    return launch_split_reduce(a, p.splits, st);
}

static int launch_split_reduce(const GemmArgs& a, int splits, hipStream_t st) {
    const int64_t groups = a.M * ((a.N + 3) / 4);
    const int64_t sblocks = (groups + kSplitGroups - 1) / kSplitGroups;
    const int64_t rblocks = a.red_out && a.red_cols > 0 ? (a.red_cols + kRedCols - 1) / kRedCols : 0;
    SplitReduceK r{a.split_partial, splits, a.M * a.N, (int)a.M, (int)a.N, a.row_exp, a.col_exp, a.glob_exp,
                   a.glob_add, a.bias, a.out, a.ldo, a.out_dtype,
                   sblocks, a.red_partial, a.red_chunks, a.red_cols, a.red_out};
    splitk_reduce_kernel<<<dim3((unsigned)(sblocks + rblocks)), 256, 0, st>>>(r);
    return check_launch("gemm_splitk_reduce");
}

}  // namespace axs6
