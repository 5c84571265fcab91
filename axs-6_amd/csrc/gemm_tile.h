// Device building blocks of the fp16 MFMA GEMM tiles (gfx950), shared by the
// plain GEMM (gemm_f16.hip) and the forward with streamed operand packing
// (nf5_linear_stream.hip): the XOR-swizzled LDS slab layout, the per-wave
// accumulator tile and its 16x16x32 MFMA K-step, the epilogue that leaves
// through LDS as whole-row-segment stores, and vmcnt waits with immediate
// counts.
#pragma once

#include <limits.h>

#include "linear_internal.h"

namespace axs6 {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4m __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));

constexpr int kBufferConfig = 0x00020000;   // raw 32-bit buffer access, gfx9 family

__device__ __forceinline__ uint16_t to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// LDS layout of a K-slab: row r of the tile holds BK halves = BK/8 slots of
// 16 bytes; logical chunk c of row r lives in slot c ^ key(r).  gfx950's LDS
// serves a 16-lane group of ds_read_b128 from 64 four-byte banks, i.e. 256
// bytes, which covers 256/(2*BK) consecutive rows; key(r) is taken from the
// row bits above those so that the 16 rows of a fragment read fill the 64
// banks exactly once (measured with the key on the low row bits instead:
// SQ_LDS_BANK_CONFLICT at 50% of LDS-active cycles; with this key, 0).
template <int BK>
__device__ __forceinline__ int swz_key(int row) {
    constexpr int SHIFT = BK == 64 ? 1 : 2;   // log2(256 / (2 * BK))
    return (row >> SHIFT) & (BK / 8 - 1);
}
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
    return row * (BK * 2) + ((chunk ^ swz_key<BK>(row)) << 4);
}

// The wave's accumulators for a WM x WN sub-tile: 16x16 blocks of
// v_mfma_f32_16x16x32_f16, 4 floats per lane (128 per lane for a 128x64
// sub-tile).  The 16x16x32 instruction runs the same FLOPs per cycle as the
// 32x32x16 one with half-size fragments and, in the 256x256 tiles, clocks
// higher under the power limit (3-5% shorter GEMMs at 4096^3 and the Llama
// shapes than the same kernel on 32x32x16 blocks).
template <int WM, int WN> struct WaveAcc {
    static constexpr int TM = WM / 16, TN = WN / 16, R = 4;
    f32x4m v[TM][TN];
};

// One K-step on 16x16 blocks: per 32-deep slice, lane l reads row l%16 of
// its A and B blocks at K-group l/16 (chunk 4*slice + l/16; 16 consecutive
// rows per 16-lane group, conflict-free under swz), then TM x TN MFMAs.
template <int BK, int WM, int WN>
__device__ __forceinline__ void mma_step16(WaveAcc<WM, WN>& acc, const char* as, const char* bs, int a_row0,
                                           int b_row0, int fq) {
    constexpr int TM = WaveAcc<WM, WN>::TM, TN = WaveAcc<WM, WN>::TN;
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
        const int chunk = kk * 4 + fq;
        f16x8 af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const f16x8*>(as + swz<BK>(a_row0 + i * 16, chunk));
#pragma unroll
        for (int j = 0; j < TN; ++j) bf[j] = *reinterpret_cast<const f16x8*>(bs + swz<BK>(b_row0 + j * 16, chunk));
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc.v[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc.v[i][j], 0, 0, 0);
    }
    __builtin_amdgcn_iglp_opt(1);
}

// Stages the wave's 32-row block row i (32 x WN floats, row stride LDW) in
// LDS: accumulator r of block (2i+h, j) is row 16*h + 4*(lane/16) + r,
// column lane%16 of the 16x16 block.  The write pattern is bank-conflict
// free with LDW = WN + 4.
template <int WM, int WN, int LDW>
__device__ __forceinline__ void stage_block_row(const WaveAcc<WM, WN>& acc, int i, float* ws, int lane) {
    const int fc = lane & 15, fq = lane >> 4;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < WaveAcc<WM, WN>::TN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) ws[(h * 16 + fq * 4 + r) * LDW + j * 16 + fc] = acc.v[2 * i + h][j][r];
}

// Writes 4 consecutive output values of row `row` starting at column `col`
// (col % 4 == 0): one vector store when the 4 columns exist and the row
// segment is aligned, else element by element up to N.
__device__ __forceinline__ void store4(void* out, int64_t ldo, int N, int out_dtype, int row, int col,
                                       const float (&v)[4], bool vec) {
    const int64_t o = (int64_t)row * ldo + col;
    if (vec && col + 3 < N) {
        if (out_dtype == AXS6_F32) {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + o) = make_float4(v[0], v[1], v[2], v[3]);
        } else if (out_dtype == AXS6_BF16) {
            uint2 w;
            w.x = (uint32_t)to_bf16(v[0]) | ((uint32_t)to_bf16(v[1]) << 16);
            w.y = (uint32_t)to_bf16(v[2]) | ((uint32_t)to_bf16(v[3]) << 16);
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) = w;
        } else {
            typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
            f16x4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            *reinterpret_cast<f16x4*>(reinterpret_cast<_Float16*>(out) + o) = h;
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (col + t >= N) break;
        if (out_dtype == AXS6_F32) reinterpret_cast<float*>(out)[o + t] = v[t];
        else if (out_dtype == AXS6_BF16) reinterpret_cast<uint16_t*>(out)[o + t] = to_bf16(v[t]);
        else reinterpret_cast<_Float16*>(out)[o + t] = (_Float16)v[t];
    }
}

// A store with the nontemporal hint (the `nt` bit) when NT, else a plain one.
// The choice is a template argument: with a run-time flag the compiler
// merges the two stores of the branch into one and drops the hint.
template <bool NT, typename T>
__device__ __forceinline__ void st_hint(T v, T* p) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// store4 with the output type fixed at compile time; `full` = the 4 columns
// exist and the row segment is aligned for one vector store.  NT: nontemporal
// stores.  A plain store leaves the line dirty in the last-level cache
// (256 MiB), and its write-back to HBM then lands in whichever later kernel
// evicts it: a 361 MB read after a 360 MB plain fill took 109 us against
// 69 us after the same fill with nt stores (the fill 53 against 67 us).  The
// GEMM's caller picks per launch (gemm_streams_output).
template <int OUT, bool NT>
__device__ __forceinline__ void store4t(void* out, int64_t ldo, int N, int row, int col, const float (&v)[4],
                                        bool full) {
    const int64_t o = (int64_t)row * ldo + col;
    if (full) {
        if constexpr (OUT == AXS6_F32) {
            const f32x4m w = {v[0], v[1], v[2], v[3]};
            st_hint<NT>(w, reinterpret_cast<f32x4m*>(reinterpret_cast<float*>(out) + o));
        } else if constexpr (OUT == AXS6_BF16) {
            typedef uint32_t u32x2g __attribute__((ext_vector_type(2)));
            const u32x2g w = {(uint32_t)to_bf16(v[0]) | ((uint32_t)to_bf16(v[1]) << 16),
                              (uint32_t)to_bf16(v[2]) | ((uint32_t)to_bf16(v[3]) << 16)};
            st_hint<NT>(w, reinterpret_cast<u32x2g*>(reinterpret_cast<uint16_t*>(out) + o));
        } else {
            typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
            const f16x4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            st_hint<NT>(h, reinterpret_cast<f16x4*>(reinterpret_cast<_Float16*>(out) + o));
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (col + t >= N) break;
        if constexpr (OUT == AXS6_F32) st_hint<NT>(v[t], reinterpret_cast<float*>(out) + o + t);
        else if constexpr (OUT == AXS6_BF16) st_hint<NT>(to_bf16(v[t]), reinterpret_cast<uint16_t*>(out) + o + t);
        else st_hint<NT>((_Float16)v[t], reinterpret_cast<_Float16*>(out) + o + t);
    }
}

// The wave's share of the epilogue: per 32-row block row i of its sub-tile,
// stage the accumulators in LDS (row stride LDW floats), then read back
// 4 consecutive columns per lane for all PASSES row groups and their row
// exponents at once -- one LDS wait per block row instead of two per row
// group -- and write them with the output type fixed at compile time.
template <int OUT, bool NT, int WM, int WN, int LDW>
__device__ __forceinline__ void epilogue_store(const WaveAcc<WM, WN>& acc, float* ws, const int (&rexp_l)[WM / 64],
                                               const int (&cexp)[4], const float (&cbias)[4], void* out, int64_t ldo,
                                               int M, int N, int row0, int gcol, bool vec, int lane) {
    constexpr int LANES_PER_ROW = WN / 4;
    constexpr int ROWS_PER_PASS = 64 / LANES_PER_ROW;
    constexpr int PASSES = 32 / ROWS_PER_PASS;
    const int c4 = (lane % LANES_PER_ROW) * 4;
    const int rsub = lane / LANES_PER_ROW;
    const bool full = vec && gcol + 3 < N;
#pragma unroll
    for (int i = 0; i < WM / 32; ++i) {
        stage_block_row<WM, WN, LDW>(acc, i, ws, lane);
        float4 q[PASSES];
        int rx[PASSES];
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int lr = p * ROWS_PER_PASS + rsub;
            q[p] = *reinterpret_cast<const float4*>(ws + lr * LDW + c4);
            // row i*32 + lr of the wave tile: register i/2 of lane (i%2)*32 + lr
            rx[p] = __shfl(rexp_l[i / 2], (i % 2) * 32 + lr, 64);
        }
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int grow = row0 + i * 32 + p * ROWS_PER_PASS + rsub;
            if (grow < M && gcol < N) {
                float v[4] = {__builtin_amdgcn_ldexpf(q[p].x, rx[p] + cexp[0]) + cbias[0],
                              __builtin_amdgcn_ldexpf(q[p].y, rx[p] + cexp[1]) + cbias[1],
                              __builtin_amdgcn_ldexpf(q[p].z, rx[p] + cexp[2]) + cbias[2],
                              __builtin_amdgcn_ldexpf(q[p].w, rx[p] + cexp[3]) + cbias[3]};
                store4t<OUT, NT>(out, ldo, N, grow, gcol, v, full);
            }
        }
    }
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Waits until at most `ahead` slabs of IPW loads each are outstanding
// (ahead <= MAXA, wave-uniform): s_waitcnt takes an immediate count.
template <int MAXA, int IPW>
__device__ __forceinline__ void wait_slabs(int ahead) {
    if constexpr (MAXA == 0) {
        wait_vmcnt<0>();
    } else {
        if (ahead >= MAXA) wait_vmcnt<MAXA * IPW>();
        else wait_slabs<MAXA - 1, IPW>(ahead);
    }
}

// Origin (m0, n0) of workgroup `bid`'s BM x BN output tile: workgroup ids are
// dispatched round-robin over the 8 XCDs, so the id is remapped to give each
// XCD a contiguous range of the grouped order (kGroupM rows of tiles per
// group), whose A rows and B columns then stay inside that XCD's L2.
constexpr int kGroupM = 8;

template <int BM, int BN>
__device__ __forceinline__ void tile_origin_mn(int M, int N, int bid, int& m0, int& n0) {
    const int tiles_m = (M + BM - 1) / BM;
    const int tiles_n = (N + BN - 1) / BN;
    const int total = tiles_m * tiles_n;
    if (total % 8 == 0) bid = (bid % 8) * (total / 8) + bid / 8;
    const int per_group = kGroupM * tiles_n;
    const int group = bid / per_group;
    const int first_m = group * kGroupM;
    const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int in_group = bid - group * per_group;
    m0 = (first_m + in_group % gsize) * BM;
    n0 = (in_group / gsize) * BN;
}

}  // namespace
}  // namespace axs6
