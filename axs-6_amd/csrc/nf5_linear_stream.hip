// Quantized linear forward with the operand packing streamed through the
// GEMM (gfx950): Y = FQ(X) FQ(W)^T + b in one launch whose workgroups both
// pack the operands and contract them, for outputs whose 256x256 tiles fit
// one workgroup per CU (4096 x 4096: 256 tiles on 256 CUs).
//
// Why.  The two-launch forward (pack X and W, then the GEMM) runs the
// packing alone (~33 us at 4096^3, latency-bound, the shader clock at its
// maximum) and then the power-capped GEMM (~110 us).  Here the packing of
// K-chunk c+1 runs in the VALU and memory slots of the waves that multiply
// chunk c, so only the first chunk's packing is exposed.
//
// Chunked shifts.  A row's packing needs the power-of-two shift that brings
// its largest value under fp16's range, and with whole-row shifts that needs
// the whole row before any chunk can be packed.  Here the shift is a running
// maximum along the row, one per (row, 512-wide K-chunk):
//   S(r, 0) = m(r, 0) + kHead - 15,  S(r, c) = max(S(r, c-1), m(r, c) - 15)
// with m(r, c) the chunk's largest finite nonzero block exponent e1 (INT_MIN
// while the row has none).  Chunk c of row r is stored as
// fp16(FQ(x) * 2^-S(r, c)), |value| <= 2^15, and its shift goes to a table.
// A tile accumulates in units of 2^(S_x(r, c) + S_w(n, c)); when a chunk
// raises a shift, the accumulators of that row (or column) are scaled by
// 2^-(increase) first -- exact, and rare: the first chunk's shift leaves
// kHead binades of headroom.  Where both shifts keep every value in fp16's
// normal range, each packed value is the two-launch path's value times a
// power of two, so Y is bit-identical to that path's.
//
// Workgroup (one 256x256 tile, 8 waves, 2 K-slabs in LDS as the plain GEMM):
//   waves 0-3  issue the K-slab loads (HBM/L2 -> LDS) and multiply;
//   waves 4-7  pack their rows' next chunk (raw values prefetched into LDS a
//              step ahead with buffer_load ... lds), then multiply.  On a
//              SIMD the packing wave's VALU work runs while the loading
//              wave's MFMAs keep the matrix core busy.
// Rows of [X; W] are dealt out round-robin over the workgroups and, inside
// one, over the packing waves; every workgroup packs every chunk of its rows.
//
// Publication.  Packing waves publish chunk c with an agent-scope release
// and an increment of the chunk's counter (the L2s of the 8 XCDs are not
// coherent with each other); wave 0 of every workgroup polls the counter of
// chunk c+1 before the loads of chunk c+1's first slab and acquires at agent
// scope.  Chunk 0 is packed by all 8 waves before the K loop (the only
// exposed packing).  The poll is bounded (kSpinLimit): a workgroup that times
// out sets the error flag, writes NaN to its tile and finishes, so a launch
// never hangs.  Every workgroup must be resident at once (the host checks
// the tile count against the CU count and the occupancy); concurrent
// launches on one device must use different counter slots.  The last
// workgroup to finish resets the counters for the next launch.
#include <limits.h>

#include <atomic>

#include "nf5_device.h"
#include "gemm_tile.h"

namespace axs6 {
namespace {

constexpr int kCh = 512;                 // K values per packing chunk
constexpr int kSpc = kCh / 64;           // 64-deep K-steps per chunk
constexpr int kHead = 4;                 // headroom binades of a row's first shift
[[maybe_unused]] constexpr int kAhead = 2;              // chunks packed ahead of the one being multiplied
constexpr int kMaxChunks = 64;           // K up to 32768
constexpr int kSlots = 16;               // flag sets for launches that overlap in time
constexpr int kMaxG = 1024;              // workgroups (one per CU)
constexpr int kMaxPps = 2;               // row-chunks a packing wave packs per K-step
constexpr int kMaxRpp = kMaxPps * kSpc;  // rows per packing wave
constexpr int kMaxRowsPerWg = 4 * kMaxRpp;
[[maybe_unused]] constexpr uint32_t kSpinLimit = 1u << 22;  // polls of ~0.15 us: ~0.6 s before a workgroup gives up
constexpr int kF16Max = 15;
constexpr int kWT = 17;                  // buffer store cache policy sc0 sc1: written through to memory

// Per slot: each workgroup's published-chunk word, the slot's launch count
// (zero-initialised at load) and the timeout flag.  A launch with count g
// publishes chunk c of workgroup b as flag[b] = g * 65 + (chunks done); the
// words only grow, so nothing is reset between launches.
__device__ uint32_t g_stream_flag[kSlots][kMaxG];
__device__ uint32_t g_stream_gen[kSlots];
__device__ int g_stream_err;

struct StreamK {
    const void* x; const void* w;        // [M, K], [N, K], dtype DT
    int M, N, K, Kp, T, G;               // Kp = 64 * ceil(K / 64), T = ceil(Kp / kCh), G workgroups
    int Mp, Np;                          // shift-table row strides (multiples of 32: whole 128-byte lines per chunk)
    int rows_wg, rpp, pps;               // rows per workgroup, per packing wave, per step
    bool quantize_x;
    const float* bias; void* y;          // y [M, N], dtype DT
    _Float16* xq; _Float16* wq;          // [M, Kp], [N, Kp]
    int32_t* sx; int32_t* sw;            // [T, Mp], [T, Np]
    uint32_t* flag; uint32_t* gen;       // this launch's slot
    int* err;
    const float* lut; const uint8_t* band;
};

// v[0..V) * 2^sh (or * factor) as V fp16 values packed in u32 words
template <int V>
__device__ __forceinline__ void halves_ldexp(uint32_t (&wv)[V / 2], const float* v, int sh) {
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
        const uint16_t lo = __builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(v[2 * i], sh));
        const uint16_t hi = __builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(v[2 * i + 1], sh));
        wv[i] = lo | ((uint32_t)hi << 16);
    }
}
template <int V>
__device__ __forceinline__ void halves_mul(uint32_t (&wv)[V / 2], const float* v, float factor) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int i = 0; i < V / 2; ++i) {
        const f32x2 t = {v[2 * i] * factor, v[2 * i + 1] * factor};
        wv[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(t, f16x2));
    }
}

// shift increase from a to b (both INT_MIN-or-defined): 0 unless both defined
__device__ __forceinline__ int shift_rise(int a, int b) { return (a == INT_MIN || b == INT_MIN) ? 0 : b - a; }

template <int DT, int BS>
struct Packer {
    using E = Elem<DT>;
    static constexpr int V = E::V;
    static constexpr int NVL = kCh / V / 64;            // 16-byte vectors per lane per row-chunk
    static constexpr int GL = BS / V > 0 ? BS / V : 1;  // lanes per NF5 block
    static constexpr bool DEFER = DT != AXS6_F16;       // +-lut values, block scale folded into the store
    static constexpr int ROW_BYTES = kCh * (int)sizeof(typename E::S);
};

// Packs chunk c of row `row` of [X; W] from the raw 16-byte vectors raw[u]
// (vector l + 64u of the chunk; zeros past K) and returns the row's new
// running shift, given the previous one (INT_MIN: none yet).  The packed
// values (zeros between K and Kp) and the shift table entry are written
// through to memory (the consumers run on other XCDs).
template <int DT, int BS>
__device__ __forceinline__ int pack_row_chunk(const StreamK& k, __amdgpu_buffer_rsrc_t xq_rsrc,
                                              __amdgpu_buffer_rsrc_t wq_rsrc, int row, int c,
                                              const u32x4 (&raw)[Packer<DT, BS>::NVL], int s_prev,
                                              const float* lut_s, const float* lut_fast, const uint8_t* band_s,
                                              int lane) {
    using P = Packer<DT, BS>;
    using E = typename P::E;
    constexpr int V = P::V, NVL = P::NVL;
    const bool is_x = row < k.M;
    const int r = is_x ? row : row - k.M;
    const bool fq = !is_x || k.quantize_x;
    float f[NVL][V];
    int e1v[NVL];
    int cm = INT_MIN;
#pragma unroll
    for (int u = 0; u < NVL; ++u) {
        E::unpack(raw[u], f[u]);
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const uint32_t a = __float_as_uint(f[u][e]) & 0x7fffffffu;
            m = m > a ? m : a;
        }
        m = group_umax<P::GL>(m);
        const FqScale s = fq_scale(m, band_s);
        e1v[u] = INT_MIN;
        if (fq) {
            if constexpr (P::DEFER) {
                const bool full = fq_vector_unscaled<V>(f[u], s, lut_s, lut_fast);
                if (full) round_to_elem<DT>(f[u]);
                else e1v[u] = s.e1;
            } else {
                const float d[V] = {};
                fq_vector<V>(f[u], s, lut_s, false, d);
                round_to_elem<DT>(f[u]);
            }
        }
        const bool finite_block = !(s.nan_block || s.inf_scale || m == 0u);
        if (finite_block) cm = s.e1 > cm ? s.e1 : cm;
    }
    cm = wave_imax(cm);
    int s_new;
    if (s_prev == INT_MIN) s_new = cm == INT_MIN ? INT_MIN : cm + kHead - kF16Max;
    else s_new = (cm != INT_MIN && cm - kF16Max > s_prev) ? cm - kF16Max : s_prev;
    const int s_use = s_new == INT_MIN ? 0 : s_new;
    const int base = (r * k.Kp + c * kCh) * 2;         // byte offset of the chunk in its packed operand
    const int lim = k.Kp - c * kCh;                     // halves of this chunk inside Kp
#pragma unroll
    for (int u = 0; u < NVL; ++u) {
        const int off = (lane + 64 * u) * V;
        if (off < lim) {
            uint32_t wv[V / 2];
            // e1 <= S + 15, so 2^(e1 - S) <= 2^15; below 2^-149 it is 0, as is the fp16 of anything that small
            if (e1v[u] != INT_MIN) halves_mul<V>(wv, f[u], __builtin_amdgcn_ldexpf(1.0f, e1v[u] - s_use));
            else halves_ldexp<V>(wv, f[u], -s_use);
            const __amdgpu_buffer_rsrc_t rs = is_x ? xq_rsrc : wq_rsrc;
            if constexpr (V == 8) {
                typedef uint32_t u32x4b __attribute__((ext_vector_type(4)));
                __builtin_amdgcn_raw_buffer_store_b128(u32x4b{wv[0], wv[1], wv[2], wv[3]}, rs, base + off * 2, 0, kWT);
            } else {
                typedef uint32_t u32x2b __attribute__((ext_vector_type(2)));
                __builtin_amdgcn_raw_buffer_store_b64(u32x2b{wv[0], wv[1]}, rs, base + off * 2, 0, kWT);
            }
        }
    }
    if (lane == 0)
        __hip_atomic_store((is_x ? k.sx + (int64_t)c * k.Mp : k.sw + (int64_t)c * k.Np) + r, s_new, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    return s_new;
}

// Byte offset of 16-byte vector q of chunk c of row `row` in its raw
// operand, or an offset past every buffer (the load reads zeros) when the
// vector lies past K.
template <int DT>
__device__ __forceinline__ int raw_offset(const StreamK& k, int row, int c, int q) {
    constexpr int V = Elem<DT>::V;
    const int col = c * kCh + q * V;
    if (col >= k.K) return INT_MIN;                       // 0x80000000: out of range
    const int r = row < k.M ? row : row - k.M;
    return (r * k.K + col) * (int)sizeof(typename Elem<DT>::S);
}

template <int DT, int BS>
__global__ __launch_bounds__(512, 1) void linear_stream_kernel(StreamK k) {
#if defined(__HIP_DEVICE_COMPILE__)  // LDS-DMA builtins exist only in the device pass
    using P = Packer<DT, BS>;
    using S = typename P::E::S;
    constexpr int BM = 256, BN = 256, BK = 64, WGM = 2, WGN = 4, LW = 4;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int RB = BK * 2;
    constexpr int SPR = BK / 8;
    constexpr int ROWS_PER_INST = 1024 / RB;
    constexpr int A_INST = BM / ROWS_PER_INST / LW, B_INST = BN / ROWS_PER_INST / LW;
    constexpr int SLAB = (BM + BN) * RB;
    constexpr int STAGES = 2;
    constexpr bool ROUNDED_LUT = DT == AXS6_BF16;
    // LDS, all dynamic: the K-slabs at offset 0 (as in the plain GEMM), then
    // the packing waves' staging and the small tables (stream_lds_bytes)
    extern __shared__ __align__(16) char smem[];
    char* stage_base = smem + STAGES * SLAB;              // packing waves' raw-value staging
    char* tail = stage_base + 4 * kMaxPps * P::ROW_BYTES;
    float* lut_s = reinterpret_cast<float*>(tail);
    float* lutr_s = lut_s + kLutSize;                     // bf16 only: the LUT rounded to bf16
    uint32_t* band_w = reinterpret_cast<uint32_t*>(lutr_s + (ROUNDED_LUT ? kLutSize : 0));
    int* cur_x = reinterpret_cast<int*>(band_w + kBandSize / 4);   // the tile's row / column shifts
    int* cur_w = cur_x + BM;                              // of the current chunk
    int* rise_x = cur_w + BN;                             // their increase at the latest boundary
    int* rise_w = rise_x + BM;
    int* s_run = rise_w + BN;                             // running shifts of this workgroup's packed rows
    int& timed_out = s_run[kMaxRowsPerWg];
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const bool loader = wave < LW;
    const int bid = blockIdx.x;
    int m0, n0;
    tile_origin_mn<BM, BN>(k.M, k.N, bid, m0, n0);
    // this slot's launch count: every workgroup reads it before publishing
    // anything; workgroup 0 advances it at the end, after it has seen every
    // workgroup's last chunk
    const uint32_t gen0 = __hip_atomic_load(k.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t fbase = gen0 * (uint32_t)(kMaxChunks + 1);

    if constexpr (ROUNDED_LUT) {
        if (tid < kLutSize / 4) {
            const float4 v = reinterpret_cast<const float4*>(k.lut)[tid];
            float4 r;
            r.x = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.x)); r.y = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.y));
            r.z = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.z)); r.w = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(v.w));
            reinterpret_cast<float4*>(lutr_s)[tid] = r;
        }
    }
    if (tid == 0) timed_out = 0;
    stage_tables(lut_s, band_w, k.lut, k.band);           // ends with a barrier
    const float* lut_fast = ROUNDED_LUT ? lutr_s : lut_s;

    const __amdgpu_buffer_rsrc_t xr_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(k.x), 0, (int)((int64_t)k.M * k.K * (int64_t)sizeof(S)), kBufferConfig);
    const __amdgpu_buffer_rsrc_t wr_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(k.w), 0, (int)((int64_t)k.N * k.K * (int64_t)sizeof(S)), kBufferConfig);
    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)k.xq, 0, (int)((int64_t)k.M * k.Kp * 2), kBufferConfig);
    const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)k.wq, 0, (int)((int64_t)k.N * k.Kp * 2), kBufferConfig);
    auto lds_ptr = [](char* p) { return (__attribute__((address_space(3))) void*)p; };
    const int rows_total = k.M + k.N;
    // row j of this workgroup is row bid + G * j of [X; W]
    auto wg_row = [&](int j) { return bid + k.G * j; };
    auto publish = [&](uint32_t chunks_done) {
        // every wave's packed values and shifts have been written through and
        // acknowledged (each waited for its stores); then the word, at agent scope
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        if (lane == 0) __hip_atomic_store(k.flag + bid, fbase + chunks_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    // ---- prologue: chunks 0 .. kAhead-1 of this workgroup's rows, all 8 waves
    const int P0 = k.T < kAhead ? k.T : kAhead;
    constexpr int PB = 4;                                 // rows' loads in flight together
    for (int pc = 0; pc < P0; ++pc) {
        for (int j0 = wave; j0 < k.rows_wg; j0 += 8 * PB) {
            u32x4 raw[PB][P::NVL];
#pragma unroll
            for (int b = 0; b < PB; ++b) {
                const int j = j0 + 8 * b, row = wg_row(j);
                const bool live = j < k.rows_wg && row < rows_total;
                const bool is_x = row < k.M;
                const u32x4* src = reinterpret_cast<const u32x4*>(
                    reinterpret_cast<const S*>(is_x ? k.x : k.w) + (int64_t)(is_x ? row : row - k.M) * k.K + pc * kCh);
#pragma unroll
                for (int u = 0; u < P::NVL; ++u) {
                    const int q = lane + 64 * u;
                    raw[b][u] = (live && pc * kCh + q * P::V < k.K) ? src[q] : u32x4{0u, 0u, 0u, 0u};
                }
            }
#pragma unroll
            for (int b = 0; b < PB; ++b) {
                const int j = j0 + 8 * b, row = wg_row(j);
                if (j >= k.rows_wg || row >= rows_total) break;
                const int sn = pack_row_chunk<DT, BS>(k, a_rsrc, b_rsrc, row, pc, raw[b], pc == 0 ? INT_MIN : s_run[j],
                                                      lut_s, lut_fast, band_s, lane);
                if (lane == 0) s_run[j] = sn;
            }
        }
    }
    wait_vmcnt<0>();                                      // this wave's stores acknowledged
    __syncthreads();
    if (wave == 0) publish((uint32_t)P0);

    // packing-wave schedule: wave p packs rows j = p + 4i (i < rpp) of chunk
    // c + kAhead during chunk c, pps of them per K-step after its MFMAs,
    // finished at step s_pub; published after the next barrier
    const int pw = wave - LW;
    const int s_pub = k.rpp > 0 ? (k.rpp + k.pps - 1) / k.pps - 1 : 0;
    char* stage = stage_base + (pw > 0 ? pw : 0) * (kMaxPps * P::ROW_BYTES);
    // the LDS-DMA prefetch of the row-chunks packed at (chunk c, step s)
    auto prefetch = [&](int c, int s) {
#pragma unroll
        for (int h = 0; h < kMaxPps; ++h) {
            const int i = s * k.pps + h;
            if (h >= k.pps || i >= k.rpp) break;
            const int row = wg_row(pw + 4 * i);
            if (row >= rows_total) break;
            const bool is_x = row < k.M;
#pragma unroll
            for (int u = 0; u < P::NVL; ++u) {
                const int off = raw_offset<DT>(k, row, c, lane + 64 * u);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(is_x ? xr_rsrc : wr_rsrc,
                                                         lds_ptr(stage + h * P::ROW_BYTES + u * 1024), 16, off, 0, 0, 0);
            }
        }
    };
    if (!loader && k.T > kAhead) prefetch(kAhead, 0);

    // ---- wait until every workgroup has published `need` chunks ----------
    auto acquire_chunks = [&](uint32_t need) {
        if (wave == 0) {
            const uint32_t want = fbase + need;
            uint32_t spins = 0;
            for (;;) {
                bool ok = true;
                for (int i = lane; i < k.G; i += 64)
                    ok &= (int)(__hip_atomic_load(k.flag + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - want) >= 0;
                if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
                if (++spins > kSpinLimit) {
                    if (lane == 0) { timed_out = 1; atomicOr(k.err, 1); }
                    break;
                }
                __builtin_amdgcn_s_sleep(4);
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
    };
    auto tile_shift = [&](int c) {
        // thread t < 256: tile row m0 + t; else tile column n0 + t - 256
        if (tid < BM) return m0 + tid < k.M ? k.sx[(int64_t)c * k.Mp + m0 + tid] : INT_MIN;
        return n0 + tid - BM < k.N ? k.sw[(int64_t)c * k.Np + n0 + tid - BM] : INT_MIN;
    };
    acquire_chunks(1);
    {
        const int s0 = tile_shift(0);
        if (tid < BM) cur_x[tid] = s0; else cur_w[tid - BM] = s0;
    }

    // ---- K loop (the plain GEMM's, plus chunk boundaries and packing) ------
    const int lrow = lane / SPR, lslot = lane % SPR;
    int a_goff[A_INST], a_loff[A_INST], b_goff[B_INST], b_loff[B_INST];
#pragma unroll
    for (int i = 0; i < A_INST; ++i) {
        const int row = (wave % LW + LW * i) * ROWS_PER_INST + lrow;
        a_goff[i] = (int)((int64_t)(m0 + row) * k.Kp * 2) + ((lslot ^ swz_key<BK>(row)) << 4);
        a_loff[i] = (wave % LW + LW * i) * 1024;
    }
#pragma unroll
    for (int i = 0; i < B_INST; ++i) {
        const int row = (wave % LW + LW * i) * ROWS_PER_INST + lrow;
        b_goff[i] = (int)((int64_t)(n0 + row) * k.Kp * 2) + ((lslot ^ swz_key<BK>(row)) << 4);
        b_loff[i] = BM * RB + (wave % LW + LW * i) * 1024;
    }
    using Acc = WaveAcc<WM, WN>;
    Acc acc;
#pragma unroll
    for (int i = 0; i < Acc::TM; ++i)
#pragma unroll
        for (int j = 0; j < Acc::TN; ++j)
#pragma unroll
            for (int r = 0; r < Acc::R; ++r) acc.v[i][j][r] = 0.0f;

    const int KT = k.Kp / BK;
    if (loader) {
#pragma unroll
        for (int i = 0; i < A_INST; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, lds_ptr(smem + a_loff[i]), 16, a_goff[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < B_INST; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, lds_ptr(smem + b_loff[i]), 16, b_goff[i], 0, 0, 0);
    }
    const int fr = lane % 16, fg = lane / 16;
    const int a_row0 = wm * WM + fr, b_row0 = wn * WN + fr;
    int nshift = INT_MIN;      // this thread's tile row / column shift of the next chunk
    int pending = 0;           // packing wave LW: chunks done to publish after the next barrier (0: none)
    for (int kt = 0; kt < KT; ++kt) {
        const int c = kt / kSpc, s = kt - c * kSpc;
        const bool last_of_chunk = s == kSpc - 1 && c + 1 < k.T;
        if (loader) wait_vmcnt<0>();                       // slab kt has landed
        if (last_of_chunk) {
            acquire_chunks((uint32_t)(c + 2));             // chunk c+1 from every workgroup
            nshift = tile_shift(c + 1);
        } else {
            __builtin_amdgcn_s_barrier();
        }
        if (pending) {                                     // (wave LW only) every packing wave's stores are in
            publish((uint32_t)pending);
            pending = 0;
        }
        if (loader && kt + 1 < KT) {
            char* slab = smem + ((kt + 1) % STAGES) * SLAB;
#pragma unroll
            for (int i = 0; i < A_INST; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rsrc, lds_ptr(slab + a_loff[i]), 16, a_goff[i] + (kt + 1) * RB, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < B_INST; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, lds_ptr(slab + b_loff[i]), 16, b_goff[i] + (kt + 1) * RB, 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        const char* slab = smem + (kt % STAGES) * SLAB;
        mma_step16<BK, WM, WN>(acc, slab, slab + BM * RB, a_row0, b_row0, fg);
        __builtin_amdgcn_sched_barrier(0);
        // packing waves, after their MFMAs (whose issue covers the loading
        // waves' slab-load burst): row-chunks [s*pps, (s+1)*pps) of chunk c + kAhead
        if (!loader && c + kAhead < k.T && s <= s_pub) {
            wait_vmcnt<0>();                               // the prefetch issued a step ago has landed
#pragma unroll
            for (int h = 0; h < kMaxPps; ++h) {
                const int i = s * k.pps + h;
                if (h >= k.pps || i >= k.rpp) break;
                const int j = pw + 4 * i;
                const int row = wg_row(j);
                if (row >= rows_total) break;
                u32x4 raw[P::NVL];
#pragma unroll
                for (int u = 0; u < P::NVL; ++u)
                    raw[u] = *reinterpret_cast<const u32x4*>(stage + h * P::ROW_BYTES + u * 1024 + lane * 16);
                const int sn = pack_row_chunk<DT, BS>(k, a_rsrc, b_rsrc, row, c + kAhead, raw, s_run[j], lut_s,
                                                      lut_fast, band_s, lane);
                if (lane == 0) s_run[j] = sn;
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0): staging read before the DMA rewrites it
            if (s == s_pub) {
                wait_vmcnt<0>();                           // this wave's stores of the chunk acknowledged
                if (wave == LW) pending = c + kAhead + 1;
            }
            if (s < s_pub) prefetch(c + kAhead, s + 1);
            else if (c + kAhead + 1 < k.T) prefetch(c + kAhead + 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (last_of_chunk) {
            // chunk c's products are in; move the accumulators to chunk c+1's
            // units: the rise of each tile row / column shift, then the
            // accumulators of the rows and columns that rose scaled by
            // 2^-(rise) (rows, then columns: powers of two <= 1; the branch is
            // uniform per wave).  Placed after the MFMA block: ahead of it, the
            // compiler keeps the fragments and the scaling live together.
            if (tid < BM) { rise_x[tid] = shift_rise(cur_x[tid], nshift); cur_x[tid] = nshift; }
            else { rise_w[tid - BM] = shift_rise(cur_w[tid - BM], nshift); cur_w[tid - BM] = nshift; }
            __syncthreads();
            int any = 0;
#pragma unroll
            for (int i = 0; i < Acc::TM; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) any |= rise_x[wm * WM + i * 16 + fg * 4 + q];
#pragma unroll
            for (int j = 0; j < Acc::TN; ++j) any |= rise_w[wn * WN + j * 16 + fr];
            if (__builtin_amdgcn_ballot_w64(any != 0) != 0) {
#pragma unroll
                for (int i = 0; i < Acc::TM; ++i)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float f = __builtin_amdgcn_ldexpf(1.0f, -rise_x[wm * WM + i * 16 + fg * 4 + q]);
#pragma unroll
                        for (int j = 0; j < Acc::TN; ++j) acc.v[i][j][q] *= f;
                    }
#pragma unroll
                for (int j = 0; j < Acc::TN; ++j) {
                    const float f = __builtin_amdgcn_ldexpf(1.0f, -rise_w[wn * WN + j * 16 + fr]);
#pragma unroll
                    for (int i = 0; i < Acc::TM; ++i)
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc.v[i][j][q] *= f;
                }
            }
        }
    }
    if (pending) publish((uint32_t)pending);           // a last step's chunk (not read by this launch's tiles)

    // ---- epilogue: 2^(S_x(r) + S_w(n)) of the last chunk, + bias ----------
    wait_vmcnt<0>();
    __syncthreads();
    if (timed_out) {
#pragma unroll
        for (int i = 0; i < Acc::TM; ++i)
#pragma unroll
            for (int j = 0; j < Acc::TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) acc.v[i][j][q] = __builtin_nanf("");
    }
    constexpr int LDW = WN + 4;
    constexpr int LANES_PER_ROW = WN / 4;
    float* ws = reinterpret_cast<float*>(smem) + wave * (32 * LDW);
    const int gcol = n0 + wn * WN + (lane % LANES_PER_ROW) * 4;
    int cexp[4];
    float cbias[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const bool in = gcol + t < k.N;
        const int sw_ = cur_w[wn * WN + (lane % LANES_PER_ROW) * 4 + t];
        cexp[t] = (in && sw_ != INT_MIN) ? sw_ : 0;
        cbias[t] = (k.bias && in) ? k.bias[gcol + t] : 0.0f;
    }
    constexpr int RPL = WM / 64;
    int rexp_l[RPL];
#pragma unroll
    for (int q = 0; q < RPL; ++q) {
        const int sx_ = cur_x[wm * WM + q * 64 + lane];
        rexp_l[q] = sx_ == INT_MIN ? 0 : sx_;
    }
    constexpr int ES = (int)sizeof(S);
    const bool vec = (k.N % 4 == 0) && ((uintptr_t)k.y % (4 * ES) == 0);
    epilogue_store<DT, WM, WN, LDW>(acc, ws, rexp_l, cexp, cbias, k.y, k.N, k.M, k.N, m0 + wm * WM, gcol, vec, true,
                                    lane);
    // workgroup 0 has seen every workgroup's chunk T-1 (chunk 0 when T == 1),
    // so every workgroup has read this launch's count: advance it
    if (bid == 0 && tid == 0) __hip_atomic_store(k.gen, gen0 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#endif
}

// Device addresses of the flag sets, launch counts and the error flag, per device.
struct StreamSyms { uint32_t* flag = nullptr; uint32_t* gen = nullptr; int* err = nullptr; };

int stream_syms(StreamSyms* out) {
    static StreamSyms cache[64];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(AXS6_ERR_NO_DEVICE, "no current HIP device");
    if (!cache[dev].flag) {
        void* f = nullptr;
        void* g = nullptr;
        void* e = nullptr;
        hipError_t rc = hipGetSymbolAddress(&f, HIP_SYMBOL(g_stream_flag));
        if (rc == hipSuccess) rc = hipGetSymbolAddress(&g, HIP_SYMBOL(g_stream_gen));
        if (rc == hipSuccess) rc = hipGetSymbolAddress(&e, HIP_SYMBOL(g_stream_err));
        if (rc != hipSuccess || !f || !g || !e)
            return fail(AXS6_ERR_HIP, "stream linear: symbol lookup failed: %s", hipGetErrorString(rc));
        cache[dev].flag = (uint32_t*)f;
        cache[dev].gen = (uint32_t*)g;
        cache[dev].err = (int*)e;
    }
    *out = cache[dev];
    return AXS6_OK;
}

int cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return n;
}

constexpr size_t kWsAlign = 256;
inline size_t ws_align(size_t v) { return (v + kWsAlign - 1) / kWsAlign * kWsAlign; }

struct StreamPlan {
    int64_t Kp, T, G, Mp, Np, rows_wg, rpp, pps;
    size_t xq, wq, sx, sw, total;   // workspace offsets
};

// Whether the shape runs on the streamed kernel, and its launch plan: one
// round of 256x256 tiles on at least 3/4 of the CUs (fewer tiles leave CUs
// idle and put more rows on each workgroup), K up to kMaxChunks chunks, at
// most kMaxRpp rows per packing wave, operands within 32-bit buffer offsets.
int stream_plan(int64_t M, int64_t N, int64_t K, int dtype, StreamPlan* p) {
    if (M <= 0 || N <= 0 || K <= 0) return AXS6_ERR_UNSUPPORTED;
    p->Kp = pad_to(K, kGemmK);
    p->T = (p->Kp + kCh - 1) / kCh;
    p->G = ((M + 255) / 256) * ((N + 255) / 256);
    const int cus = cu_count();
    if (p->T > kMaxChunks || cus <= 0 || cus > kMaxG || p->G > cus || 4 * p->G < 3 * cus) return AXS6_ERR_UNSUPPORTED;
    p->rows_wg = (M + N + p->G - 1) / p->G;
    p->rpp = (p->rows_wg + 3) / 4;
    if (p->rpp > kMaxRpp || p->rows_wg > kMaxRowsPerWg) return AXS6_ERR_UNSUPPORTED;
    p->pps = (p->rpp + kSpc - 1) / kSpc;
    if (p->pps < 1) p->pps = 1;
    const int64_t es = dtype == AXS6_F32 ? 4 : 2;
    if (M * K * es >= ((int64_t)1 << 31) || N * K * es >= ((int64_t)1 << 31) ||
        (M + 256) * p->Kp * 2 >= ((int64_t)1 << 31) || (N + 256) * p->Kp * 2 >= ((int64_t)1 << 31))
        return AXS6_ERR_UNSUPPORTED;
    p->Mp = pad_to(M, 32);
    p->Np = pad_to(N, 32);
    size_t off = 0;
    auto take = [&](size_t b) { size_t o = off; off = ws_align(off + b); return o; };
    p->xq = take((size_t)M * p->Kp * 2);
    p->wq = take((size_t)N * p->Kp * 2);
    p->sx = take((size_t)p->T * p->Mp * 4);
    p->sw = take((size_t)p->T * p->Np * 4);
    p->total = off;
    return AXS6_OK;
}

// Dynamic LDS of the kernel: 2 K-slabs, 4 packing waves' staging, the LUT
// (and its bf16 rounding), the band table, 4 x 256 shifts, the running
// shifts and the timeout flag.
template <int DT>
size_t stream_lds_bytes(int row_bytes) {
    return (size_t)2 * (256 + 256) * 64 * 2 + (size_t)4 * kMaxPps * row_bytes +
           sizeof(float) * kLutSize * (DT == AXS6_BF16 ? 2 : 1) + kBandSize + sizeof(int) * (4 * 256 + kMaxRowsPerWg + 1);
}

template <int DT, int BS>
int launch_stream(const StreamK& k, hipStream_t st) {
    using P = Packer<DT, BS>;
    const size_t lds = stream_lds_bytes<DT>(P::ROW_BYTES);
    static bool checked = false;
    static int occ = 0;
    if (!checked) {
        (void)hipFuncSetAttribute((const void*)linear_stream_kernel<DT, BS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, linear_stream_kernel<DT, BS>, 512, lds) != hipSuccess)
            occ = 0;
        checked = true;
    }
    if (occ < 1) return fail(AXS6_ERR_UNSUPPORTED, "stream linear: the kernel does not fit a CU");
    linear_stream_kernel<DT, BS><<<dim3((unsigned)k.G), 512, lds, st>>>(k);
    return check_launch("linear_stream");
}

}  // namespace
}  // namespace axs6

using namespace axs6;

extern "C" size_t axs6_nf5_linear_forward_stream_workspace(int64_t M, int64_t N, int64_t K, int32_t dtype) {
    StreamPlan p;
    if (!valid_dtype(dtype) || stream_plan(M, N, K, dtype, &p) != AXS6_OK) return 0;
    return p.total;
}

extern "C" int axs6_nf5_linear_forward_stream(const void* x, const void* w, const float* bias, void* y, int32_t dtype,
                                              int64_t M, int64_t N, int64_t K, int32_t block_size,
                                              int32_t quantize_input, void* workspace, size_t workspace_bytes,
                                              void* stream) {
    const char* fn = "axs6_nf5_linear_forward_stream";
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    if (!valid_block(block_size))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: block_size must be 8, 16 or 32 (got %d)", fn, block_size);
    if (M < 0 || N < 0 || K < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative dimension", fn);
    const int64_t vm = dtype == AXS6_F32 ? 4 : 8;
    if (K % vm != 0)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: K (%lld) must be a multiple of %lld", fn, (long long)K,
                    (long long)vm);
    if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: dimension too large", fn);
    StreamPlan p;
    if (stream_plan(M, N, K, dtype, &p) != AXS6_OK)
        return fail(AXS6_ERR_UNSUPPORTED, "%s: shape %lld x %lld x %lld does not fit one round of 256x256 tiles "
                    "(use axs6_nf5_linear_forward)", fn, (long long)M, (long long)K, (long long)N);
    if (!x || !w || !y) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if ((uintptr_t)x % 16 || (uintptr_t)w % 16) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: x and w must be 16-byte aligned", fn);
    if (!workspace || workspace_bytes < p.total || (uintptr_t)workspace % kWsAlign)
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: workspace of %zu bytes (256-byte aligned) required, got %zu", fn,
                    p.total, workspace_bytes);
    DeviceTables t;
    int rc = device_tables(&t);
    if (rc) return rc;
    StreamSyms sy;
    if ((rc = stream_syms(&sy))) return rc;
    static std::atomic<uint32_t> next_slot{0};
    const uint32_t slot = next_slot.fetch_add(1) % kSlots;
    char* ws = (char*)workspace;
    StreamK k{x, w, (int)M, (int)N, (int)K, (int)p.Kp, (int)p.T, (int)p.G, (int)p.Mp, (int)p.Np, (int)p.rows_wg,
              (int)p.rpp, (int)p.pps, quantize_input != 0, bias, y, (_Float16*)(ws + p.xq), (_Float16*)(ws + p.wq),
              (int32_t*)(ws + p.sx), (int32_t*)(ws + p.sw), sy.flag + (size_t)slot * kMaxG, sy.gen + slot, sy.err,
              t.lut, t.band};
    hipStream_t st = (hipStream_t)stream;
#define AXS6_STREAM_BS(DT_)                                                  \
    do {                                                                     \
        if (block_size == 32) return launch_stream<DT_, 32>(k, st);          \
        if (block_size == 16) return launch_stream<DT_, 16>(k, st);          \
        return launch_stream<DT_, 8>(k, st);                                 \
    } while (0)
    if (dtype == AXS6_F32) AXS6_STREAM_BS(AXS6_F32);
    if (dtype == AXS6_BF16) AXS6_STREAM_BS(AXS6_BF16);
    AXS6_STREAM_BS(AXS6_F16);
#undef AXS6_STREAM_BS
}

extern "C" int axs6_nf5_linear_stream_error(int32_t* flag) {
    if (!flag) return fail(AXS6_ERR_INVALID_ARGUMENT, "axs6_nf5_linear_stream_error: null pointer");
    StreamSyms sy;
    int rc = stream_syms(&sy);
    if (rc) return rc;
    int v = 0;
    hipError_t e = hipMemcpy(&v, sy.err, sizeof(int), hipMemcpyDeviceToHost);
    if (e == hipSuccess && v) {
        const int zero = 0;
        e = hipMemcpy(sy.err, &zero, sizeof(int), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) return fail(AXS6_ERR_HIP, "axs6_nf5_linear_stream_error: %s", hipGetErrorString(e));
    *flag = v;
    return AXS6_OK;
}
