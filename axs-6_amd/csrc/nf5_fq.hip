// NF5 fake-quantize, quantize and dequantize kernels for gfx950.
//
// Per block of 8/16/32 values along the last dim (the arithmetic of
// fused_fake_quantize, axs/unified/quantize_unified.py:121-204):
//   amax   = max |x|                     (NaN if any element is NaN)
//   e1     = floor(log2(max(amax, 2^-149))) + 1, taken from the exponent
//            bits plus the log2 rounding band (see axs6_runtime.hip)
//   scale  = 2^e1 (inf when e1 >= 128; 1 for all-zero blocks)
//   idx    = clamp(trunc((|x| / scale) * 1023), 0, 1023)
//            (stochastic: trunc((|x|/scale + (U - 0.5)/1023) * 1023))
//   y      = (sign(x) * lut[idx]) * scale
// Every step rounds exactly as torch's CPU float32 ops do, so the output is
// bit-identical to the reference's eager path (FP contraction is off).
//
// Layout and launch.  Fast path (cols % block == 0, 16-byte aligned
// pointers): the tensor is one contiguous run of blocks; each lane loads one
// 16-byte vector (4 x f32 or 8 x bf16/f16), so a 32-value f32 block spans 8
// neighbouring lanes and its amax is a 3-step DPP butterfly (quad_perm x2,
// row_half_mirror) -- no LDS round trip.  A wave instruction moves 1 KiB of
// contiguous HBM; each thread keeps kUnroll vectors in flight.  The 4 KiB
// LUT and the band table are staged in LDS once per workgroup and the grid
// is capped (grid-stride loop) so that staging is amortised.
// Row path (rows of >= 64 values with a ragged last block, or unaligned
// views): four values (or one) per lane in row order, a block is
// `block` / 4 (or `block`) neighbouring lanes (DPP / permlane maximum), rows
// cut into segments of 256 (or 64) values, the next segment's loads in
// flight (fq_rows_kernel).  Shorter rows: whole rows per wave, one value per
// lane, block maxima by segmented shuffle reductions (fq_short_kernel).
#include <math.h>

#include <type_traits>

#pragma clang fp contract(off)

#include "nf5_device.h"

namespace axs6 {
namespace {

// Streaming loads and stores carry the nontemporal hint: the kernel reads
// each input once and writes each output once.  At 8192x4096 f32 on inputs
// and outputs past the 256 MiB last-level cache (HBM-cold, 4 rotating
// buffers) 45.1 us against 48.6 us for plain accesses (3 vectors in flight
// per thread; 2, 4, 5, 6 and 8 measured 47.1, 45.5, 46.0, 46.8 and 47.1 us;
// nontemporal stores alone 46.4 us).  An input replayed from the last-level
// cache reads slower with the hint (44.1 against 39.5 us): the hint trades
// that warm case for the cold one.
__device__ __forceinline__ u32x4 stream_load(const u32x4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void stream_store(u32x4 v, u32x4* p) { __builtin_nontemporal_store(v, p); }

// ---- fake-quantize kernels -----------------------------------------------

template <int DT, int BS, bool STOCH>
__global__ __launch_bounds__(kThreads) void fq_vec_kernel(const typename Elem<DT>::S* x,
                                                          typename Elem<DT>::S* y, int64_t n_vec,
                                                          const float* __restrict__ lut_g,
                                                          const uint8_t* __restrict__ band_g,
                                                          uint64_t seed, const uint64_t* __restrict__ seed_dev, uint64_t offset) {
    using E = Elem<DT>;
    const uint64_t key = STOCH ? dither_key(seed + (seed_dev ? *seed_dev : 0ull)) : 0ull;
    constexpr int V = E::V;
    constexpr int G = BS / V;
    static_assert(G >= 1 && G <= 8, "group size");
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    u32x4* yv = reinterpret_cast<u32x4*>(y);
    const int tid = threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * (kThreads * kUnroll);
    // The first tile's HBM loads go out before the LUT is staged, so the two
    // latencies overlap; later tiles are prefetched one iteration ahead.
    int64_t base = (int64_t)blockIdx.x * (kThreads * kUnroll);
    u32x4 raw[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t vi = base + u * kThreads + tid;
        raw[u] = vi < n_vec ? stream_load(xv + vi) : u32x4{0u, 0u, 0u, 0u};
    }
    stage_tables(lut_s, band_w, lut_g, band_g);
    for (; base < n_vec; base += step) {
        u32x4 nxt[kUnroll];
        const int64_t nbase = base + step;
        if (nbase < n_vec) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t vi = nbase + u * kThreads + tid;
                nxt[u] = vi < n_vec ? stream_load(xv + vi) : u32x4{0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            int64_t vi = base + u * kThreads + tid;
            float f[V];
            E::unpack(raw[u], f);
            uint32_t m = 0;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                uint32_t a = __float_as_uint(f[j]) & 0x7fffffffu;
                m = m > a ? m : a;
            }
            m = group_umax<G>(m);
            FqScale s = fq_scale(m, band_s);
            float d[V];
            const DitherVec dv = dither_vec(key, offset + (uint64_t)(vi * V));
#pragma unroll
            for (int j = 0; j < V; ++j) d[j] = STOCH ? dither_step(dv, j) : 0.0f;
            fq_vector<V>(f, s, lut_s, STOCH, d);
            if (vi < n_vec) stream_store(E::pack(f), yv + vi);
        }
        if (nbase < n_vec) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) raw[u] = nxt[u];
        }
    }
}

// Rows under 64 values that do not tile into vectors of whole blocks: each
// wave takes R = 64 / cols whole rows per step, lane l holding value l of the
// wave's contiguous run of R * cols values, so loads and stores are
// consecutive and at most cols - 1 lanes idle.  A lane's block is the run of
// lanes from the block's first value to its end (BS values, or the row's end
// for a ragged last block); its maximum is a segmented suffix maximum
// (log2(BS) shuffle steps that never cross the block's end) read back from
// the block's first lane.  Lanes past the run, and rows past the tensor,
// form blocks of their own holding 0 and store nothing.
// Four consecutive values at p (aligned to four values) from floats.
template <int DT>
__device__ __forceinline__ void store4(typename Elem<DT>::S* p, const float (&f)[4]) {
    using E = Elem<DT>;
    if constexpr (DT == AXS6_F32) {
        *reinterpret_cast<u32x4*>(p) = E::pack(f);
    } else {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const float g[8] = {f[0], f[1], f[2], f[3], 0.0f, 0.0f, 0.0f, 0.0f};
        const u32x4 w = E::pack(g);
        *reinterpret_cast<u32x2*>(p) = u32x2{w.x, w.y};
    }
}

// Rows too short for the row-segment layout (under 64 values, or under 256
// with four values per lane): each wave takes R = 64 * VL / cols whole rows
// per step, lane l holding values VL*l .. VL*l + VL-1 of the wave's
// contiguous run of R * cols values, so loads and stores are consecutive
// (VL = 4: the rows are whole 4-value groups, x and y aligned to them, one
// 16-byte f32 or 8-byte 16-bit access per lane) and at most cols - 1 values'
// lanes idle.  A lane's block is the run of lanes from the block's first
// value to its end (BS values, or the row's end for a ragged last block);
// its maximum is a segmented suffix maximum (log2(BS / VL) shuffle steps
// that never cross the block's end) read back from the block's first lane.
// Lanes past the run, and rows past the tensor, form blocks of their own
// holding 0 and store nothing.
template <int DT, int BS, bool STOCH, int VL>
__global__ __launch_bounds__(kThreads) void fq_short_kernel(const typename Elem<DT>::S* __restrict__ x,
                                                            typename Elem<DT>::S* __restrict__ y, int64_t rows,
                                                            int cols, const float* __restrict__ lut_g,
                                                            const uint8_t* __restrict__ band_g, uint64_t seed,
                                                            const uint64_t* __restrict__ seed_dev, uint64_t offset) {
    using E = Elem<DT>;
    static_assert(VL == 1 || VL == 4, "values per lane");
    const uint64_t key = STOCH ? dither_key(seed + (seed_dev ? *seed_dev : 0ull)) : 0ull;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    stage_tables(lut_s, band_w, lut_g, band_g);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int lane = threadIdx.x & 63;
    const int R = 64 * VL / cols;                  // whole rows per wave step
    const int pos = VL * lane;                     // first value of the lane in the run
    const bool in_run = pos < R * cols;
    const int lr = pos / cols;                     // row of the lane within the step
    const int row0 = lr * cols;
    const int bstart = row0 + ((pos - row0) & ~(BS - 1));
    const int bstop = bstart + BS < row0 + cols ? bstart + BS : row0 + cols;
    const int b0 = in_run ? bstart / VL : lane;                       // first lane of the block
    const int bend = in_run ? (bstop + VL - 1) / VL : lane + 1;       // one past its last lane
    const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int64_t rstep = (int64_t)gridDim.x * (kThreads / 64) * R;
    for (int64_t r0 = wave * R; r0 < rows; r0 += rstep) {
        const int64_t base = r0 * cols;
        const bool valid = in_run && r0 + lr < rows;
        float f[VL];
        if constexpr (VL == 1) {
            f[0] = valid ? E::to_f(x[base + pos]) : 0.0f;
        } else if constexpr (DT == AXS6_F32) {
            const u32x4 w = valid ? *reinterpret_cast<const u32x4*>(x + base + pos) : u32x4{0u, 0u, 0u, 0u};
            E::unpack(w, f);
        } else {
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 h = valid ? *reinterpret_cast<const u32x2*>(x + base + pos) : u32x2{0u, 0u};
            float g[8];
            E::unpack(u32x4{h.x, h.y, 0u, 0u}, g);
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = g[e];
        }
        uint32_t v = 0;
#pragma unroll
        for (int e = 0; e < VL; ++e) {
            const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
            v = v > a ? v : a;
        }
#pragma unroll
        for (int d = 1; d < BS / VL; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_down((int)v, (unsigned)d, 64);
            if (lane + d < bend) v = v > o ? v : o;
        }
        const uint32_t m = (uint32_t)__shfl((int)v, b0, 64);
        const FqScale s = fq_scale(m, band_s);
        float d[VL];
#pragma unroll
        for (int e = 0; e < VL; ++e) d[e] = STOCH ? dither_step(key, offset + (uint64_t)(base + pos + e)) : 0.0f;
        fq_vector<VL>(f, s, lut_s, STOCH, d);
        if (valid) {
            if constexpr (VL == 1) y[base + pos] = E::from_f(f[0]);
            else store4<DT>(y + base + pos, f);
        }
    }
}

// Rows that do not tile into 16-byte vectors of whole blocks (a ragged last
// block, or row starts off 16-byte alignment): VL values per lane (4 when
// the row length is a multiple of 4 and the pointers allow 4-value loads,
// else 1), lanes in row order, so a block is BS / VL neighbouring lanes and
// its maximum a DPP (and, for 32 lanes, permlane) reduction; a load or store
// instruction covers 64 * VL consecutive values of one row.  A row is cut
// into segments of 64 * VL * U values (a multiple of BS, so blocks never
// straddle segments); each wave walks a contiguous range of segments,
// stepping its row index instead of dividing, with the next segment's loads
// in flight.  Lanes past the row's end read 0 -- the reference's zero
// padding of the last block -- and store nothing.
template <int DT, int BS, bool STOCH, int U, int VL>
__global__ __launch_bounds__(kThreads) void fq_rows_kernel(const typename Elem<DT>::S* __restrict__ x,
                                                           typename Elem<DT>::S* __restrict__ y, int64_t rows,
                                                           int64_t cols, int64_t segs_per_row, int64_t segs_per_wave,
                                                           const float* __restrict__ lut_g,
                                                           const uint8_t* __restrict__ band_g, uint64_t seed,
                                                           const uint64_t* __restrict__ seed_dev, uint64_t offset) {
    using E = Elem<DT>;
    constexpr int SEG = 64 * VL * U;
    static_assert(VL == 1 || VL == 4, "values per lane");
    static_assert(SEG % BS == 0 && BS % VL == 0, "segments hold whole blocks");
    const uint64_t key = STOCH ? dither_key(seed + (seed_dev ? *seed_dev : 0ull)) : 0ull;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    stage_tables(lut_s, band_w, lut_g, band_g);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t total = rows * segs_per_row;
    int64_t seg = wave * segs_per_wave;
    const int64_t end = seg + segs_per_wave < total ? seg + segs_per_wave : total;
    if (seg >= end) return;
    int64_t r = seg / segs_per_row;
    int64_t sx = seg - r * segs_per_row;
    // raw words of segment (row rr, index ss) for this lane, zero past the
    // row's end; converted to floats only when the segment is processed, so
    // the loads of the next segment stay in flight meanwhile
    using Raw = typename std::conditional<VL == 1, typename E::S, u32x4>::type;
    auto load_seg = [&](int64_t rr, int64_t ss, Raw (&w)[U]) {
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t c = ss * SEG + VL * lane + 64 * VL * k;
            if constexpr (VL == 1) {
                w[k] = c < cols ? x[rr * cols + c] : (typename E::S)0;
            } else if constexpr (DT == AXS6_F32) {
                w[k] = c < cols ? *reinterpret_cast<const u32x4*>(x + rr * cols + c) : u32x4{0u, 0u, 0u, 0u};
            } else {
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 h = c < cols ? *reinterpret_cast<const u32x2*>(x + rr * cols + c) : u32x2{0u, 0u};
                w[k] = u32x4{h.x, h.y, 0u, 0u};
            }
        }
    };
    Raw nw[U];
    load_seg(r, sx, nw);
    for (; seg < end; ++seg) {
        const int64_t base = r * cols;
        float f[U][VL];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            if constexpr (VL == 1) {
                f[k][0] = E::to_f(nw[k]);
            } else {
                float g[E::V];
                E::unpack(nw[k], g);
#pragma unroll
                for (int e = 0; e < VL; ++e) f[k][e] = g[e];
            }
        }
        int64_t rn = r, sn = sx + 1;
        if (sn == segs_per_row) {
            sn = 0;
            ++rn;
        }
        if (seg + 1 < end) load_seg(rn, sn, nw);
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t c = sx * SEG + VL * lane + 64 * VL * k;
            uint32_t a = 0;
#pragma unroll
            for (int e = 0; e < VL; ++e) {
                const uint32_t b = __float_as_uint(f[k][e]) & 0x7fffffffu;
                a = a > b ? a : b;
            }
            uint32_t m;
            if constexpr (VL == 1) m = lanes_umax<BS>(a);
            else m = group_umax<BS / VL>(a);
            const FqScale s = fq_scale(m, band_s);
            float d[VL];
#pragma unroll
            for (int e = 0; e < VL; ++e) d[e] = STOCH ? dither_step(key, offset + (uint64_t)(base + c + e)) : 0.0f;
            fq_vector<VL>(f[k], s, lut_s, STOCH, d);
            if (c < cols) {
                if constexpr (VL == 1) y[base + c] = E::from_f(f[k][0]);
                else store4<DT>(y + base + c, f[k]);
            }
        }
        r = rn;
        sx = sn;
    }
}

// ---- quantize / dequantize -------------------------------------------------

// quantize_unified (quantize_unified.py:211-282): shared exponent
// e = clamp(floor(log2(amax)) + 1 + 127, 0, 255) (0 for zero blocks and for
// NaN / inf amax, whose int32 cast is INT_MIN), scale = 2^(e-127),
// idx as above with the normalised value clamped to [0, 1], code =
// reverse_lut[idx], sign = x < 0.  Optionally also writes FQ(x).
template <int DT, int BS, bool STOCH>
__global__ __launch_bounds__(kThreads) void quantize_kernel(
    const typename Elem<DT>::S* x, int64_t rows, int64_t cols, int64_t nblk,
    const float* __restrict__ lut_g, const uint8_t* __restrict__ band_g,
    const uint8_t* __restrict__ rev_g, uint64_t seed, const uint64_t* __restrict__ seed_dev, uint64_t offset, uint8_t* __restrict__ exps,
    uint8_t* __restrict__ codes, uint8_t* __restrict__ signs, typename Elem<DT>::S* fq) {
    using E = Elem<DT>;
    const uint64_t key = STOCH ? dither_key(seed + (seed_dev ? *seed_dev : 0ull)) : 0ull;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ uint8_t rev_s[kLutSize];
    reinterpret_cast<uint32_t*>(rev_s)[threadIdx.x] = reinterpret_cast<const uint32_t*>(rev_g)[threadIdx.x];
    stage_tables(lut_s, band_w, lut_g, band_g);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    constexpr int BPW = 64 / BS;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t total = rows * nblk;
    const int64_t wstep = (int64_t)gridDim.x * (kThreads / 64) * BPW;
    for (int64_t wb = ((int64_t)blockIdx.x * (kThreads / 64) + wave) * BPW; wb < total; wb += wstep) {
        const int64_t blk = wb + lane / BS;
        const int j = lane % BS;
        const bool vb = blk < total;
        const int64_t r = vb ? blk / nblk : 0;
        const int64_t c = (vb ? blk - r * nblk : 0) * BS + j;
        const bool valid = vb && c < cols;
        const int64_t gi = r * cols + c;
        float f = valid ? E::to_f(x[gi]) : 0.0f;
        uint32_t ab = __float_as_uint(f) & 0x7fffffffu;
        uint32_t m = group_umax_shfl<BS>(ab);
        const float d = STOCH ? dither_step(key, offset + (uint64_t)gi) : 0.0f;

        // shared exponent
        int e = (m == 0u || m >= kInfBits) ? 0 : floor_log2_torch(m, band_s) + 1 + kExpBias;
        e = e < 0 ? 0 : (e > 255 ? 255 : e);
        const int se = e - kExpBias;               // scale = 2^se, se in [-127, 128]
        float n;
        if (se >= 128) n = ab >= kInfBits ? __uint_as_float(kNanBits) : 0.0f;   // x / inf
        else n = __builtin_amdgcn_ldexpf(__uint_as_float(ab), -se);
        n = (n > 1.0f) ? 1.0f : n;                 // clamp(0, 1); NaN passes through
        const int idx = lut_index(n, STOCH, d);
        if (vb) {
            const int64_t o = blk * BS + j;
            codes[o] = rev_s[idx];
            if (signs) signs[o] = f < 0.0f ? 1 : 0;
            if (j == 0) exps[blk] = (uint8_t)e;
        }
        if (fq) {
            FqScale s = fq_scale(m, band_s);
            float v = fq_value(f, s, lut_s, STOCH, d);
            if (valid) fq[gi] = E::from_f(v);
        }
    }
}

// quantize_unified of V values of one block whose maximum |x| bits are m:
// the shared exponent (returned), the V codes and V signs as bytes packed
// little-endian into cw / sw, and, with want_fq, f replaced by its FQ values.
// When no lane of the wave holds a block with a NaN or an infinite scale or
// an exponent below kFastMinE1 (one ballot, so the branch is uniform), the
// shared exponent is e1 + 127 (0 for a zero block) without a clamp and one
// LUT index serves the code and the FQ value (fq_vector's short sequence;
// its range argument bounds the index); otherwise the general sequence.
template <int V, bool STOCH>
__device__ __forceinline__ int quant_values(float (&f)[V], uint32_t m, const float (&d)[V], const float* lut_s,
                                            const uint8_t* band_s, const uint8_t* rev_s, bool want_fq,
                                            uint32_t (&cw)[2], uint32_t (&sw)[2]) {
    cw[0] = cw[1] = sw[0] = sw[1] = 0u;
#pragma unroll
    for (int e = 0; e < V; ++e) sw[e / 4] |= (f[e] < 0.0f ? 1u : 0u) << (8 * (e % 4));
    const FqScale sc = fq_scale(m, band_s);
    int ex;
    if (__builtin_amdgcn_ballot_w64(sc.nan_block || sc.inf_scale || sc.e1 < kFastMinE1) == 0) {
        ex = sc.zero ? 0 : sc.e1 + kExpBias;
        const float c = __builtin_amdgcn_ldexpf(1023.0f, -sc.e1);
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const uint32_t xb = __float_as_uint(f[e]);
            const uint32_t ab = xb & 0x7fffffffu;
            const float t = STOCH ? (__builtin_amdgcn_ldexpf(__uint_as_float(ab), -sc.e1) + d[e]) * 1023.0f
                                  : lut_pos(ab, c);
            const int idx = (int)t;
            cw[e / 4] |= (uint32_t)rev_s[idx] << (8 * (e % 4));
            if (want_fq) {
                const float mag = __builtin_amdgcn_ldexpf(lut_s[idx], sc.e1);
                const uint32_t nz = (uint32_t)((int32_t)(ab + 0x7fffffffu) >> 31);
                f[e] = __uint_as_float((__float_as_uint(mag) ^ (xb & 0x80000000u)) & nz);
            }
        }
    } else {
        ex = (m == 0u || m >= kInfBits) ? 0 : floor_log2_torch(m, band_s) + 1 + kExpBias;
        ex = ex < 0 ? 0 : (ex > 255 ? 255 : ex);
        const int se = ex - kExpBias;          // scale = 2^se, se in [-127, 128]
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const uint32_t ab = __float_as_uint(f[e]) & 0x7fffffffu;
            float n;
            if (se >= 128) n = ab >= kInfBits ? __uint_as_float(kNanBits) : 0.0f;   // x / inf
            else n = __builtin_amdgcn_ldexpf(__uint_as_float(ab), -se);
            n = (n > 1.0f) ? 1.0f : n;         // clamp(0, 1); NaN passes through
            const int idx = lut_index(n, STOCH, d[e]);
            cw[e / 4] |= (uint32_t)rev_s[idx] << (8 * (e % 4));
        }
        if (want_fq) fq_vector<V>(f, sc, lut_s, STOCH, d);
    }
    return ex;
}

// Vector form of quantize_kernel for rows that tile into whole blocks
// (cols % BS == 0: codes and signs are then the flat [rows * cols] layout,
// exponents one per BS flat values) and aligned pointers: each lane takes one
// 16-byte vector of V values, a block is G = BS / V neighbouring lanes (DPP
// amax), and the lane writes its V codes and V signs as one V-byte store.
// Same arithmetic and dither counters as quantize_kernel.
template <int DT, int BS, bool STOCH>
__global__ __launch_bounds__(kThreads) void quantize_vec_kernel(
    const typename Elem<DT>::S* x, int64_t n_vec, const float* __restrict__ lut_g, const uint8_t* __restrict__ band_g,
    const uint8_t* __restrict__ rev_g, uint64_t seed, const uint64_t* __restrict__ seed_dev, uint64_t offset,
    uint8_t* __restrict__ exps, uint8_t* __restrict__ codes, uint8_t* __restrict__ signs, typename Elem<DT>::S* fq) {
    using E = Elem<DT>;
    constexpr int V = E::V;
    constexpr int G = BS / V > 0 ? BS / V : 1;
    static_assert(BS % V == 0, "a vector lies inside one block");
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const uint64_t key = STOCH ? dither_key(seed + (seed_dev ? *seed_dev : 0ull)) : 0ull;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ uint8_t rev_s[kLutSize];
    const u32x4* xv = reinterpret_cast<const u32x4*>(x);
    const int64_t step = (int64_t)gridDim.x * kThreads;
    // the bound is rounded up to whole waves so every lane of a block's DPP
    // group runs every iteration
    const int64_t span = (n_vec + 63) / 64 * 64;
    int64_t vi = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    // the first vector's HBM load goes out before the tables are staged (the
    // two latencies overlap); later ones one iteration ahead
    u32x4 cur = vi < n_vec ? ld_stream(xv + vi) : u32x4{0u, 0u, 0u, 0u};
    reinterpret_cast<uint32_t*>(rev_s)[threadIdx.x] = reinterpret_cast<const uint32_t*>(rev_g)[threadIdx.x];
    stage_tables(lut_s, band_w, lut_g, band_g);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);
    for (; vi < span; vi += step) {
        const bool live = vi < n_vec;
        const u32x4 nxt = vi + step < n_vec ? ld_stream(xv + vi + step) : u32x4{0u, 0u, 0u, 0u};
        float f[V];
        E::unpack(cur, f);
        cur = nxt;
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
            m = m > a ? m : a;
        }
        m = group_umax<G>(m);
        float d[V];
        const DitherVec dv = dither_vec(key, offset + (uint64_t)(vi * V));
#pragma unroll
        for (int e = 0; e < V; ++e) d[e] = STOCH ? dither_step(dv, e) : 0.0f;
        uint32_t cw[2], sw[2];                         // V bytes of codes and signs
        const int ex = quant_values<V, STOCH>(f, m, d, lut_s, band_s, rev_s, fq != nullptr, cw, sw);
        // the outputs are written once: streaming stores
        if (live) {
            if constexpr (V == 4) {
                st_stream(cw[0], reinterpret_cast<uint32_t*>(codes) + vi);
                if (signs) st_stream(sw[0], reinterpret_cast<uint32_t*>(signs) + vi);
            } else {
                st_stream(u32x2{cw[0], cw[1]}, reinterpret_cast<u32x2*>(codes) + vi);
                if (signs) st_stream(u32x2{sw[0], sw[1]}, reinterpret_cast<u32x2*>(signs) + vi);
            }
            if (vi % G == 0) st_stream((uint8_t)ex, exps + vi / G);
        }
        if (fq && live) st_stream(E::pack(f), reinterpret_cast<u32x4*>(fq) + vi);
    }
}

// quantize_kernel for short padded rows (cpad = nblk * BS positions):
// the codes, signs and exponents of such a tensor are one run of whole
// blocks, so each lane takes four consecutive positions of that run (a block
// is BS / 4 neighbouring lanes, DPP amax; one 4-byte code and sign store) and
// reads the values at positions inside the row one by one (zero past the
// row's end, as the reference pads).  The row of a position comes from one
// wave-uniform division per step and a 32-bit division inside it.  Same
// arithmetic and dither counters (offset + r * cols + c, padding positions
// included) as quantize_kernel.
template <int DT, int BS, bool STOCH>
__global__ __launch_bounds__(kThreads) void quantize_short_kernel(
    const typename Elem<DT>::S* __restrict__ x, int64_t rows, int64_t cols, int64_t nblk,
    const float* __restrict__ lut_g, const uint8_t* __restrict__ band_g, const uint8_t* __restrict__ rev_g,
    uint64_t seed, const uint64_t* __restrict__ seed_dev, uint64_t offset, uint8_t* __restrict__ exps,
    uint8_t* __restrict__ codes, uint8_t* __restrict__ signs, typename Elem<DT>::S* __restrict__ fq) {
    using E = Elem<DT>;
    constexpr int G = BS / 4;
    const uint64_t key = STOCH ? dither_key(seed + (seed_dev ? *seed_dev : 0ull)) : 0ull;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ uint8_t rev_s[kLutSize];
    reinterpret_cast<uint32_t*>(rev_s)[threadIdx.x] = reinterpret_cast<const uint32_t*>(rev_g)[threadIdx.x];
    stage_tables(lut_s, band_w, lut_g, band_g);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int lane = threadIdx.x & 63;
    const int cpad = (int)(nblk * BS);
    const int64_t n4 = rows * nblk * G;                // four-position groups
    const int64_t step = (int64_t)gridDim.x * kThreads;
    const int64_t span = (n4 + 63) / 64 * 64;          // whole waves: every DPP group runs
    for (int64_t vi = (int64_t)blockIdx.x * kThreads + threadIdx.x; vi < span; vi += step) {
        const uint64_t w0 = (uint64_t)(vi - lane);
        const int64_t p0 = 4 * (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(w0 >> 32)) << 32) |
                                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)w0));
        const int64_t r0 = p0 / cpad;                  // wave-uniform
        const uint32_t q = (uint32_t)(p0 - r0 * cpad) + 4u * (uint32_t)lane;
        const uint32_t lr = q / (uint32_t)cpad;
        const int64_t r = r0 + lr;
        const int c = (int)(q - lr * (uint32_t)cpad);
        const bool live = vi < n4;
        const int64_t base = r * cols;
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = live && c + e < cols ? E::to_f(x[base + c + e]) : 0.0f;
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
            m = m > a ? m : a;
        }
        m = group_umax<G>(m);
        float d[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = STOCH ? dither_step(key, offset + (uint64_t)(base + c + e)) : 0.0f;
        uint32_t cw[2], sw[2];
        const int ex = quant_values<4, STOCH>(f, m, d, lut_s, band_s, rev_s, fq != nullptr, cw, sw);
        if (live) {
            reinterpret_cast<uint32_t*>(codes)[vi] = cw[0];
            if (signs) reinterpret_cast<uint32_t*>(signs)[vi] = sw[0];
            if (c % BS == 0) exps[vi / G] = (uint8_t)ex;
            if (fq) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c + e < cols) fq[base + c + e] = E::from_f(f[e]);
            }
        }
    }
}

// Vector form of dequantize_kernel (cols % bs == 0, 4-byte aligned codes and
// signs, 16-byte aligned y): four values per lane, one 16-byte store.
__global__ __launch_bounds__(kThreads) void dequantize_vec_kernel(const uint8_t* __restrict__ exps,
                                                                  const uint8_t* __restrict__ codes,
                                                                  const uint8_t* __restrict__ signs,
                                                                  float* __restrict__ y, int64_t n4, int bs,
                                                                  const float* __restrict__ cb_g) {
    __shared__ float cb[kLevels];
    if (threadIdx.x < kLevels) cb[threadIdx.x] = cb_g[threadIdx.x];
    __syncthreads();
    const int sh = bs == 8 ? 1 : (bs == 16 ? 2 : 3);    // groups of 4 per block: 2^sh
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4; i += (int64_t)gridDim.x * kThreads) {
        const uint32_t cw = ld_stream(reinterpret_cast<const uint32_t*>(codes) + i);
        const uint32_t sw = signs ? ld_stream(reinterpret_cast<const uint32_t*>(signs) + i) : 0u;
        const float scale = pow2_float((int)exps[i >> sh] - kExpBias);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float a = cb[(cw >> (8 * e)) & 31] * scale;
            v[e] = ((sw >> (8 * e)) & 0xffu) ? -a : a;
        }
        u32x4 w;
        w.x = __float_as_uint(v[0]); w.y = __float_as_uint(v[1]);
        w.z = __float_as_uint(v[2]); w.w = __float_as_uint(v[3]);
        st_stream(w, reinterpret_cast<u32x4*>(y) + i);
    }
}

__global__ __launch_bounds__(kThreads) void dequantize_kernel(const uint8_t* __restrict__ exps,
                                                              const uint8_t* __restrict__ codes,
                                                              const uint8_t* __restrict__ signs,
                                                              float* __restrict__ y, int64_t rows,
                                                              int64_t cols, int64_t nblk, int bs,
                                                              const float* __restrict__ cb_g) {
    __shared__ float cb[kLevels];
    if (threadIdx.x < kLevels) cb[threadIdx.x] = cb_g[threadIdx.x];
    __syncthreads();
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kThreads) {
        const int64_t r = i / cols;
        const int64_t c = i - r * cols;
        const int64_t b = c / bs;
        const float scale = pow2_float((int)exps[r * nblk + b] - kExpBias);
        const int64_t o = r * nblk * bs + c;
        const float v = cb[codes[o] & 31] * scale;
        y[i] = (signs && signs[o]) ? -v : v;
    }
}

// Row-segment forms of quantize_kernel and dequantize_kernel, for rows of at
// least 64 values that do not tile into vectors of whole blocks: the lane
// and segment layout of fq_rows_kernel over the padded row (cpad = nblk * BS
// values: the codes and signs of the padding positions are written too, as
// quantize_kernel writes them), one value per lane.
template <int DT, int BS, bool STOCH, int U, int VL>
__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(
    const typename Elem<DT>::S* __restrict__ x, int64_t rows, int64_t cols, int64_t nblk, int64_t segs_per_row,
    int64_t segs_per_wave, const float* __restrict__ lut_g, const uint8_t* __restrict__ band_g,
    const uint8_t* __restrict__ rev_g, uint64_t seed, const uint64_t* __restrict__ seed_dev, uint64_t offset,
    uint8_t* __restrict__ exps, uint8_t* __restrict__ codes, uint8_t* __restrict__ signs,
    typename Elem<DT>::S* __restrict__ fq) {
    using E = Elem<DT>;
    constexpr int SEG = 64 * VL * U;
    static_assert(VL == 1 || VL == 4, "values per lane");
    static_assert(SEG % BS == 0 && BS % VL == 0, "segments hold whole blocks");
    const uint64_t key = STOCH ? dither_key(seed + (seed_dev ? *seed_dev : 0ull)) : 0ull;
    __shared__ float lut_s[kLutSize];
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ uint8_t rev_s[kLutSize];
    reinterpret_cast<uint32_t*>(rev_s)[threadIdx.x] = reinterpret_cast<const uint32_t*>(rev_g)[threadIdx.x];
    stage_tables(lut_s, band_w, lut_g, band_g);
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int lane = threadIdx.x & 63;
    const int64_t cpad = nblk * BS;
    const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t total = rows * segs_per_row;
    int64_t seg = wave * segs_per_wave;
    const int64_t end = seg + segs_per_wave < total ? seg + segs_per_wave : total;
    if (seg >= end) return;
    int64_t r = seg / segs_per_row;
    int64_t sx = seg - r * segs_per_row;
    // raw words of the next segment in flight while the current one is processed
    using Raw = typename std::conditional<VL == 1, typename E::S, u32x4>::type;
    auto load_seg = [&](int64_t rr, int64_t ss, Raw (&w)[U]) {
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t c = ss * SEG + VL * lane + 64 * VL * k;
            if constexpr (VL == 1) {
                w[k] = c < cols ? x[rr * cols + c] : (typename E::S)0;
            } else if constexpr (DT == AXS6_F32) {
                w[k] = c < cols ? *reinterpret_cast<const u32x4*>(x + rr * cols + c) : u32x4{0u, 0u, 0u, 0u};
            } else {
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 h = c < cols ? *reinterpret_cast<const u32x2*>(x + rr * cols + c) : u32x2{0u, 0u};
                w[k] = u32x4{h.x, h.y, 0u, 0u};
            }
        }
    };
    Raw nw[U];
    load_seg(r, sx, nw);
    for (; seg < end; ++seg) {
        const int64_t base = r * cols;
        float f[U][VL];
#pragma unroll
        for (int k = 0; k < U; ++k) {
            if constexpr (VL == 1) {
                f[k][0] = E::to_f(nw[k]);
            } else {
                float g[E::V];
                E::unpack(nw[k], g);
#pragma unroll
                for (int e = 0; e < VL; ++e) f[k][e] = g[e];
            }
        }
        int64_t rn = r, sn = sx + 1;
        if (sn == segs_per_row) {
            sn = 0;
            ++rn;
        }
        if (seg + 1 < end) load_seg(rn, sn, nw);
#pragma unroll
        for (int k = 0; k < U; ++k) {
            const int64_t c = sx * SEG + VL * lane + 64 * VL * k;
            uint32_t a = 0;
#pragma unroll
            for (int e = 0; e < VL; ++e) {
                const uint32_t b = __float_as_uint(f[k][e]) & 0x7fffffffu;
                a = a > b ? a : b;
            }
            uint32_t m;
            if constexpr (VL == 1) m = lanes_umax<BS>(a);
            else m = group_umax<BS / VL>(a);
            float d[VL];
#pragma unroll
            for (int e = 0; e < VL; ++e) d[e] = STOCH ? dither_step(key, offset + (uint64_t)(base + c + e)) : 0.0f;
            uint32_t cw[2], sw[2];
            const int ex = quant_values<VL, STOCH>(f[k], m, d, lut_s, band_s, rev_s, fq != nullptr, cw, sw);
            if (c < cpad) {
                const int64_t o = r * cpad + c;
                if constexpr (VL == 1) {
                    codes[o] = (uint8_t)cw[0];
                    if (signs) signs[o] = (uint8_t)sw[0];
                } else {
                    *reinterpret_cast<uint32_t*>(codes + o) = cw[0];
                    if (signs) *reinterpret_cast<uint32_t*>(signs + o) = sw[0];
                }
                if (c % BS == 0) exps[r * nblk + c / BS] = (uint8_t)ex;
            }
            if (fq && c < cols) {
                if constexpr (VL == 1) fq[base + c] = E::from_f(f[k][0]);
                else store4<DT>(fq + base + c, f[k]);
            }
        }
        r = rn;
        sx = sn;
    }
}

// Dequantize rows: the codes and signs of a row start at r * cpad, a
// multiple of 8 bytes, so a lane reads its four consecutive codes and signs
// as one 4-byte load each (four values per lane, 256 per wave segment) and
// writes the values it has inside the row (one 16-byte store when the row
// length is a multiple of four and y is 16-byte aligned).
__global__ __launch_bounds__(kThreads) void dequantize_rows_kernel(const uint8_t* __restrict__ exps,
                                                                   const uint8_t* __restrict__ codes,
                                                                   const uint8_t* __restrict__ signs,
                                                                   float* __restrict__ y, int64_t rows, int64_t cols,
                                                                   int64_t nblk, int bs, int64_t segs_per_row,
                                                                   int64_t segs_per_wave,
                                                                   const float* __restrict__ cb_g) {
    constexpr int SEG = 256;
    __shared__ float cb[kLevels];
    if (threadIdx.x < kLevels) cb[threadIdx.x] = cb_g[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int sh = bs == 8 ? 3 : (bs == 16 ? 4 : 5);
    const int64_t cpad = nblk * bs;
    // one 16-byte store per lane where the row's four values are whole and aligned
    const bool vec4 = cols % 4 == 0 && (uintptr_t)y % 16 == 0;
    const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t total = rows * segs_per_row;
    int64_t seg = wave * segs_per_wave;
    const int64_t end = seg + segs_per_wave < total ? seg + segs_per_wave : total;
    if (seg >= end) return;
    int64_t r = seg / segs_per_row;
    int64_t sx = seg - r * segs_per_row;
    for (; seg < end; ++seg) {
        const int64_t c = sx * SEG + 4 * lane;
        if (c < cols) {
            const uint32_t cw = *reinterpret_cast<const uint32_t*>(codes + r * cpad + c);
            const uint32_t sw = signs ? *reinterpret_cast<const uint32_t*>(signs + r * cpad + c) : 0u;
            const float scale = pow2_float((int)exps[r * nblk + (c >> sh)] - kExpBias);
            float* yr = y + r * cols + c;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a = cb[(cw >> (8 * e)) & 31] * scale;
                v[e] = ((sw >> (8 * e)) & 0xffu) ? -a : a;
            }
            if (vec4 && c + 4 <= cols) {
                *reinterpret_cast<float4*>(yr) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c + e < cols) yr[e] = v[e];
            }
        }
        if (++sx == segs_per_row) {
            sx = 0;
            ++r;
        }
    }
}

// dequantize_kernel for rows under 64 values: four positions per lane over
// the codes' run of whole blocks (the padded rows, rows * cpad positions,
// are contiguous), one 4-byte code and sign load each, writing the values at
// positions inside the row; the row of a position as in quantize_short_kernel.
__global__ __launch_bounds__(kThreads) void dequantize_short_kernel(const uint8_t* __restrict__ exps,
                                                                    const uint8_t* __restrict__ codes,
                                                                    const uint8_t* __restrict__ signs,
                                                                    float* __restrict__ y, int64_t rows, int64_t cols,
                                                                    int64_t nblk, int bs,
                                                                    const float* __restrict__ cb_g) {
    __shared__ float cb[kLevels];
    if (threadIdx.x < kLevels) cb[threadIdx.x] = cb_g[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int sh = bs == 8 ? 3 : (bs == 16 ? 4 : 5);
    const int cpad = (int)(nblk * bs);
    const int64_t n4 = rows * cpad / 4;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t vi = (int64_t)blockIdx.x * kThreads + threadIdx.x; vi - lane < n4; vi += step) {
        const uint64_t w0 = (uint64_t)(vi - lane);
        const int64_t p0 = 4 * (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(w0 >> 32)) << 32) |
                                         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)w0));
        const int64_t r0 = p0 / cpad;                  // wave-uniform
        const uint32_t q = (uint32_t)(p0 - r0 * cpad) + 4u * (uint32_t)lane;
        const uint32_t lr = q / (uint32_t)cpad;
        const int c = (int)(q - lr * (uint32_t)cpad);
        if (vi >= n4 || c >= cols) continue;
        const int64_t r = r0 + lr;
        const uint32_t cw = reinterpret_cast<const uint32_t*>(codes)[vi];
        const uint32_t sw = signs ? reinterpret_cast<const uint32_t*>(signs)[vi] : 0u;
        const float scale = pow2_float((int)exps[(4 * vi) >> sh] - kExpBias);
        float* yr = y + r * cols + c;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float a = cb[(cw >> (8 * e)) & 31] * scale;
            if (c + e < cols) yr[e] = ((sw >> (8 * e)) & 0xffu) ? -a : a;
        }
    }
}

// ---- launch helpers ---------------------------------------------------------

int num_cus() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Workgroups per CU the grid-stride kernels are capped at: 1024, i.e. in
// effect one workgroup per 256*kUnroll vectors -- at 8192x4096 f32 that grid
// (10923 workgroups at kUnroll 3) beat caps of 2..16 per CU (HBM-cold: 8 and
// 16 per CU measured 48.8 and 47.8 against 47.9 us uncapped at kUnroll 2).
constexpr int kWgPerCu = 1024;

int64_t capped_grid(int64_t work_items, int64_t per_wg) {
    int64_t need = (work_items + per_wg - 1) / per_wg;
    int64_t cap = (int64_t)num_cus() * kWgPerCu;
    if (need < 1) need = 1;
    return need < cap ? need : cap;
}

// Row-segment launches (fq_rows_kernel and its quantize counterpart) for rows
// of at least kRowsMinCols elements; shorter rows take the short-row kernels
// (whole rows per wave step).  Segments of 64 * u elements, a contiguous range of per_wave of
// them per wave, sized for about kRowsWavesPerCu waves per CU and at least
// kRowsMinSegs segments per wave (the tables are staged once per workgroup).
constexpr int64_t kRowsMinCols = 64;
constexpr int64_t kRowsWavesPerCu = 64;
constexpr int64_t kRowsMinSegs = 2;
// Quantize rows padded to fewer positions than this take quantize_short_kernel
// (measured: 131072 x 100 at block 32, 128 positions, 27.0 -> 20.7 us; at 224
// positions the row-segment kernel's 17.3 us beat 19.2 us).
constexpr int64_t kQuantShortMax = 192;

struct RowSegs {
    int u;
    int64_t per_row, per_wave;
    dim3 grid;
};

RowSegs row_segs(int64_t rows, int64_t cols, int u) {
    RowSegs g;
    g.u = u;
    g.per_row = (cols + 64 * u - 1) / (64 * u);
    const int64_t total = rows * g.per_row;
    const int64_t waves = (int64_t)num_cus() * kRowsWavesPerCu;
    int64_t per = (total + waves - 1) / waves;
    g.per_wave = per < kRowsMinSegs ? kRowsMinSegs : per;
    const int64_t need = (total + g.per_wave - 1) / g.per_wave;            // waves
    g.grid = dim3((unsigned)((need + kThreads / 64 - 1) / (kThreads / 64)));
    return g;
}

template <int DT, int BS>
void launch_fq_typed(const void* x, void* y, int64_t rows, int64_t cols, bool stochastic, uint64_t seed, const uint64_t* seed_dev,
                     uint64_t offset, const DeviceTables& t, hipStream_t st) {
    using S = typename Elem<DT>::S;
    constexpr int V = Elem<DT>::V;
    const bool aligned = (cols % BS == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0);
    if (aligned) {
        const int64_t n_vec = rows * cols / V;
        const dim3 grid((unsigned)capped_grid(n_vec, (int64_t)kThreads * kUnroll));
        if (stochastic)
            fq_vec_kernel<DT, BS, true><<<grid, kThreads, 0, st>>>((const S*)x, (S*)y, n_vec, t.lut, t.band, seed, seed_dev, offset);
        else
            fq_vec_kernel<DT, BS, false><<<grid, kThreads, 0, st>>>((const S*)x, (S*)y, n_vec, t.lut, t.band, seed, seed_dev, offset);
        return;
    }
    const int esize = (int)sizeof(S);
    const bool four = cols % 4 == 0 && (uintptr_t)x % (4 * esize) == 0 && (uintptr_t)y % (4 * esize) == 0;
    if (cols >= 4 * kRowsMinCols || (cols >= kRowsMinCols && !four)) {
#define AXS6_FQROWS(U_, VL_)                                                                                   \
        do {                                                                                                   \
            const RowSegs g = row_segs(rows, cols, (U_) * (VL_));                                              \
            if (stochastic)                                                                                    \
                fq_rows_kernel<DT, BS, true, U_, VL_><<<g.grid, kThreads, 0, st>>>(                            \
                    (const S*)x, (S*)y, rows, cols, g.per_row, g.per_wave, t.lut, t.band, seed, seed_dev, offset); \
            else                                                                                               \
                fq_rows_kernel<DT, BS, false, U_, VL_><<<g.grid, kThreads, 0, st>>>(                           \
                    (const S*)x, (S*)y, rows, cols, g.per_row, g.per_wave, t.lut, t.band, seed, seed_dev, offset); \
        } while (0)
        if (four) AXS6_FQROWS(1, 4);
        else if (cols >= 4 * kRowsMinCols) AXS6_FQROWS(4, 1);
        else AXS6_FQROWS(1, 1);
#undef AXS6_FQROWS
    } else {
        // short rows: 1..63 values one per lane, or whole 4-value groups under
        // 256 values (aligned) four per lane; R = 64 * VL / cols rows per wave
        // step, at least kRowsMinSegs steps per wave, about kRowsWavesPerCu
        // waves per CU
        const int vl = four ? 4 : 1;
        const int64_t per = 64 * vl / cols;
        const int64_t steps = (rows + per - 1) / per;
        int64_t waves = (steps + kRowsMinSegs - 1) / kRowsMinSegs;
        const int64_t cap = (int64_t)num_cus() * kRowsWavesPerCu;
        waves = waves < cap ? waves : cap;
        const dim3 grid((unsigned)((waves + kThreads / 64 - 1) / (kThreads / 64)));
#define AXS6_FQSHORT(VL_)                                                                                      \
        do {                                                                                                   \
            if (stochastic)                                                                                    \
                fq_short_kernel<DT, BS, true, VL_><<<grid, kThreads, 0, st>>>((const S*)x, (S*)y, rows, (int)cols, \
                                                                              t.lut, t.band, seed, seed_dev, offset); \
            else                                                                                               \
                fq_short_kernel<DT, BS, false, VL_><<<grid, kThreads, 0, st>>>((const S*)x, (S*)y, rows, (int)cols, \
                                                                               t.lut, t.band, seed, seed_dev, offset); \
        } while (0)
        if (vl == 4) AXS6_FQSHORT(4);
        else AXS6_FQSHORT(1);
#undef AXS6_FQSHORT
    }
}

template <int DT>
void launch_fq(const void* x, void* y, int64_t rows, int64_t cols, int bs, bool stochastic, uint64_t seed, const uint64_t* seed_dev,
               uint64_t offset, const DeviceTables& t, hipStream_t st) {
    if (bs == 8) launch_fq_typed<DT, 8>(x, y, rows, cols, stochastic, seed, seed_dev, offset, t, st);
    else if (bs == 16) launch_fq_typed<DT, 16>(x, y, rows, cols, stochastic, seed, seed_dev, offset, t, st);
    else launch_fq_typed<DT, 32>(x, y, rows, cols, stochastic, seed, seed_dev, offset, t, st);
}

template <int DT, int BS>
void launch_quant_typed(const void* x, int64_t rows, int64_t cols, bool stochastic, uint64_t seed, const uint64_t* seed_dev,
                        uint64_t offset, uint8_t* exps, uint8_t* codes, uint8_t* signs, void* fq,
                        const DeviceTables& t, hipStream_t st) {
    using S = typename Elem<DT>::S;
    constexpr int V = Elem<DT>::V;
    if (cols % BS == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)codes % V == 0 && (uintptr_t)signs % V == 0 &&
        (uintptr_t)fq % 16 == 0) {
        const int64_t n_vec = rows * cols / V;
        const dim3 grid((unsigned)capped_grid(n_vec, (int64_t)kThreads * 2));   // two iterations per workgroup
        if (stochastic)
            quantize_vec_kernel<DT, BS, true><<<grid, kThreads, 0, st>>>((const S*)x, n_vec, t.lut, t.band, t.rev, seed, seed_dev, offset, exps, codes, signs, (S*)fq);
        else
            quantize_vec_kernel<DT, BS, false><<<grid, kThreads, 0, st>>>((const S*)x, n_vec, t.lut, t.band, t.rev, seed, seed_dev, offset, exps, codes, signs, (S*)fq);
        return;
    }
    const int64_t nblk = (cols + BS - 1) / BS;
    const int64_t cpad = nblk * BS;
    const bool c4 = (uintptr_t)codes % 4 == 0 && (uintptr_t)signs % 4 == 0;
    const bool x4 = cols % 4 == 0 && (uintptr_t)x % (4 * sizeof(S)) == 0;
    // Four positions per lane over the run of blocks (quantize_short_kernel)
    // for padded rows under kQuantShortMax positions, and for longer rows
    // that the row-segment kernel would read one value per lane when there
    // is no FQ output (4-byte code and sign stores against byte stores:
    // 8192 x 4095 f32 53-56 -> 41-44 us, 32768 x 999 53-56 -> 40-41 us; with
    // an FQ output its per-lane value stores lose: 82-85 -> 117-120 us).
    // Otherwise long rows fill most of the row-segment kernel's 256-position
    // segments, whose vector loads then win.
    // (its in-wave row arithmetic is 32-bit: rows of fewer than 2^30 positions)
    const bool short_form = c4 && (cpad < kQuantShortMax || (fq == nullptr && !x4 && cpad < ((int64_t)1 << 30)));
    if (!short_form && cpad >= kRowsMinCols) {
        const int esize = (int)sizeof(S);
        const bool four = cols % 4 == 0 && (uintptr_t)x % (4 * esize) == 0 && (uintptr_t)fq % (4 * esize) == 0 &&
                          (uintptr_t)codes % 4 == 0 && (uintptr_t)signs % 4 == 0;
#define AXS6_QROWS(U_, VL_)                                                                                  \
        do {                                                                                                 \
            const RowSegs g = row_segs(rows, cpad, (U_) * (VL_));                                            \
            if (stochastic)                                                                                  \
                quantize_rows_kernel<DT, BS, true, U_, VL_><<<g.grid, kThreads, 0, st>>>(                    \
                    (const S*)x, rows, cols, nblk, g.per_row, g.per_wave, t.lut, t.band, t.rev, seed, seed_dev, \
                    offset, exps, codes, signs, (S*)fq);                                                     \
            else                                                                                             \
                quantize_rows_kernel<DT, BS, false, U_, VL_><<<g.grid, kThreads, 0, st>>>(                   \
                    (const S*)x, rows, cols, nblk, g.per_row, g.per_wave, t.lut, t.band, t.rev, seed, seed_dev, \
                    offset, exps, codes, signs, (S*)fq);                                                     \
        } while (0)
        if (four) AXS6_QROWS(1, 4);
        else if (cpad >= 4 * kRowsMinCols) AXS6_QROWS(4, 1);
        else AXS6_QROWS(1, 1);
#undef AXS6_QROWS
        return;
    }
    if (short_form) {
        const dim3 grid((unsigned)capped_grid(rows * cpad / 4, (int64_t)kThreads * 2));
        if (stochastic)
            quantize_short_kernel<DT, BS, true><<<grid, kThreads, 0, st>>>((const S*)x, rows, cols, nblk, t.lut, t.band, t.rev, seed, seed_dev, offset, exps, codes, signs, (S*)fq);
        else
            quantize_short_kernel<DT, BS, false><<<grid, kThreads, 0, st>>>((const S*)x, rows, cols, nblk, t.lut, t.band, t.rev, seed, seed_dev, offset, exps, codes, signs, (S*)fq);
        return;
    }
    const dim3 grid((unsigned)capped_grid(rows * nblk, (int64_t)kThreads / BS));
    if (stochastic)
        quantize_kernel<DT, BS, true><<<grid, kThreads, 0, st>>>((const S*)x, rows, cols, nblk, t.lut, t.band, t.rev, seed, seed_dev, offset, exps, codes, signs, (S*)fq);
    else
        quantize_kernel<DT, BS, false><<<grid, kThreads, 0, st>>>((const S*)x, rows, cols, nblk, t.lut, t.band, t.rev, seed, seed_dev, offset, exps, codes, signs, (S*)fq);
}

template <int DT>
void launch_quant(const void* x, int64_t rows, int64_t cols, int bs, bool stochastic, uint64_t seed, const uint64_t* seed_dev,
                  uint64_t offset, uint8_t* exps, uint8_t* codes, uint8_t* signs, void* fq,
                  const DeviceTables& t, hipStream_t st) {
    if (bs == 8) launch_quant_typed<DT, 8>(x, rows, cols, stochastic, seed, seed_dev, offset, exps, codes, signs, fq, t, st);
    else if (bs == 16) launch_quant_typed<DT, 16>(x, rows, cols, stochastic, seed, seed_dev, offset, exps, codes, signs, fq, t, st);
    else launch_quant_typed<DT, 32>(x, rows, cols, stochastic, seed, seed_dev, offset, exps, codes, signs, fq, t, st);
}

int check_shape(const char* fn, int64_t rows, int64_t cols, int bs) {
    if (!valid_block(bs)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: block_size must be 8, 16 or 32 (got %d)", fn, bs);
    if (rows < 0 || cols < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative shape (%lld, %lld)", fn, (long long)rows, (long long)cols);
    if (cols > 0 && rows > ((int64_t)1 << 50) / (cols + 32))
        return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: tensor too large (%lld x %lld)", fn, (long long)rows, (long long)cols);
    return AXS6_OK;
}

}  // namespace
}  // namespace axs6

using namespace axs6;

extern "C" int axs6_nf5_fake_quantize(const void* x, void* y, int32_t dtype, int64_t rows, int64_t cols,
                                      int32_t block_size, int32_t stochastic, uint64_t seed,
                                      uint64_t offset, const uint64_t* seed_dev, void* stream) {
    const char* fn = "axs6_nf5_fake_quantize";
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    int rc = check_shape(fn, rows, cols, block_size);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return AXS6_OK;
    if (!x || !y) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null tensor pointer", fn);
    DeviceTables t;
    if ((rc = device_tables(&t))) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == AXS6_F32) launch_fq<AXS6_F32>(x, y, rows, cols, block_size, stochastic != 0, seed, seed_dev, offset, t, st);
    else if (dtype == AXS6_BF16) launch_fq<AXS6_BF16>(x, y, rows, cols, block_size, stochastic != 0, seed, seed_dev, offset, t, st);
    else launch_fq<AXS6_F16>(x, y, rows, cols, block_size, stochastic != 0, seed, seed_dev, offset, t, st);
    return check_launch(fn);
}

extern "C" int axs6_nf5_quantize(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                                 int32_t stochastic, uint64_t seed, uint64_t offset, uint8_t* exponents,
                                 uint8_t* codes, uint8_t* signs, void* fq, const uint64_t* seed_dev, void* stream) {
    const char* fn = "axs6_nf5_quantize";
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    int rc = check_shape(fn, rows, cols, block_size);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return AXS6_OK;
    if (!x || !exponents || !codes) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null tensor pointer", fn);
    DeviceTables t;
    if ((rc = device_tables(&t))) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == AXS6_F32) launch_quant<AXS6_F32>(x, rows, cols, block_size, stochastic != 0, seed, seed_dev, offset, exponents, codes, signs, fq, t, st);
    else if (dtype == AXS6_BF16) launch_quant<AXS6_BF16>(x, rows, cols, block_size, stochastic != 0, seed, seed_dev, offset, exponents, codes, signs, fq, t, st);
    else launch_quant<AXS6_F16>(x, rows, cols, block_size, stochastic != 0, seed, seed_dev, offset, exponents, codes, signs, fq, t, st);
    return check_launch(fn);
}

extern "C" int axs6_nf5_dequantize(const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs, float* y,
                                   int64_t rows, int64_t cols, int32_t block_size, void* stream) {
    const char* fn = "axs6_nf5_dequantize";
    int rc = check_shape(fn, rows, cols, block_size);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return AXS6_OK;
    if (!exponents || !codes || !y) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null tensor pointer", fn);
    DeviceTables t;
    if ((rc = device_tables(&t))) return rc;
    const int64_t nblk = (cols + block_size - 1) / block_size;
    if (cols % block_size == 0 && (uintptr_t)codes % 4 == 0 && (uintptr_t)signs % 4 == 0 && (uintptr_t)y % 16 == 0) {
        const int64_t n4 = rows * cols / 4;
        dequantize_vec_kernel<<<dim3((unsigned)capped_grid(n4, kThreads)), kThreads, 0, (hipStream_t)stream>>>(
            exponents, codes, signs, y, n4, block_size, t.codebook);
        return check_launch(fn);
    }
    if (cols >= kRowsMinCols && (uintptr_t)codes % 4 == 0 && (uintptr_t)signs % 4 == 0) {
        const RowSegs g = row_segs(rows, cols, 4);
        dequantize_rows_kernel<<<g.grid, kThreads, 0, (hipStream_t)stream>>>(
            exponents, codes, signs, y, rows, cols, nblk, block_size, g.per_row, g.per_wave, t.codebook);
        return check_launch(fn);
    }
    if ((uintptr_t)codes % 4 == 0 && (uintptr_t)signs % 4 == 0 && 4 * cols >= nblk * block_size) {
        // rows under 64 values filling at least a quarter of their padded
        // blocks: four positions per lane over the padded run (sparser rows,
        // e.g. 3 values in a block of 32, keep one thread per value: 2^20 x 3
        // 16.3 us against 27.7 in this form)
        const dim3 grid((unsigned)capped_grid(rows * nblk * block_size / 4, kThreads));
        dequantize_short_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(exponents, codes, signs, y, rows, cols,
                                                                            nblk, block_size, t.codebook);
        return check_launch(fn);
    }
    const dim3 grid((unsigned)capped_grid(rows * cols, kThreads));
    dequantize_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(exponents, codes, signs, y, rows, cols, nblk,
                                                                  block_size, t.codebook);
    return check_launch(fn);
}
