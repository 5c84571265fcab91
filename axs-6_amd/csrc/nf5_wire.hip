// NF5 wire format (gfx950): the reference's 6.25-bit gradient encoding,
// produced and consumed on the device in one pass each way.
//
// Record of one block of `bs` values (bs in {8, 16, 32}), blocks in row-major
// order, a row's last block zero-padded virtually:
//   byte 0                 shared exponent e (uint8, quantize_unified's rule)
//   bytes 1 .. 3*bs/4      6-bit codes q = (sign << 5) | code, four per three
//                          bytes:  b0 = q0 | q1<<6,  b1 = q1>>2 | q2<<4,
//                                  b2 = q2>>4 | q3<<2   (low bits first)
// so a 32-value block takes 25 bytes.  Layout of _pack_to_flat_buffer
// (axs/unified/distributed.py:147-198); the codes are those of
// _pack_gradient (:70-115), i.e. quantize_unified with nearest rounding.
//
// The AXSBlock byte form (AXSBlock.to_bytes / from_bytes, axs/core.py:97-152)
// differs only in its header: two bytes, the little-endian word
// e << 2 | config (config DENSE = 0 when written, ignored when decoded, as
// the reference's decoder ignores it), then the same 6-bit little-endian
// stream, so a 32-value block takes 26 bytes.  Every kernel below takes the
// header size HB (1 wire, 2 AXSBlock) as a template parameter.
//
// One thread handles one group of four values (three bytes); a block is
// bs/4 neighbouring lanes, whose amax is a DPP reduction.
//
// Fast path (cols % bs == 0, so the blocks tile the flattened tensor, and
// aligned pointers): a lane loads its group as one 16-byte (f32) or 8-byte
// vector; a workgroup assembles the records of kWireTiles tiles of 256
// groups in LDS -- 800, 832 or 896 bytes per tile for bs 32, 16, 8, each a
// multiple of 16 -- and writes them as whole 16-byte vectors.  Unpacking
// reverses it: 16-byte record loads into LDS, one 16-byte f32 store per
// group.  Ragged rows (the virtual zero padding) and values off 4-value
// alignment keep these record tiles -- the record stream is the same run of
// whole blocks -- and read or write the values by row geometry (RowGeom);
// only a buffer off 16-byte alignment takes the general kernels, one group
// per thread with byte accesses.
#include "nf5_device.h"

namespace axs6 {
namespace {

__device__ __forceinline__ void pack3(const int (&q)[4], uint8_t* out) {
    out[0] = (uint8_t)((q[0] & 0x3F) | ((q[1] & 0x03) << 6));
    out[1] = (uint8_t)(((q[1] >> 2) & 0x0F) | ((q[2] & 0x0F) << 4));
    out[2] = (uint8_t)(((q[2] >> 4) & 0x03) | ((q[3] & 0x3F) << 2));
}

__device__ __forceinline__ void unpack3(const uint8_t* in, int (&q)[4]) {
    const int b0 = in[0], b1 = in[1], b2 = in[2];
    q[0] = b0 & 0x3F;
    q[1] = ((b0 >> 6) & 0x03) | ((b1 & 0x0F) << 2);
    q[2] = ((b1 >> 4) & 0x0F) | ((b2 & 0x03) << 4);
    q[3] = (b2 >> 2) & 0x3F;
}

// Record header of HB bytes.  HB = 1 (wire): the exponent byte.  HB = 2
// (AXSBlock): the little-endian 16-bit word e << 2 | config, written with
// config DENSE (0); bits 10..15 are padding, read as zero.
template <int HB>
__device__ __forceinline__ void put_header(uint8_t* rec, int e8) {
    if constexpr (HB == 1) {
        rec[0] = (uint8_t)e8;
    } else {
        rec[0] = (uint8_t)(e8 << 2);
        rec[1] = (uint8_t)(e8 >> 6);
    }
}

template <int HB>
__device__ __forceinline__ int get_exponent(const uint8_t* rec) {
    if constexpr (HB == 1) return rec[0];
    else return (rec[0] >> 2) | ((rec[1] & 0x03) << 6);
}

struct WireGeom {
    int64_t rows, cols, nblk, groups;   // groups = rows * nblk * bs / 4
};

// Record fields of one group of four values of a block whose largest |x|
// has the float bits m (reduced over the block's lanes).  Exponent:
// e = clamp(floor(log2(max(amax, 1e-45))) + 1 + 127, 0, 255), 0 for an
// all-zero block (and for NaN/inf amax, whose int cast is INT_MIN);
// index = trunc(clamp(|x| / 2^(e-127), 0, 1) * 1023); code = reverse_lut[index];
// q = code | (x < 0) << 5.  Returns e.
__device__ __forceinline__ int wire_codes(const float (&f)[4], uint32_t m, const uint8_t* band_s,
                                          const uint8_t* rev_s, int (&qv)[4]) {
    int e8 = (m == 0u || m >= kInfBits) ? 0 : floor_log2_torch(m, band_s) + 1 + kExpBias;
    e8 = e8 < 0 ? 0 : (e8 > 255 ? 255 : e8);
    const int se = e8 - kExpBias;           // scale 2^se, se in [-127, 128]
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t ab = __float_as_uint(f[e]) & 0x7fffffffu;
        float n;
        if (se >= 128) n = ab >= kInfBits ? __uint_as_float(kNanBits) : 0.0f;
        else n = __builtin_amdgcn_ldexpf(__uint_as_float(ab), -se);
        n = n > 1.0f ? 1.0f : n;            // clamp(0, 1); NaN passes to the index rule
        const int idx = lut_index(n, false, 0.0f);
        qv[e] = (int)rev_s[idx] | ((f[e] < 0.0f ? 1 : 0) << 5);
    }
    return e8;
}

// x [rows, cols] -> records (general path), one group per thread.
template <int HB, int DT, int BS>
__global__ __launch_bounds__(kThreads) void wire_pack_kernel(const typename Elem<DT>::S* __restrict__ x, WireGeom g,
                                                             const uint8_t* __restrict__ band_g,
                                                             const uint8_t* __restrict__ rev_g,
                                                             uint8_t* __restrict__ buf) {
    using E = Elem<DT>;
    constexpr int GPB = BS / 4;                 // groups (lanes) per block
    constexpr int REC = HB + BS * 3 / 4;        // bytes per block record
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ uint8_t rev_s[kLutSize];
    const int tid = threadIdx.x;
    reinterpret_cast<uint32_t*>(rev_s)[tid] = reinterpret_cast<const uint32_t*>(rev_g)[tid];
    if (tid < kBandSize / 4) band_w[tid] = reinterpret_cast<const uint32_t*>(band_g)[tid];
    __syncthreads();
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);

    const int64_t step = (int64_t)gridDim.x * kThreads;
    // the loop bound is rounded up to whole waves so every lane of a block's
    // DPP group runs every iteration
    const int64_t span = (g.groups + 63) / 64 * 64;
    for (int64_t q = (int64_t)blockIdx.x * kThreads + tid; q < span; q += step) {
        const bool vq = q < g.groups;
        const int64_t blk = vq ? q / GPB : 0;
        const int j4 = (int)(q % GPB);
        const int64_t r = blk / g.nblk;
        const int64_t c0 = (blk - r * g.nblk) * BS + j4 * 4;
        float f[4];
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t c = c0 + e;
            f[e] = (vq && c < g.cols) ? E::to_f(x[r * g.cols + c]) : 0.0f;
            const uint32_t a = __float_as_uint(f[e]) & 0x7fffffffu;
            m = m > a ? m : a;
        }
        m = group_umax<GPB>(m);
        int qv[4];
        const int e8 = wire_codes(f, m, band_s, rev_s, qv);
        if (vq) {
            uint8_t* rec = buf + blk * REC;
            if (j4 == 0) put_header<HB>(rec, e8);
            pack3(qv, rec + HB + 3 * j4);
        }
    }
}

// Fast-path geometry: kWireTiles tiles of kThreads groups per workgroup
// iteration; a tile's records take wire_tile_bytes<HB, BS>() bytes
// (800, 832, 896 for wire blocks of 32, 16, 8; 832, 896, 1024 for AXSBlocks).
constexpr int kWireTiles = 4;
template <int HB, int BS>
constexpr int wire_tile_bytes() { return kThreads / (BS / 4) * (HB + BS * 3 / 4); }

// The four values of group q (flat index 4q), as floats.
template <int DT>
__device__ __forceinline__ void load_group(const typename Elem<DT>::S* x, int64_t q, float (&f)[4]) {
    using E = Elem<DT>;
    if constexpr (DT == AXS6_F32) {
        const u32x4 v = ld_stream(reinterpret_cast<const u32x4*>(x + q * 4));
        f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
        f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
    } else {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 v = ld_stream(reinterpret_cast<const u32x2*>(x + q * 4));
        using S = typename E::S;
        f[0] = E::to_f(__builtin_bit_cast(S, (uint16_t)(v.x & 0xffffu)));
        f[1] = E::to_f(__builtin_bit_cast(S, (uint16_t)(v.x >> 16)));
        f[2] = E::to_f(__builtin_bit_cast(S, (uint16_t)(v.y & 0xffffu)));
        f[3] = E::to_f(__builtin_bit_cast(S, (uint16_t)(v.y >> 16)));
    }
}

// Rows that do not tile into whole blocks (a ragged last block) or whose
// values are not aligned to 4-value groups: the record stream is the same
// run of whole blocks over the zero-padded rows (gpr = groups per padded
// row), so the fast kernels keep their record tiles and only the values'
// side changes.  Group q holds values 4 * (q % gpr) .. + 3 of row q / gpr;
// the row of a tile's first group comes from one wave-uniform division and
// each lane steps forward over whole rows from it.
struct RowGeom {
    int64_t cols, gpr;
    bool vec4;      // cols % 4 == 0 and the tensor aligned to 4 values: one load/store per group
};

__device__ __forceinline__ void group_pos(int64_t q, int64_t qt, const RowGeom& rg, int64_t& r, int64_t& c) {
    const uint64_t u = (uint64_t)qt;
    const int64_t qs = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(u >> 32)) << 32) |
                                 (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u));
    r = qs / rg.gpr;
    int64_t qq = q - r * rg.gpr;
    while (qq >= rg.gpr) {
        qq -= rg.gpr;
        ++r;
    }
    c = 4 * qq;
}

template <int DT>
__device__ __forceinline__ void load_group_rows(const typename Elem<DT>::S* x, int64_t q, int64_t qt,
                                                const RowGeom& rg, float (&f)[4]) {
    using E = Elem<DT>;
    int64_t r, c;
    group_pos(q, qt, rg, r, c);
    const typename E::S* p = x + r * rg.cols + c;
    if (rg.vec4 && c + 4 <= rg.cols) {
        load_group<DT>(p, 0, f);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = c + e < rg.cols ? E::to_f(p[e]) : 0.0f;
    }
}

// Fast-path pack: groups = rows * cols / 4 with cols % BS == 0; x aligned to
// its 4-value group, buf to 16 bytes.  Same record bytes as wire_pack_kernel.
// ROWS: any rows, values read through RowGeom (buf still 16-byte aligned).
template <int HB, int DT, int BS, bool ROWS>
__global__ __launch_bounds__(kThreads) void wire_pack_vec_kernel(const typename Elem<DT>::S* __restrict__ x,
                                                                 int64_t groups, RowGeom rg,
                                                                 const uint8_t* __restrict__ band_g,
                                                                 const uint8_t* __restrict__ rev_g,
                                                                 uint8_t* __restrict__ buf) {
    constexpr int GPB = BS / 4;
    constexpr int REC = HB + BS * 3 / 4;
    constexpr int TB = wire_tile_bytes<HB, BS>();
    constexpr int U = kWireTiles;
    static_assert(TB % 16 == 0 && kThreads % GPB == 0, "tiles of whole blocks and 16-byte chunks");
    __shared__ uint32_t band_w[kBandSize / 4];
    __shared__ uint8_t rev_s[kLutSize];
    __shared__ __align__(16) uint8_t recs[U * TB];
    const int tid = threadIdx.x;
    reinterpret_cast<uint32_t*>(rev_s)[tid] = reinterpret_cast<const uint32_t*>(rev_g)[tid];
    if (tid < kBandSize / 4) band_w[tid] = reinterpret_cast<const uint32_t*>(band_g)[tid];
    __syncthreads();
    const uint8_t* band_s = reinterpret_cast<const uint8_t*>(band_w);
    const int64_t ntiles = (groups + kThreads - 1) / kThreads;
    const int64_t total_bytes = groups / GPB * REC;
    uint8_t* rec = recs + (tid / GPB) * REC;   // this lane's block record within a tile
    const int j4 = tid % GPB;

    for (int64_t t0 = (int64_t)blockIdx.x * U; t0 < ntiles; t0 += (int64_t)gridDim.x * U) {
        float f[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t qt = (t0 + u) * kThreads;
            const int64_t q = qt + tid;
            if (q < groups) {
                if constexpr (ROWS) load_group_rows<DT>(x, q, qt, rg, f[u]);
                else load_group<DT>(x, q, f[u]);
            } else {
                f[u][0] = f[u][1] = f[u][2] = f[u][3] = 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint32_t m = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t a = __float_as_uint(f[u][e]) & 0x7fffffffu;
                m = m > a ? m : a;
            }
            // a block is GPB lanes at a multiple of GPB: all inside or all past the end
            m = group_umax<GPB>(m);
            int qv[4];
            const int e8 = wire_codes(f[u], m, band_s, rev_s, qv);
            if (j4 == 0) put_header<HB>(rec + u * TB, e8);
            pack3(qv, rec + u * TB + HB + 3 * j4);
        }
        __syncthreads();
        // the U tiles' records are contiguous in buf from t0 * TB
        const int64_t base = t0 * TB;
        const int64_t left = total_bytes - base;
        const int nbytes = left < U * TB ? (int)left : U * TB;
        for (int c = tid; c * 16 < nbytes; c += kThreads) {
            if (c * 16 + 16 <= nbytes) {
                st_stream(*reinterpret_cast<const u32x4*>(recs + c * 16), reinterpret_cast<u32x4*>(buf + base + c * 16));
            } else {
                for (int b = c * 16; b < nbytes; ++b) buf[base + b] = recs[b];
            }
        }
        __syncthreads();   // recs is rewritten by the next iteration
    }
}

// Fast-path unpack, the inverse geometry: y [groups * 4] f32 (16-byte aligned), buf 16-byte aligned.
template <int HB, int BS, bool ROWS>
__global__ __launch_bounds__(kThreads) void wire_unpack_vec_kernel(const uint8_t* __restrict__ buf, int64_t groups,
                                                                   RowGeom rg, const float* __restrict__ cb_g,
                                                                   float* __restrict__ y) {
    constexpr int GPB = BS / 4;
    constexpr int REC = HB + BS * 3 / 4;
    constexpr int TB = wire_tile_bytes<HB, BS>();
    constexpr int U = kWireTiles;
    static_assert(TB % 16 == 0 && kThreads % GPB == 0, "tiles of whole blocks and 16-byte chunks");
    __shared__ float cb[kLevels];
    __shared__ __align__(16) uint8_t recs[U * TB];
    const int tid = threadIdx.x;
    if (tid < kLevels) cb[tid] = cb_g[tid];
    const int64_t ntiles = (groups + kThreads - 1) / kThreads;
    const int64_t total_bytes = groups / GPB * REC;
    const uint8_t* rec = recs + (tid / GPB) * REC;
    const int j4 = tid % GPB;

    for (int64_t t0 = (int64_t)blockIdx.x * U; t0 < ntiles; t0 += (int64_t)gridDim.x * U) {
        const int64_t base = t0 * TB;
        const int64_t left = total_bytes - base;
        const int nbytes = left < U * TB ? (int)left : U * TB;
        for (int c = tid; c * 16 < nbytes; c += kThreads) {
            if (c * 16 + 16 <= nbytes) {
                *reinterpret_cast<u32x4*>(recs + c * 16) = ld_stream(reinterpret_cast<const u32x4*>(buf + base + c * 16));
            } else {
                for (int b = c * 16; b < nbytes; ++b) recs[b] = buf[base + b];
            }
        }
        __syncthreads();   // records (and, the first time, the codebook) staged
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t qt = (t0 + u) * kThreads;
            const int64_t q = qt + tid;
            if (q < groups) {
                const uint8_t* r = rec + u * TB;
                const float scale = pow2_float(get_exponent<HB>(r) - kExpBias);
                int qv[4];
                unpack3(r + HB + 3 * j4, qv);
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float a = cb[qv[e] & 0x1F] * scale;
                    v[e] = (qv[e] & 0x20) ? -a : a;
                }
                u32x4 w;
                w.x = __float_as_uint(v[0]); w.y = __float_as_uint(v[1]);
                w.z = __float_as_uint(v[2]); w.w = __float_as_uint(v[3]);
                if constexpr (ROWS) {
                    int64_t row, c;
                    group_pos(q, qt, rg, row, c);
                    float* p = y + row * rg.cols + c;
                    if (rg.vec4 && c + 4 <= rg.cols) {
                        *reinterpret_cast<u32x4*>(p) = w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (c + e < rg.cols) p[e] = v[e];
                    }
                } else {
                    st_stream(w, reinterpret_cast<u32x4*>(y + q * 4));
                }
            }
        }
        __syncthreads();   // recs is rewritten by the next iteration
    }
}

unsigned wire_vec_grid(int64_t groups) {
    const int64_t ntiles = (groups + kThreads - 1) / kThreads;
    const int64_t wgs = (ntiles + kWireTiles - 1) / kWireTiles;
    return (unsigned)(wgs < 32768 ? (wgs > 0 ? wgs : 1) : 32768);
}

// records -> y [rows, cols] f32: codebook[code] * 2^(e-127), negated where the
// sign bit is set (_unpack_from_flat_buffer + _unpack_gradient, :118-144,201-232).
// General path, one group per thread.
template <int HB, int BS>
__global__ __launch_bounds__(kThreads) void wire_unpack_kernel(const uint8_t* __restrict__ buf, WireGeom g,
                                                               const float* __restrict__ cb_g, float* __restrict__ y) {
    constexpr int GPB = BS / 4;
    constexpr int REC = HB + BS * 3 / 4;
    __shared__ float cb[kLevels];
    if (threadIdx.x < kLevels) cb[threadIdx.x] = cb_g[threadIdx.x];
    __syncthreads();
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < g.groups; q += step) {
        const int64_t blk = q / GPB;
        const int j4 = (int)(q % GPB);
        const int64_t r = blk / g.nblk;
        const int64_t c0 = (blk - r * g.nblk) * BS + j4 * 4;
        const uint8_t* rec = buf + blk * REC;
        const float scale = pow2_float(get_exponent<HB>(rec) - kExpBias);
        int qv[4];
        unpack3(rec + HB + 3 * j4, qv);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t c = c0 + e;
            if (c < g.cols) {
                const float v = cb[qv[e] & 0x1F] * scale;
                y[r * g.cols + c] = (qv[e] & 0x20) ? -v : v;
            }
        }
    }
}

// AXSTensor components (exponents [rows, nblk], codes and signs [rows, nblk, bs])
// <-> records, for the component-level API (_pack_to_flat_buffer /
// _unpack_from_flat_buffer).
template <int HB>
__global__ __launch_bounds__(kThreads) void wire_from_codes_kernel(const uint8_t* __restrict__ exps,
                                                                   const uint8_t* __restrict__ codes,
                                                                   const uint8_t* __restrict__ signs, int bs,
                                                                   int64_t groups, uint8_t* __restrict__ buf) {
    const int gpb = bs / 4, rec_bytes = HB + bs * 3 / 4;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < groups; q += step) {
        const int64_t blk = q / gpb;
        const int j4 = (int)(q % gpb);
        int qv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t o = q * 4 + e;
            qv[e] = (codes[o] & 0x1F) | ((signs && signs[o]) ? 0x20 : 0);
        }
        uint8_t* rec = buf + blk * rec_bytes;
        if (j4 == 0) put_header<HB>(rec, exps[blk]);
        pack3(qv, rec + HB + 3 * j4);
    }
}

template <int HB>
__global__ __launch_bounds__(kThreads) void wire_to_codes_kernel(const uint8_t* __restrict__ buf, int bs,
                                                                 int64_t groups, uint8_t* __restrict__ exps,
                                                                 uint8_t* __restrict__ codes,
                                                                 uint8_t* __restrict__ signs) {
    const int gpb = bs / 4, rec_bytes = HB + bs * 3 / 4;
    const int64_t step = (int64_t)gridDim.x * kThreads;
    for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < groups; q += step) {
        const int64_t blk = q / gpb;
        const int j4 = (int)(q % gpb);
        const uint8_t* rec = buf + blk * rec_bytes;
        int qv[4];
        unpack3(rec + HB + 3 * j4, qv);
        if (j4 == 0) exps[blk] = (uint8_t)get_exponent<HB>(rec);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t o = q * 4 + e;
            codes[o] = (uint8_t)(qv[e] & 0x1F);
            if (signs) signs[o] = (uint8_t)((qv[e] >> 5) & 1);
        }
    }
}

unsigned wire_grid(int64_t groups) {
    const int64_t wgs = (groups + kThreads - 1) / kThreads;
    return (unsigned)(wgs < 65536 ? (wgs > 0 ? wgs : 1) : 65536);
}

int check_wire(const char* fn, int64_t rows, int64_t cols, int bs) {
    if (!valid_block(bs)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: block_size must be 8, 16 or 32 (got %d)", fn, bs);
    if (rows < 0 || cols < 0) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: negative shape", fn);
    if (rows > ((int64_t)1 << 40) / (cols + 1)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: tensor too large", fn);
    return AXS6_OK;
}

int64_t record_bytes(int hb, int64_t rows, int64_t cols, int bs) {
    if (rows < 0 || cols < 0 || !valid_block(bs)) return -1;
    const int64_t nblk = (cols + bs - 1) / bs;
    return rows * nblk * (hb + bs * 3 / 4);
}

// vec: whole-block rows, x aligned to 4 values, buf to 16 bytes; rows: any
// rows with buf aligned to 16 bytes (the fast kernels' row-geometry mode).
//
// The row-geometry mode steps each lane from its tile's first row over whole
// rows, one step per row passed, so its cost grows as rows get short: rows of
// fewer than kWireRowsMinGroups 4-value groups (padded) take the general
// kernels, which divide per group.  Measured (f32, pack / unpack us):
// 2^20 x 3 (2 groups per row) 46.7 / 43.8 in row mode against 11.0 / 8.5;
// 2^18 x 40 (16) 26.0 / 20.4 against 22.3 / 20.8; 2^17 x 100 (32)
// 21.2 / 16.6 against 22.8 / 22.4; 2^15 x 1000 30.2 / 25.1 against 45.7 / 46.5.
constexpr int64_t kWireRowsMinGroups = 32;
template <int HB, int DT>
void launch_pack(const void* x, const WireGeom& g, int bs, bool vec, bool rows, const RowGeom& rg,
                 const DeviceTables& t, uint8_t* buf, hipStream_t st) {
    using S = typename Elem<DT>::S;
    const S* xs = (const S*)x;
    if (vec || rows) {
        const dim3 grid(wire_vec_grid(g.groups));
#define AXS6_WPACK(R_)                                                                                                 \
        do {                                                                                                           \
            if (bs == 8) wire_pack_vec_kernel<HB, DT, 8, R_><<<grid, kThreads, 0, st>>>(xs, g.groups, rg, t.band, t.rev, buf);   \
            else if (bs == 16) wire_pack_vec_kernel<HB, DT, 16, R_><<<grid, kThreads, 0, st>>>(xs, g.groups, rg, t.band, t.rev, buf); \
            else wire_pack_vec_kernel<HB, DT, 32, R_><<<grid, kThreads, 0, st>>>(xs, g.groups, rg, t.band, t.rev, buf); \
        } while (0)
        if (vec) AXS6_WPACK(false);
        else AXS6_WPACK(true);
#undef AXS6_WPACK
    } else {
        const dim3 grid(wire_grid(g.groups));
        if (bs == 8) wire_pack_kernel<HB, DT, 8><<<grid, kThreads, 0, st>>>(xs, g, t.band, t.rev, buf);
        else if (bs == 16) wire_pack_kernel<HB, DT, 16><<<grid, kThreads, 0, st>>>(xs, g, t.band, t.rev, buf);
        else wire_pack_kernel<HB, DT, 32><<<grid, kThreads, 0, st>>>(xs, g, t.band, t.rev, buf);
    }
}

// x [rows, cols] -> records with HB-byte headers.
template <int HB>
int pack_records(const char* fn, const void* x, int dtype, int64_t rows, int64_t cols, int bs, uint8_t* buffer,
                 void* stream) {
    if (!valid_dtype(dtype)) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: unknown dtype code %d", fn, dtype);
    int rc = check_wire(fn, rows, cols, bs);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return AXS6_OK;
    if (!x || !buffer) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    DeviceTables t;
    if ((rc = device_tables(&t))) return rc;
    const int64_t nblk = (cols + bs - 1) / bs;
    const WireGeom g{rows, cols, nblk, rows * nblk * (bs / 4)};
    const int esize = dtype == AXS6_F32 ? 4 : 2;
    const bool xal = (uintptr_t)x % (4 * esize) == 0;
    const bool vec = cols % bs == 0 && xal && (uintptr_t)buffer % 16 == 0;
    const bool rows_mode = !vec && (uintptr_t)buffer % 16 == 0 && nblk * (bs / 4) >= kWireRowsMinGroups;
    const RowGeom rg{cols, nblk * (bs / 4), cols % 4 == 0 && xal};
    hipStream_t st = (hipStream_t)stream;
    if (dtype == AXS6_F32) launch_pack<HB, AXS6_F32>(x, g, bs, vec, rows_mode, rg, t, buffer, st);
    else if (dtype == AXS6_BF16) launch_pack<HB, AXS6_BF16>(x, g, bs, vec, rows_mode, rg, t, buffer, st);
    else launch_pack<HB, AXS6_F16>(x, g, bs, vec, rows_mode, rg, t, buffer, st);
    return check_launch(fn);
}

// records -> y [rows, cols] f32.
template <int HB>
int unpack_records(const char* fn, const uint8_t* buffer, int64_t rows, int64_t cols, int bs, float* y,
                   void* stream) {
    int rc = check_wire(fn, rows, cols, bs);
    if (rc) return rc;
    if (rows == 0 || cols == 0) return AXS6_OK;
    if (!buffer || !y) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    DeviceTables t;
    if ((rc = device_tables(&t))) return rc;
    const int64_t nblk = (cols + bs - 1) / bs;
    const WireGeom g{rows, cols, nblk, rows * nblk * (bs / 4)};
    hipStream_t st = (hipStream_t)stream;
    const bool yal = (uintptr_t)y % 16 == 0;
    const bool vec = cols % bs == 0 && yal;
    if ((uintptr_t)buffer % 16 == 0 && (vec || nblk * (bs / 4) >= kWireRowsMinGroups)) {
        const RowGeom rg{cols, nblk * (bs / 4), cols % 4 == 0 && yal};
        const dim3 grid(wire_vec_grid(g.groups));
#define AXS6_WUNPACK(R_)                                                                                       \
        do {                                                                                                   \
            if (bs == 8) wire_unpack_vec_kernel<HB, 8, R_><<<grid, kThreads, 0, st>>>(buffer, g.groups, rg, t.codebook, y);   \
            else if (bs == 16) wire_unpack_vec_kernel<HB, 16, R_><<<grid, kThreads, 0, st>>>(buffer, g.groups, rg, t.codebook, y); \
            else wire_unpack_vec_kernel<HB, 32, R_><<<grid, kThreads, 0, st>>>(buffer, g.groups, rg, t.codebook, y); \
        } while (0)
        if (vec) AXS6_WUNPACK(false);
        else AXS6_WUNPACK(true);
#undef AXS6_WUNPACK
        return check_launch(fn);
    }
    const dim3 grid(wire_grid(g.groups));
    if (bs == 8) wire_unpack_kernel<HB, 8><<<grid, kThreads, 0, st>>>(buffer, g, t.codebook, y);
    else if (bs == 16) wire_unpack_kernel<HB, 16><<<grid, kThreads, 0, st>>>(buffer, g, t.codebook, y);
    else wire_unpack_kernel<HB, 32><<<grid, kThreads, 0, st>>>(buffer, g, t.codebook, y);
    return check_launch(fn);
}

template <int HB>
int records_from_codes(const char* fn, const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs,
                       int64_t rows, int64_t nblk, int bs, uint8_t* buffer, void* stream) {
    int rc = check_wire(fn, rows, nblk * (int64_t)bs, bs);
    if (rc) return rc;
    if (rows == 0 || nblk == 0) return AXS6_OK;
    if (!exponents || !codes || !buffer) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    const int64_t groups = rows * nblk * (bs / 4);
    wire_from_codes_kernel<HB><<<dim3(wire_grid(groups)), kThreads, 0, (hipStream_t)stream>>>(exponents, codes, signs,
                                                                                              bs, groups, buffer);
    return check_launch(fn);
}

template <int HB>
int records_to_codes(const char* fn, const uint8_t* buffer, int64_t rows, int64_t nblk, int bs, uint8_t* exponents,
                     uint8_t* codes, uint8_t* signs, void* stream) {
    int rc = check_wire(fn, rows, nblk * (int64_t)bs, bs);
    if (rc) return rc;
    if (rows == 0 || nblk == 0) return AXS6_OK;
    if (!buffer || !exponents || !codes) return fail(AXS6_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    const int64_t groups = rows * nblk * (bs / 4);
    wire_to_codes_kernel<HB><<<dim3(wire_grid(groups)), kThreads, 0, (hipStream_t)stream>>>(buffer, bs, groups,
                                                                                            exponents, codes, signs);
    return check_launch(fn);
}

}  // namespace
}  // namespace axs6

using namespace axs6;

extern "C" int64_t axs6_nf5_wire_bytes(int64_t rows, int64_t cols, int32_t block_size) {
    return record_bytes(1, rows, cols, block_size);
}

extern "C" int axs6_nf5_pack_wire(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                                  uint8_t* buffer, void* stream) {
    return pack_records<1>("axs6_nf5_pack_wire", x, dtype, rows, cols, block_size, buffer, stream);
}

extern "C" int axs6_nf5_unpack_wire(const uint8_t* buffer, int64_t rows, int64_t cols, int32_t block_size, float* y,
                                    void* stream) {
    return unpack_records<1>("axs6_nf5_unpack_wire", buffer, rows, cols, block_size, y, stream);
}

extern "C" int axs6_nf5_wire_from_codes(const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs,
                                        int64_t rows, int64_t nblk, int32_t block_size, uint8_t* buffer,
                                        void* stream) {
    return records_from_codes<1>("axs6_nf5_wire_from_codes", exponents, codes, signs, rows, nblk, block_size, buffer,
                                 stream);
}

extern "C" int axs6_nf5_wire_to_codes(const uint8_t* buffer, int64_t rows, int64_t nblk, int32_t block_size,
                                      uint8_t* exponents, uint8_t* codes, uint8_t* signs, void* stream) {
    return records_to_codes<1>("axs6_nf5_wire_to_codes", buffer, rows, nblk, block_size, exponents, codes, signs,
                               stream);
}

extern "C" int64_t axs6_nf5_block_bytes(int64_t rows, int64_t cols, int32_t block_size) {
    return record_bytes(2, rows, cols, block_size);
}

extern "C" int axs6_nf5_pack_blocks(const void* x, int32_t dtype, int64_t rows, int64_t cols, int32_t block_size,
                                    uint8_t* buffer, void* stream) {
    return pack_records<2>("axs6_nf5_pack_blocks", x, dtype, rows, cols, block_size, buffer, stream);
}

extern "C" int axs6_nf5_unpack_blocks(const uint8_t* buffer, int64_t rows, int64_t cols, int32_t block_size, float* y,
                                      void* stream) {
    return unpack_records<2>("axs6_nf5_unpack_blocks", buffer, rows, cols, block_size, y, stream);
}

extern "C" int axs6_nf5_blocks_from_codes(const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs,
                                          int64_t rows, int64_t nblk, int32_t block_size, uint8_t* buffer,
                                          void* stream) {
    return records_from_codes<2>("axs6_nf5_blocks_from_codes", exponents, codes, signs, rows, nblk, block_size,
                                 buffer, stream);
}

extern "C" int axs6_nf5_blocks_to_codes(const uint8_t* buffer, int64_t rows, int64_t nblk, int32_t block_size,
                                        uint8_t* exponents, uint8_t* codes, uint8_t* signs, void* stream) {
    return records_to_codes<2>("axs6_nf5_blocks_to_codes", buffer, rows, nblk, block_size, exponents, codes, signs,
                               stream);
}
