// Device-side NF5 arithmetic shared by the fake-quantize kernels and the
// operand-packing kernels of the quantized linear.  Every function rounds
// exactly as the torch CPU operation it replaces (see nf5_fq.hip for the
// per-step mapping to axs/unified/quantize_unified.py); include only from
// translation units compiled with FP contraction off.
#pragma once

#include "axs6_internal.h"

#pragma clang fp contract(off)

namespace axs6 {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 3;  // 16-byte vectors in flight per thread (fq_vec_kernel)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---- element types ------------------------------------------------------

template <int DT> struct Elem;

template <> struct Elem<AXS6_F32> {
    using S = float;
    static constexpr int V = 4;
    __device__ static float to_f(S v) { return v; }
    __device__ static S from_f(float f) { return f; }
    __device__ static void unpack(u32x4 r, float* f) {
        f[0] = __uint_as_float(r.x); f[1] = __uint_as_float(r.y);
        f[2] = __uint_as_float(r.z); f[3] = __uint_as_float(r.w);
    }
    __device__ static u32x4 pack(const float* f) {
        u32x4 r;
        r.x = __float_as_uint(f[0]); r.y = __float_as_uint(f[1]);
        r.z = __float_as_uint(f[2]); r.w = __float_as_uint(f[3]);
        return r;
    }
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    // torch's c10::BFloat16 rounding: NaN -> 0x7FC0, otherwise round to
    // nearest even on the upper 16 bits.
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <> struct Elem<AXS6_BF16> {
    using S = uint16_t;
    static constexpr int V = 8;
    __device__ static float to_f(S v) { return __uint_as_float((uint32_t)v << 16); }
    __device__ static S from_f(float f) { return f32_to_bf16_rne(f); }
    __device__ static void unpack(u32x4 r, float* f) {
        uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    // gfx950's v_cvt_pk_bf16_f32 rounds to nearest even exactly as
    // f32_to_bf16_rne for every non-NaN float (checked over all 2^32 inputs);
    // NaN inputs here are the FQ's canonical 0x7fc00000, which it writes as
    // 0x7FC0 like torch.
    __device__ static u32x4 pack(const float* f) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x2 v = {f[2 * i], f[2 * i + 1]};
            w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
        }
        u32x4 r;
        r.x = w[0]; r.y = w[1]; r.z = w[2]; r.w = w[3];
        return r;
    }
};

template <> struct Elem<AXS6_F16> {
    using S = _Float16;
    static constexpr int V = 8;
    __device__ static float to_f(S v) { return (float)v; }
    __device__ static S from_f(float f) { return (_Float16)f; }  // v_cvt_f16_f32: RNE
    __device__ static void unpack(u32x4 r, float* f) {
        uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint16_t lo = (uint16_t)(w[i] & 0xffffu), hi = (uint16_t)(w[i] >> 16);
            f[2 * i] = (float)__builtin_bit_cast(_Float16, lo);
            f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, hi);
        }
    }
    // two values per v_cvt_pk_f16_f32, which gives the same bits as the
    // scalar v_cvt_f16_f32 for every float32 input (all 2^32 compared on the GPU)
    __device__ static u32x4 pack(const float* f) {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f32x2 v = {f[2 * i], f[2 * i + 1]};
            w[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
        }
        u32x4 r;
        r.x = w[0]; r.y = w[1]; r.z = w[2]; r.w = w[3];
        return r;
    }
};

// ---- block arithmetic ------------------------------------------------------

// v and the value DPP control `ctrl` brings to this lane, unsigned max.  Every
// control used here reads a lane inside the same row, so bound_ctrl (zero for
// lanes without a source) never applies; written this way (old value 0, the
// identity of the max) the compiler fuses the move into one v_max_u32_dpp.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
    return v > o ? v : o;
}

// Unsigned max across a group of G neighbouring lanes (G in {1,2,4,8}) with
// DPP: quad_perm [1,0,3,2], quad_perm [2,3,0,1], then row_half_mirror pairs
// each quad with the other quad of its 8-lane half-row.
template <int G>
__device__ __forceinline__ uint32_t group_umax(uint32_t v) {
    if constexpr (G >= 2) v = dpp_umax<0xB1>(v);
    if constexpr (G >= 4) v = dpp_umax<0x4E>(v);
    if constexpr (G >= 8) v = dpp_umax<0x141>(v);
    return v;
}

// Unsigned max across each group of N neighbouring lanes (N in {8, 16, 32}),
// returned in every lane of the group: the quad and half-row steps of
// group_umax, row_mirror for 16 lanes, and for 32 the v_permlane16_swap of v
// with itself, whose two results hold rows (0, 0, 2, 2) and (1, 1, 3, 3) --
// each lane's row and its partner row.
template <int N>
__device__ __forceinline__ uint32_t lanes_umax(uint32_t v) {
    static_assert(N == 8 || N == 16 || N == 32, "lane group");
    v = group_umax<8>(v);
    if constexpr (N >= 16) v = dpp_umax<0x140>(v);
    if constexpr (N >= 32) {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        v = p[0] > p[1] ? p[0] : p[1];
    }
    return v;
}

// Unsigned max over the whole wave, returned in every lane (a scalar): an
// inclusive max-scan over each row of 16 lanes (row_shr 1, 2, 4, 8; lanes
// without a source read 0), rows folded with row_bcast:15 and row_bcast:31,
// then lane 63 read out.
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
    v = dpp_umax<0x111>(v);
    v = dpp_umax<0x112>(v);
    v = dpp_umax<0x114>(v);
    v = dpp_umax<0x118>(v);
    uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);
    v = v > o ? v : o;
    o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);
    v = v > o ? v : o;
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Signed max over the whole wave (same reduction, signed order).
__device__ __forceinline__ int wave_imax(int v) {
    return (int)(wave_umax((uint32_t)v ^ 0x80000000u) ^ 0x80000000u);
}

// Same reduction for groups of up to 32 lanes through cross-lane shuffles
// (general path only).
template <int BS>
__device__ __forceinline__ uint32_t group_umax_shfl(uint32_t v) {
#pragma unroll
    for (int off = 1; off < BS; off <<= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = v > o ? v : o;
    }
    return v;
}

constexpr uint32_t kInfBits = 0x7f800000u;
constexpr uint32_t kNanBits = 0x7fc00000u;

// floor(torch.log2(a)) for a positive finite float32 given by its bits.
__device__ __forceinline__ int floor_log2_torch(uint32_t a, const uint8_t* band) {
    int f = a >= 0x00800000u ? (int)(a >> 23) - 127 : (31 - __clz((int)a)) - 149;
    int k = f + 1;
    uint32_t kb = k >= -126 ? (uint32_t)(k + 127) << 23 : 1u << (k + 149);
    return (kb - a <= (uint32_t)band[k + 149]) ? k : f;
}

__device__ __forceinline__ float pow2_float(int e) {
    // exact 2^e for e in [-149, 127]; inf above.
    return e >= 128 ? __uint_as_float(kInfBits)
                    : (e >= -126 ? __uint_as_float((uint32_t)(e + 127) << 23)
                                 : __uint_as_float(1u << (e + 149)));
}

// The per-block scale of fused_fake_quantize (quantize_unified.py:172-179).
// The scale itself (torch's `scales` entry: 2^e1, 1 for a zero block, inf,
// NaN) is only formed on the general path (scale_of); the short sequences
// use e1.
struct FqScale {
    int e1;         // exponent used to normalise when scale is finite (0 for a zero block)
    bool inf_scale;
    bool nan_block;
    bool zero;
};

__device__ __forceinline__ FqScale fq_scale_general(uint32_t amax, const uint8_t* band) {
    FqScale s;
    s.nan_block = amax > kInfBits;
    s.zero = amax == 0u;
    bool inf_amax = amax == kInfBits;
    int e1 = (s.zero || amax >= kInfBits) ? 0 : floor_log2_torch(amax, band) + 1;
    s.inf_scale = inf_amax || e1 >= 128;
    s.e1 = s.inf_scale ? 0 : e1;
    return s;
}

// Bits of 2^-101: a block maximum at or above it has e1 >= -100.
constexpr uint32_t kFastMinAmaxBits = (uint32_t)(kExpBias - 101) << 23;

// fq_scale_general's result.  For a normal block maximum the exponent takes a
// short form (floor_log2_torch without its subnormal branch: f from the
// exponent field, k = f + 1 at the power of two above); a wave with a block
// outside [2^-101, 2^128) other than zero -- subnormal, tiny, inf, NaN or
// rounding to e1 = 128 -- recomputes with the general form (uniform branch).
__device__ __forceinline__ FqScale fq_scale(uint32_t amax, const uint8_t* band) {
    const int f = (int)(amax >> 23) - kExpBias;
    const uint32_t kb = (amax & 0x7f800000u) + 0x00800000u;     // bits of 2^(f + 1)
    const int e1 = (kb - amax <= (uint32_t)band[f + 150]) ? f + 2 : f + 1;
    const bool wide = amax != 0u && (amax < kFastMinAmaxBits || e1 >= 128);
    if (__builtin_amdgcn_ballot_w64(wide) != 0) return fq_scale_general(amax, band);
    FqScale s;
    s.nan_block = false;
    s.inf_scale = false;
    s.zero = amax == 0u;
    s.e1 = s.zero ? 0 : e1;
    return s;
}

__device__ __forceinline__ float scale_of(const FqScale& s) {
    return s.nan_block ? __uint_as_float(kNanBits)
                       : (s.inf_scale ? __uint_as_float(kInfBits) : (s.zero ? 1.0f : pow2_float(s.e1)));
}

// |x| / scale exactly, for power-of-two scales.
__device__ __forceinline__ float normalise(uint32_t abits, const FqScale& s) {
    if (s.inf_scale) return abits >= kInfBits ? __uint_as_float(kNanBits) : 0.0f;
    return __builtin_amdgcn_ldexpf(__uint_as_float(abits), -s.e1);
}

// `d` is the dither (U - 0.5) / 1023 of the stochastic mode (0 for nearest).
__device__ __forceinline__ int lut_index(float n, bool stochastic, float d) {
    float t = stochastic ? (n + d) * 1023.0f : n * 1023.0f;
    t = (t == t) ? t : 0.0f;              // NaN -> INT_MIN -> clamped to 0 in torch
    int i = (int)t;                       // truncation toward zero
    return i < 0 ? 0 : (i > kLutMax ? kLutMax : i);
}

__device__ __forceinline__ float torch_sign(float x) {
    return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
}

__device__ __forceinline__ float fq_value(float x, const FqScale& s, const float* lut, bool stochastic, float d) {
    uint32_t ab = __float_as_uint(x) & 0x7fffffffu;
    float n = normalise(ab, s);
    float rec = lut[lut_index(n, stochastic, d)];
    float r = (torch_sign(x) * rec) * scale_of(s);
    return s.nan_block ? __uint_as_float(kNanBits) : r;
}

// Lowest block exponent e1 of the short FQ sequences below: from it up to 127
// the factor 1023 * 2^-e1 is a finite normal float and lut * 2^e1 is normal.
constexpr int kFastMinE1 = -100;

// |x| * 1023 * 2^-e1 as the reference computes it, (|x| * 2^-e1) * 1023,
// for e1 >= kFastMinE1, as one product with c = 1023 * 2^-e1 (exact): when
// |x| * 2^-e1 is a normal float it is exact, so both are the one rounding of
// the same real number; when it is subnormal both are below 1023 * 2^-126
// and truncate to the same index 0.
__device__ __forceinline__ float lut_pos(uint32_t abits, float c) { return __uint_as_float(abits) * c; }

// fused_fake_quantize of the V elements of one 16-byte vector whose block
// scale is s; d[e] is element e's dither (U - 0.5) / 1023 (unused in nearest
// mode).  Blocks with a NaN or an infinite scale, or an exponent below
// kFastMinE1, take the per-element general path (fq_value).  When no lane of
// the wave holds such a block -- the normal case, tested with one ballot so
// the branch is uniform -- a shorter sequence gives the same bits: the scale
// 2^e1 exceeds every |x| of the block, so n = |x| 2^-e1 < 1 is finite,
// n * 1023 lies in [0, 1023) and (n + d) * 1023 in (-0.51, 1023.5), so the
// truncated index is in [0, 1023] without a clamp, and (sign(x) * lut) * scale
// equals lut * scale with x's sign bit (rounding to nearest is symmetric), or
// +0 where x is +-0 (torch.sign(-0.0) is +0).
template <int V>
__device__ __forceinline__ void fq_vector(float (&f)[V], const FqScale& s, const float* lut, bool stochastic,
                                          const float (&d)[V]) {
    const bool special = s.nan_block || s.inf_scale || s.e1 < kFastMinE1;
    if (__builtin_amdgcn_ballot_w64(special) != 0) {
#pragma unroll
        for (int e = 0; e < V; ++e) f[e] = fq_value(f[e], s, lut, stochastic, d[e]);
    } else {
        const float c = __builtin_amdgcn_ldexpf(1023.0f, -s.e1);
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const uint32_t xb = __float_as_uint(f[e]);
            const uint32_t ab = xb & 0x7fffffffu;
            float t;
            if (stochastic) t = (__builtin_amdgcn_ldexpf(__uint_as_float(ab), -s.e1) + d[e]) * 1023.0f;
            else t = lut_pos(ab, c);
            const float mag = __builtin_amdgcn_ldexpf(lut[(int)t], s.e1);   // lut * 2^e1, exact (normal)
            // +0 where x is +-0, else mag with x's sign -- as a mask, not a
            // select, so the compiler does not branch around the LUT read per
            // element: (ab + 0x7fffffff) has bit 31 set exactly when ab != 0
            const uint32_t nz = (uint32_t)((int32_t)(ab + 0x7fffffffu) >> 31);
            f[e] = __uint_as_float((__float_as_uint(mag) ^ (xb & 0x80000000u)) & nz);
        }
    }
}

// Nearest-mode FQ of one 16-byte vector without the block scale, for callers
// that fold 2^e1 into a power-of-two scaling of their own: f[e] becomes
// +-lut_fast[i] (+0 where x is +-0), with i the index fq_vector computes.
// lut_fast is the LUT, or the LUT rounded to the input type when the caller
// must round FQ values to it (rounding commutes with 2^e1 while lut * 2^e1
// is normal, which e1 >= kFastMinE1 guarantees).  When any lane of the wave
// holds a block the fast sequence does not cover, every lane writes its full
// FQ values instead (fq_value, from the unrounded lut) and the call returns
// true -- wave-uniform, so the caller's branch on it is too.
template <int V>
__device__ __forceinline__ bool fq_vector_unscaled(float (&f)[V], const FqScale& s, const float* lut,
                                                   const float* lut_fast) {
    const bool special = s.nan_block || s.inf_scale || s.e1 < kFastMinE1;
    if (__builtin_amdgcn_ballot_w64(special) != 0) {
#pragma unroll
        for (int e = 0; e < V; ++e) f[e] = fq_value(f[e], s, lut, false, 0.0f);
        return true;
    }
    const float c = __builtin_amdgcn_ldexpf(1023.0f, -s.e1);
#pragma unroll
    for (int e = 0; e < V; ++e) {
        const uint32_t xb = __float_as_uint(f[e]);
        const uint32_t ab = xb & 0x7fffffffu;
        const float mag = lut_fast[(int)lut_pos(ab, c)];
        const uint32_t nz = (uint32_t)((int32_t)(ab + 0x7fffffffu) >> 31);
        f[e] = __uint_as_float((__float_as_uint(mag) ^ (xb & 0x80000000u)) & nz);
    }
    return false;
}

// FQ values rounded to the element type's precision, as the reference's
// fake-quantize returns them for a bf16 or f16 tensor (the output is cast back
// to the input dtype, quantize_unified.py:201-204) before its F.linear or
// matmul contracts them: bf16 to nearest even (NaN stays NaN), f16 through the
// hardware conversion (values past 65504 become inf, as in torch); f32 as is.
template <int DT, int V>
__device__ __forceinline__ void round_to_elem(float (&f)[V]) {
    if constexpr (DT == AXS6_BF16) {
#pragma unroll
        for (int e = 0; e < V; ++e) f[e] = Elem<AXS6_BF16>::to_f(f32_to_bf16_rne(f[e]));
    } else if constexpr (DT == AXS6_F16) {
#pragma unroll
        for (int e = 0; e < V; ++e) f[e] = (float)(_Float16)f[e];
    }
}

// Dither stream of the stochastic mode.  A call's 64-bit seed is turned into
// a key once (the splitmix64 finaliser); the draw for element counter i is a
// 32-bit multiply-xorshift hash (the "lowbias32" constants published by
// C. Wellons) of i's low word mixed with the key and i's high word, and its
// top 24 bits scaled by 2^-24 give U in [0, 1) -- the resolution of
// torch.rand's float32 draws.  Three 32-bit multiplies per element instead of
// splitmix64's 64-bit ones, which made the dY packing kernels VALU-bound.
__host__ __device__ __forceinline__ uint64_t dither_key(uint64_t seed) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ uint32_t dither_mix(uint32_t h) {
    h ^= h >> 16;
    h *= 0x7feb352du;
    h ^= h >> 15;
    h *= 0x846ca68bu;
    h ^= h >> 16;
    return h;
}

// (U - 0.5) / 1023 for the draw U = (h >> 8) * 2^-24, bit-identical to the
// IEEE float division torch performs: J = U * 2^24 - 2^23 is an exact
// integer, J / 1023 is rounded by a reciprocal product and one FMA residual
// correction (identical to the correctly rounded quotient for every one of
// the 2^24 possible J), and the rescale by 2^-24 is exact.
__device__ __forceinline__ float dither_from_hash(uint32_t h) {
    const float fj = (float)((int)(h >> 8) - (1 << 23));
    float q = fj * (1.0f / 1023.0f);
    const float r = __builtin_fmaf(-q, 1023.0f, fj);
    q = __builtin_fmaf(r, 1.0f / 1023.0f, q);
    return q * (1.0f / 16777216.0f);
}

// The dither (U - 0.5) / 1023 of element counter i.
__device__ __forceinline__ float dither_step(uint64_t key, uint64_t i) {
    const uint32_t hg = (uint32_t)(i >> 32) * 0x9E3779B9u + (uint32_t)(key >> 32);
    return dither_from_hash(dither_mix((uint32_t)i ^ (uint32_t)key ^ hg));
}

// The same for the elements base, base + 1, ... of one vector: the high-word
// term is computed once and carried across a 2^32 boundary inside the vector.
struct DitherVec {
    uint32_t klo, hg, lo0;
};
__device__ __forceinline__ DitherVec dither_vec(uint64_t key, uint64_t base) {
    return DitherVec{(uint32_t)key, (uint32_t)(base >> 32) * 0x9E3779B9u + (uint32_t)(key >> 32), (uint32_t)base};
}
__device__ __forceinline__ float dither_step(const DitherVec& v, int e) {
    const uint32_t lo = v.lo0 + (uint32_t)e;
    const uint32_t hg = lo < v.lo0 ? v.hg + 0x9E3779B9u : v.hg;
    return dither_from_hash(dither_mix(lo ^ v.klo ^ hg));
}
// Counter low word lo with the high-word term kh = klo ^ hg fixed: for a call
// whose counters offset .. offset + n - 1 share one high word.
__device__ __forceinline__ float dither_step32(uint32_t lo, uint32_t kh) {
    return dither_from_hash(dither_mix(lo ^ kh));
}

// Nontemporal (streaming) load and store: the `nt` bit, for data a kernel
// reads or writes once.  A plain store leaves its line dirty in the 256 MiB
// last-level cache and a later kernel pays the write-back when it evicts it;
// a streaming kernel that writes through pays it itself, while its own HBM
// stream is running.  Call sites use these unconditionally: a plain and an
// nt store on the two sides of one branch get merged and lose the hint.
template <typename T>
__device__ __forceinline__ T ld_stream(const T* p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void st_stream(T v, T* p) { __builtin_nontemporal_store(v, p); }

// Stages the LUT (and the band table) in LDS, with workgroups of any size
// (one 16-byte piece per thread from 256 threads up; smaller workgroups,
// such as the fused linear's 64- and 128-thread tilings, loop).
__device__ __forceinline__ void stage_tables(float* lut_s, uint32_t* band_w, const float* lut_g,
                                             const uint8_t* band_g) {
    const int tid = threadIdx.x, nt = (int)blockDim.x;
    for (int i = tid; i < kLutSize / 4; i += nt)
        reinterpret_cast<float4*>(lut_s)[i] = reinterpret_cast<const float4*>(lut_g)[i];
    for (int i = tid; i < kBandSize / 4; i += nt) band_w[i] = reinterpret_cast<const uint32_t*>(band_g)[i];
    __syncthreads();
}

}  // namespace
}  // namespace axs6
