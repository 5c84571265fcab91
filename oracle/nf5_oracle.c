/*
 * nf5_oracle.c -- CPU restatement of the reference's eager NF5 path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels
 * under axs-6_amd/csrc.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Each function restates one torch-eager operation sequence of the
 * reference, scalar by scalar, in the order the reference applies it:
 *
 *   oracle_build_tables   axs/unified/quantize_unified.py:50-61  (codebook)
 *                         axs/unified/quantize_unified.py:68-97  (fused LUT)
 *                         axs/unified/quantize_unified.py:105-114 (reverse LUT)
 *   oracle_floor_log2     floor(torch.log2(clamp(amax, 1e-45)))   quantize_unified.py:173-175
 *   oracle_fake_quantize  fused_fake_quantize                     quantize_unified.py:121-204
 *   oracle_quantize       quantize_unified                        quantize_unified.py:211-282
 *   oracle_dequantize     dequantize_unified                      quantize_unified.py:285-308
 *   oracle_uniform        the HIP library's own dither stream (keyed 32-bit
 *                         hash), so the stochastic kernels can be checked
 *                         bit-for-bit.
 *
 * How each piece is pinned (tests/test_oracle.py):
 *   - codebook / LUT: SHA-256 of the float32 bytes against the values the
 *     closed form gives through torch.erfinv / torch.bucketize, and against
 *     the golden fixture written by tests/golden/make_golden.py;
 *   - floor_log2: compared with floor(torch.log2(x)) on every positive
 *     float32 (the reference's own library call);
 *   - fake_quantize / quantize / dequantize: golden vectors written from the
 *     reference in this container (tests/golden/), plus invariants.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math: every
 * float operation below must round exactly once, as torch's CPU kernels do).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <limits.h>

#define NF5_LEVELS 32
#define LUT_SIZE 1024
#define LUT_MAX_IDX 1023
#define EXP_BIAS 127

static float g_codebook[NF5_LEVELS];
static float g_lut[LUT_SIZE];
static uint8_t g_rev[LUT_SIZE];
static int g_ready = 0;

/* Inverse error function in long double: Newton's method on erfl, started
 * from a rational first guess.  Converges to ~1e-19 relative, far below the
 * double rounding the reference applies afterwards. */
static long double erfinv_ld(long double y) {
    long double a = 0.147L;
    long double ln = logl(1.0L - y * y);
    long double t1 = 2.0L / (3.14159265358979323846264338327950288L * a) + ln / 2.0L;
    long double x = sqrtl(sqrtl(t1 * t1 - ln / a) - t1);
    if (y < 0) x = -x;
    const long double two_over_sqrtpi = 1.12837916709551257389615890312154517L;
    for (int it = 0; it < 60; ++it) {
        long double err = erfl(x) - y;
        long double step = err / (two_over_sqrtpi * expl(-x * x));
        x -= step;
        if (fabsl(step) < 1e-21L * (fabsl(x) + 1e-30L)) break;
    }
    return x;
}

/* torch.linspace(0, 1, n, dtype=float64) on CPU: the first half counts up
 * from start, the second half counts down from end. */
static double linspace01(int i, int n) {
    double step = (1.0 - 0.0) / (double)(n - 1);
    int halfway = n / 2;
    if (i < halfway) return 0.0 + step * (double)i;
    return 1.0 - step * (double)(n - i - 1);
}

void oracle_build_tables(float* codebook_out, float* lut_out, uint8_t* rev_out) {
    if (!g_ready) {
        /* quantize_unified.py:50-61: levels[i] = sqrt(2)*erfinv((i+0.5)/32)
         * in float64, then divided by levels[31], then cast to float32. */
        double lv[NF5_LEVELS];
        for (int i = 0; i < NF5_LEVELS; ++i) {
            double p = ((double)i + 0.5) / (double)NF5_LEVELS;
            double e = (double)erfinv_ld((long double)p);
            lv[i] = sqrt(2.0) * e;
        }
        double last = lv[NF5_LEVELS - 1];
        for (int i = 0; i < NF5_LEVELS; ++i) g_codebook[i] = (float)(lv[i] / last);

        /* quantize_unified.py:80-97: boundaries = [0, midpoints, 1+1e-6]
         * (float64); code = bucketize(x, boundaries) - 1, clamped to [0,31];
         * bucketize (right=False) counts the boundaries strictly below x. */
        double cb[NF5_LEVELS];
        for (int i = 0; i < NF5_LEVELS; ++i) cb[i] = (double)g_codebook[i];
        double bnd[NF5_LEVELS + 1];
        bnd[0] = 0.0;
        for (int i = 0; i < NF5_LEVELS - 1; ++i) bnd[i + 1] = (cb[i] + cb[i + 1]) / 2.0;
        bnd[NF5_LEVELS] = 1.0 + 1e-6;
        for (int i = 0; i < LUT_SIZE; ++i) {
            double x = linspace01(i, LUT_SIZE);
            int cnt = 0;
            for (int j = 0; j <= NF5_LEVELS; ++j) cnt += (bnd[j] < x);
            int code = cnt - 1;
            if (code < 0) code = 0;
            if (code > NF5_LEVELS - 1) code = NF5_LEVELS - 1;
            g_lut[i] = (float)cb[code];
        }
        /* quantize_unified.py:105-114: argmin_j |lut[i] - cb[j]| in float64,
         * first index on ties. */
        for (int i = 0; i < LUT_SIZE; ++i) {
            double best = INFINITY;
            int arg = 0;
            for (int j = 0; j < NF5_LEVELS; ++j) {
                double d = fabs((double)g_lut[i] - cb[j]);
                if (d < best) { best = d; arg = j; }
            }
            g_rev[i] = (uint8_t)arg;
        }
        g_ready = 1;
    }
    if (codebook_out) memcpy(codebook_out, g_codebook, sizeof g_codebook);
    if (lut_out) memcpy(lut_out, g_lut, sizeof g_lut);
    if (rev_out) memcpy(rev_out, g_rev, sizeof g_rev);
}

/* ---- scalar restatements of the torch ops the reference composes ------- */

/* torch.sign: +1, -1, or 0 for +-0 and NaN. */
static inline float t_sign(float x) {
    if (x > 0.0f) return 1.0f;
    if (x < 0.0f) return -1.0f;
    return 0.0f;
}

/* torch.clamp(x, lo, hi) propagates NaN. */
static inline float t_clamp(float x, float lo, float hi) {
    if (isnan(x)) return x;
    if (x < lo) return lo;
    if (x > hi) return hi;
    return x;
}

/* float -> int32 as torch's CPU .to(torch.int32): truncation; NaN and
 * out-of-range values give INT_MIN (the x86 "integer indefinite"). */
static inline int32_t t_to_int32(float x) {
    if (isnan(x)) return INT_MIN;
    if (x >= 2147483648.0f || x < -2147483648.0f) return INT_MIN;
    return (int32_t)x;
}

static inline int32_t t_clamp_i(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* torch.log2 on float32 is correctly rounded on the CPU (checked against
 * every positive float32 by the tests); evaluate it in long double and round
 * once to float32. */
static inline float t_log2(float x) {
    if (isnan(x)) return x;
    if (x == 0.0f) return -INFINITY;
    if (isinf(x)) return x > 0 ? INFINITY : NAN;
    if (x < 0.0f) return NAN;
    return (float)log2l((long double)x);
}

/* torch.exp2 on float32 integers: exact power of two, inf above 127. */
static inline float t_exp2_int(float k) {
    if (isnan(k)) return k;
    if (isinf(k)) return k > 0 ? INFINITY : 0.0f;
    return ldexpf(1.0f, (int)k);
}

/* Smallest positive float32 -- what clamp(min=1e-45) rounds 1e-45 to. */
#define T_1E_45 1.40129846e-45f

float oracle_floor_log2(float amax) {
    float safe = isnan(amax) ? amax : (amax < T_1E_45 ? T_1E_45 : amax);
    return floorf(t_log2(safe));
}

void oracle_floor_log2_batch(const float* x, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_floor_log2(x[i]);
}

/* torch.amax over a block: NaN if any element is NaN. */
static float block_amax(const float* absv, int bs) {
    float m = 0.0f;
    int has_nan = 0;
    for (int j = 0; j < bs; ++j) {
        if (isnan(absv[j])) has_nan = 1;
        else if (absv[j] > m) m = absv[j];
    }
    return has_nan ? NAN : m;
}

/* fused_fake_quantize (quantize_unified.py:121-204) on a (rows, cols)
 * float32 matrix with blocks of `bs` along the last dim.  `uniform` is NULL
 * for rounding="nearest"; otherwise it holds one U[0,1) draw per (row, col)
 * element and takes the place of torch.rand_like at :188. */
void oracle_fake_quantize(const float* x, float* y, int64_t rows, int64_t cols,
                          int bs, const float* uniform) {
    float cb[NF5_LEVELS];
    oracle_build_tables(cb, NULL, NULL);
    int64_t nblk = (cols + bs - 1) / bs;
    float blk[32], absv[32];
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nblk; ++b) {
            for (int j = 0; j < bs; ++j) {
                int64_t c = b * bs + j;
                blk[j] = (c < cols) ? x[r * cols + c] : 0.0f;  /* F.pad, :160-162 */
                absv[j] = fabsf(blk[j]);
            }
            float amax = block_amax(absv, bs);                              /* :172 */
            float safe = isnan(amax) ? amax : (amax < T_1E_45 ? T_1E_45 : amax); /* :173 */
            float scale = t_exp2_int(floorf(t_log2(safe)) + 1.0f);          /* :174 */
            if (amax == 0.0f) scale = 1.0f;                                 /* :177-179 */
            for (int j = 0; j < bs; ++j) {
                int64_t c = b * bs + j;
                float n = t_clamp(absv[j] / scale, 0.0f, 1.0f);             /* :182 */
                int32_t idx;
                if (uniform) {                                              /* :186-189 */
                    float u = (c < cols) ? uniform[r * cols + c] : 0.5f;
                    float dither = (u - 0.5f) / (float)LUT_MAX_IDX;
                    float t = (n + dither) * (float)LUT_MAX_IDX;
                    idx = t_clamp_i(t_to_int32(t), 0, LUT_MAX_IDX);
                } else {                                                    /* :191 */
                    float t = n * (float)LUT_MAX_IDX;
                    idx = t_clamp_i(t_to_int32(t), 0, LUT_MAX_IDX);
                }
                float rec = g_lut[idx];                                     /* :194 */
                float res = (t_sign(blk[j]) * rec) * scale;                 /* :197 */
                if (c < cols) y[r * cols + c] = res;                        /* :201-202 */
            }
        }
    }
}

/* quantize_unified (quantize_unified.py:211-282).  Outputs, all in the
 * padded (rows, nblk, bs) layout of AXSTensor:
 *   exps  uint8 (rows, nblk); codes uint8 (rows, nblk*bs); signs uint8 0/1. */
void oracle_quantize(const float* x, int64_t rows, int64_t cols, int bs,
                     const float* uniform, uint8_t* exps, uint8_t* codes,
                     uint8_t* signs) {
    oracle_build_tables(NULL, NULL, NULL);
    int64_t nblk = (cols + bs - 1) / bs;
    float blk[32], absv[32];
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t b = 0; b < nblk; ++b) {
            for (int j = 0; j < bs; ++j) {
                int64_t c = b * bs + j;
                blk[j] = (c < cols) ? x[r * cols + c] : 0.0f;
                absv[j] = fabsf(blk[j]);
            }
            float amax = block_amax(absv, bs);                              /* :242 */
            float safe = isnan(amax) ? amax : (amax < T_1E_45 ? T_1E_45 : amax);
            int32_t raw = t_to_int32(floorf(t_log2(safe)));                 /* :247 */
            /* int32 arithmetic wraps like torch's (INT_MIN + 128 stays negative) */
            int32_t e = (int32_t)((uint32_t)raw + 1u + (uint32_t)EXP_BIAS);
            e = t_clamp_i(e, 0, 255);                                       /* :248 */
            if (amax == 0.0f) e = 0;                                        /* :249 */
            exps[r * nblk + b] = (uint8_t)e;
            float scale = t_exp2_int((float)e - (float)EXP_BIAS);           /* :251-253 */
            if (scale < T_1E_45) scale = T_1E_45;
            for (int j = 0; j < bs; ++j) {
                int64_t c = b * bs + j;
                float n = t_clamp(absv[j] / scale, 0.0f, 1.0f);             /* :255 */
                int32_t idx;
                if (uniform) {                                              /* :262-264 */
                    float u = (c < cols) ? uniform[r * cols + c] : 0.5f;
                    float dither = (u - 0.5f) / (float)LUT_MAX_IDX;
                    idx = t_clamp_i(t_to_int32((n + dither) * (float)LUT_MAX_IDX), 0, LUT_MAX_IDX);
                } else {                                                    /* :259 */
                    idx = t_clamp_i(t_to_int32(n * (float)LUT_MAX_IDX), 0, LUT_MAX_IDX);
                }
                int64_t o = r * nblk * bs + c;
                codes[o] = g_rev[idx];                                      /* :268-269 */
                signs[o] = (uint8_t)(blk[j] < 0.0f);                        /* :271 */
            }
        }
    }
}

/* dequantize_unified (quantize_unified.py:285-308): cb[code]*2^(e-127),
 * negated where the sign is set, padding trimmed. */
void oracle_dequantize(const uint8_t* exps, const uint8_t* codes,
                       const uint8_t* signs, float* y, int64_t rows,
                       int64_t cols, int bs) {
    float cb[NF5_LEVELS];
    oracle_build_tables(cb, NULL, NULL);
    int64_t nblk = (cols + bs - 1) / bs;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < cols; ++c) {
            int64_t b = c / bs;
            float scale = t_exp2_int((float)exps[r * nblk + b] - (float)EXP_BIAS);
            int64_t o = r * nblk * bs + c;
            float v = cb[codes[o]] * scale;
            y[r * cols + c] = signs[o] ? -v : v;
        }
    }
}

/* The HIP library's dither stream (its own design; the reference draws
 * torch.rand_like, whose stream cannot be reproduced, so stochastic parity
 * with the reference is distributional).  key = splitmix64 finaliser of the
 * seed; the draw for element counter c = offset + i is Wellons' "lowbias32"
 * multiply-xorshift hash of (low word of c) ^ key_lo ^ (high word of c *
 * 0x9E3779B9 + key_hi), whose top 24 bits times 2^-24 give U in [0, 1).
 * Restated here so the stochastic kernels can be compared bit-for-bit. */
static uint64_t dither_key(uint64_t seed) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void oracle_uniform(uint64_t seed, uint64_t offset, int64_t n, float* u) {
    const uint64_t key = dither_key(seed);
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t c = offset + (uint64_t)i;
        uint32_t h = (uint32_t)c ^ (uint32_t)key ^
                     ((uint32_t)(c >> 32) * 0x9E3779B9u + (uint32_t)(key >> 32));
        h ^= h >> 16;
        h *= 0x7feb352du;
        h ^= h >> 15;
        h *= 0x846ca68bu;
        h ^= h >> 16;
        u[i] = (float)(h >> 8) * (1.0f / 16777216.0f);
    }
}
