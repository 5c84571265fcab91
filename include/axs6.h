/*
 * axs6.h -- C ABI of the MI355X (gfx950) NF5 hot-path library, libaxs6.so.
 *
 * Every entry point takes raw device pointers, element counts and a HIP
 * stream (hipStream_t passed as void*; NULL = the null stream), launches
 * asynchronously on that stream, allocates nothing on the hot path, never
 * synchronises the host, and returns an axs6_status.  A non-zero status
 * leaves a message retrievable with axs6_last_error() (per host thread).
 *
 * Conventions shared by all calls:
 *   - tensors are dense and row-major; "rows x cols" with NF5 blocks of
 *     `block_size` (8, 16 or 32) running along `cols`; when cols is not a
 *     multiple of block_size the last block of each row is zero-padded
 *     virtually (nothing is read or written past cols);
 *   - dtype codes: AXS6_F32, AXS6_BF16, AXS6_F16 select the element type of
 *     the input and of the same-typed output; arithmetic is float32;
 *   - stochastic rounding (dither of +-0.5 LUT steps) draws U[0,1) for the
 *     element at flat index i from splitmix64(seed + (offset + i) * golden),
 *     so a (seed, offset) pair reproduces a draw exactly.
 *
 * Python binding: axs-6_amd/axs/_lib.py (ctypes).  The reference entry
 * point each call replaces is cited on its declaration.
 */
#ifndef AXS6_H
#define AXS6_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    AXS6_OK = 0,
    AXS6_ERR_INVALID_ARGUMENT = 1, /* bad shape, block size, dtype, null pointer */
    AXS6_ERR_UNSUPPORTED = 2,      /* valid request this build does not serve */
    AXS6_ERR_HIP = 3,              /* a HIP runtime call or kernel launch failed */
    AXS6_ERR_NO_DEVICE = 4         /* no usable gfx950 device is current */
} axs6_status;

typedef enum { AXS6_F32 = 0, AXS6_BF16 = 1, AXS6_F16 = 2 } axs6_dtype;

/* Library version string, e.g. "axs6-mi355x 0.1.0 (gfx950)". */
const char* axs6_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* axs6_last_error(void);

/* Uploads the constant tables to the current device.  Optional: every entry
 * point does it on first use per device.  Not hot-path. */
int axs6_init(void);

/* Host copies of the constant tables the kernels use (any pointer may be
 * NULL): NF5 codebook (32 x f32), fused LUT (1024 x f32), reverse LUT
 * (1024 x u8, LUT index -> code) and the log2 rounding band (278 x u8:
 * band[k + 149] = how many float32 values just below 2^k have
 * floor(log2(x)) == k under a correctly rounded log2).
 * Replaces: NF5_CODEBOOK, FUSED_NF5_LUT, REVERSE_NF5_LUT
 *           (axs/unified/quantize_unified.py:61,96,114). */
int axs6_get_tables(float* codebook, float* lut, uint8_t* reverse_lut, uint8_t* log2_band);

/* NF5 fake-quantize: y = FQ(x), same shape and dtype (x may equal y).
 * Replaces: fused_fake_quantize (axs/unified/quantize_unified.py:121) and
 *           triton_fused_fake_quantize (axs/unified/triton_kernels.py:295),
 *           reached through accelerated_fake_quantize (axs/unified/backend.py:495). */
int axs6_nf5_fake_quantize(const void* x, void* y, int32_t dtype, int64_t rows, int64_t cols,
                           int32_t block_size, int32_t stochastic, uint64_t seed,
                           uint64_t offset, void* stream);

/* NF5 quantize to the AXSTensor fields, optionally also writing FQ(x):
 *   exponents  u8 [rows, nblk]            (nblk = ceil(cols / block_size))
 *   codes      u8 [rows, nblk*block_size] 5-bit NF5 magnitude codes
 *   signs      u8 [rows, nblk*block_size] 1 where x < 0 (may be NULL)
 *   fq         same dtype as x [rows, cols], fused_fake_quantize of x (may be NULL)
 * Replaces: quantize_unified (axs/unified/quantize_unified.py:211). */
int axs6_nf5_quantize(const void* x, int32_t dtype, int64_t rows, int64_t cols,
                      int32_t block_size, int32_t stochastic, uint64_t seed, uint64_t offset,
                      uint8_t* exponents, uint8_t* codes, uint8_t* signs, void* fq,
                      void* stream);

/* Inverse of axs6_nf5_quantize: y[rows, cols] f32 = +-codebook[code] * 2^(e-127).
 * Replaces: dequantize_unified (axs/unified/quantize_unified.py:285). */
int axs6_nf5_dequantize(const uint8_t* exponents, const uint8_t* codes, const uint8_t* signs,
                        float* y, int64_t rows, int64_t cols, int32_t block_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AXS6_H */
